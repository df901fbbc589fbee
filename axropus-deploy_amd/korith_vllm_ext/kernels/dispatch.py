"""kernels/dispatch.py - decode-attention kernel selection.

Same registry and lookup as the reference (korith_vllm_ext/kernels/dispatch.py:
41-111): kernels are registered per (device version, storage format, active
format) and dispatch_kernel() falls back to the nearest lower device version,
then to any kernel of the storage format, then to fallback_fp16_kernel.

Every kernel registered here runs on the GPU through libamf_hip.so:

* hip_decode_attention(q, k, v, scale=None, mask=None, *, block_tables=...,
  context_lens=...) is the paged GQA INT4 decode (amf_int4_paged_decode_attn)
  when a block table is given, and dense attention otherwise: straight from
  the codes for int4_sym CompressedKV K/V (amf_int4_sym_dense_attn), else
  over the restored K/V (amf_dense_attn).
* fallback_fp16_kernel keeps the reference's name and signature
  (dispatch.py:117-143): decompress compressed K/V with the HIP codecs, then
  softmax(q k^T * scale + mask) v with the HIP dense-attention kernel, in fp32,
  rounded once to q's dtype.

There is no CPU path: without a GPU or libamf_hip.so these raise
amf_hip.AmfHipUnavailable.
"""

from __future__ import annotations

import logging
import math
import os
import threading
from collections import OrderedDict
from typing import Any, Callable, Dict, Optional, Tuple

import torch

import amf_hip

from ..codecs import (
    FMT_BF16,
    FMT_FP8_E4M3,
    FMT_FP8_E4M3_PH,
    FMT_FP16,
    FMT_INT4_ASYM_G32,
    FMT_INT4_BLOCK,
    FMT_INT4_SYM,
    CompressedKV,
    get_codec,
)

logger = logging.getLogger(__name__)

# torch.cuda.get_device_capability() of an MI355X (gfx950) under ROCm.
GFX950_VERSION = 95

_cached_sm: Optional[int] = None


def get_current_sm_version() -> int:
    """major * 10 + minor of the current device's capability (gfx950 -> 95),
    0 without a device (reference: dispatch.py:45-64)."""
    global _cached_sm
    if _cached_sm is not None:
        return _cached_sm
    if not torch.cuda.is_available():
        _cached_sm = 0
        return 0
    major, minor = torch.cuda.get_device_capability(torch.cuda.current_device())
    _cached_sm = major * 10 + minor
    return _cached_sm


KernelFn = Callable[..., torch.Tensor]

KERNEL_DISPATCH: Dict[Tuple[int, str, str], KernelFn] = {}


def register_kernel(sm: int, storage: str, active: str) -> Callable[[KernelFn], KernelFn]:
    """Decorator registering a kernel for a (device version, storage, active) triple."""

    def _wrap(fn: KernelFn) -> KernelFn:
        KERNEL_DISPATCH[(sm, storage, active)] = fn
        return fn

    return _wrap


def dispatch_kernel(storage_format: str, active_format: str) -> KernelFn:
    """Best registered kernel for the current device (lookup order of
    dispatch.py:84-111: exact triple, nearest lower device version for the
    storage format, any kernel of the storage format, fallback_fp16_kernel)."""
    sm = get_current_sm_version()
    key = (sm, storage_format, active_format)
    if key in KERNEL_DISPATCH:
        return KERNEL_DISPATCH[key]
    for hw in sorted([k[0] for k in KERNEL_DISPATCH if k[1] == storage_format], reverse=True):
        if hw <= sm and (hw, storage_format, active_format) in KERNEL_DISPATCH:
            return KERNEL_DISPATCH[(hw, storage_format, active_format)]
    for (_hw, s, _a), fn in KERNEL_DISPATCH.items():
        if s == storage_format:
            return fn
    logger.info("dispatch_kernel: no kernel for sm=%d storage=%s active=%s; dense attention",
                sm, storage_format, active_format)
    return fallback_fp16_kernel


# ------------------------------------------------------------ dense path --

_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Split-K scratch reused across calls: one buffer per (device, stream), grown
# to the largest size asked for, at most _SCRATCH_MAX of them (the one least
# recently grown or added goes first).  Calls on one stream run in order, so
# a call's kernels start after the previous call's merge has read the buffer;
# a stream under graph capture gets a buffer of its own per call instead.
_SCRATCH: "OrderedDict[Tuple[int, int], torch.Tensor]" = OrderedDict()
_SCRATCH_MAX = 16
_SCRATCH_LOCK = threading.Lock()
_SPLIT_WS: Dict[tuple, int] = {}  # (B, Hq, Hkv, Tq, T, D) -> workspace bytes


def _scratch(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), stream)
    buf = _SCRATCH.get(key)
    if buf is not None and buf.numel() >= nbytes:
        return buf  # the common case: no reordering, no lock
    with _SCRATCH_LOCK:
        buf = _SCRATCH.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _SCRATCH[key] = buf
        _SCRATCH.move_to_end(key)
        while len(_SCRATCH) > _SCRATCH_MAX:
            _SCRATCH.popitem(last=False)
        return buf


def _split_workspace_bytes(B: int, Hq: int, Hkv: int, Tq: int, T: int, D: int) -> int:
    key = (B, Hq, Hkv, Tq, T, D)
    n = _SPLIT_WS.get(key)
    if n is None:
        if len(_SPLIT_WS) > 4096:
            _SPLIT_WS.clear()
        n = _SPLIT_WS[key] = int(amf_hip.load().amf_dense_attn_workspace_bytes(*key))
    return n


def _to_tensor(obj: Any, like: torch.Tensor) -> torch.Tensor:
    """A CompressedKV (decompressed on the GPU by its codec) or a tensor, in
    like's dtype and device (reference: dispatch.py:146-152)."""
    if isinstance(obj, torch.Tensor):
        return obj.to(device=like.device, dtype=like.dtype)
    codec = get_codec(obj.format)
    return codec.decompress_to(obj, target_dtype=like.dtype).to(like.device)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float],
                    mask: Optional[torch.Tensor], out_dtype: Optional[torch.dtype] = None
                    ) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v on the GPU (amf_dense_attn).

    q [..., Hq, Tq, D]; k, v [..., Hkv, T, D] (leading dims broadcast to q's,
    Hq a multiple of Hkv); mask broadcastable to [..., Hq, Tq, T]."""
    if q.dtype not in _DTYPES:
        raise TypeError(f"dense attention: q dtype {q.dtype} is not fp16/bf16/fp32")
    if q.dim() < 3 or k.dim() < 3 or v.dim() < 3:
        raise ValueError("dense attention needs [..., heads, tokens, head_dim] tensors")
    amf_hip.require_device_tensor(q, "dense attention q")
    lead = tuple(q.shape[:-3])
    Hq, Tq, D = q.shape[-3:]
    Hkv, T, Dk = k.shape[-3:]
    if Dk != D or tuple(v.shape[-3:]) != (Hkv, T, D):
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if Hq % Hkv != 0:
        raise ValueError(f"{Hq} query heads is not a multiple of {Hkv} KV heads")
    k = k.to(q.dtype).expand(*lead, Hkv, T, D).contiguous()
    v = v.to(q.dtype).expand(*lead, Hkv, T, D).contiguous()
    qc = q.contiguous()
    B = 1
    for d in lead:
        B *= int(d)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    mptr, ms = 0, (0, 0, 0, 0)
    m4 = None
    if mask is not None:
        m4 = mask.to(device=q.device, dtype=torch.float32).expand(*lead, Hq, Tq, T)
        m4 = m4.reshape(B, Hq, Tq, T)
        mptr, ms = m4.data_ptr(), tuple(m4.stride())
    # split-K scratch (per-split softmax partials), 0 bytes when the shape
    # takes the single-pass kernel
    wsb = _split_workspace_bytes(B, Hq, Hkv, Tq, T, D)
    stream = amf_hip.stream_handle(q.device)
    ws = _scratch(q.device, stream, wsb) if wsb else None
    amf_hip.call("amf_dense_attn", qc.data_ptr(), k.data_ptr(), v.data_ptr(),
                 amf_hip.dtype_tag(q.dtype), mptr, ms[0], ms[1], ms[2], ms[3], out.data_ptr(),
                 amf_hip.dtype_tag(out.dtype), B, Hq, Hkv, Tq, T, D, float(scale),
                 ws.data_ptr() if ws is not None else None, wsb, stream)
    return out


_FUSED_HEAD_DIMS = (64, 128, 256)


def _int4_sym_operands(c: Any, q: torch.Tensor) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(codes, scales) of an int4_sym CompressedKV that the fused kernel can
    read in place: codes uint8 [*lead, Hkv, T, D/2] contiguous, scales fp16
    [D], both on q's device, lead dims equal to q's; None otherwise."""
    if not isinstance(c, CompressedKV) or c.format != FMT_INT4_SYM:
        return None
    shape = c.shape
    if not isinstance(shape, tuple):
        shape = tuple(int(d) for d in shape)
    qs = q.shape
    if len(shape) != len(qs) or shape[-1] != qs[-1] or shape[:-3] != qs[:-3]:
        return None
    D = shape[-1]
    codes, scales = c.data, c.scales
    if not isinstance(codes, torch.Tensor) or not isinstance(scales, torch.Tensor):
        return None
    dev = q.device
    if (codes.dtype != torch.uint8 or codes.shape != shape[:-1] + (D // 2,)
            or not codes.is_contiguous() or codes.device != dev):
        return None
    if (scales.dtype != torch.float16 or scales.numel() != D or not scales.is_contiguous()
            or scales.device != dev):
        return None
    return codes, scales


def int4_sym_attention(q: torch.Tensor, k: Any, v: Any, scale: Optional[float],
                       mask: Optional[torch.Tensor], out_dtype: Optional[torch.dtype] = None
                       ) -> Optional[torch.Tensor]:
    """softmax(q k^T * scale + mask) v straight from int4_sym CompressedKV
    K and V (amf_int4_sym_dense_attn), without writing them out.  Head dim
    128 with bf16/fp16 q and no mask attends over the exactly dequantized
    values (code - 8) * scale on MFMA tiles; other shapes over the values
    decompress_to(q.dtype) would restore.  None when k/v are not int4_sym
    CompressedKV of q's layout or the head dim is not 64/128/256 (the caller
    then restores and runs dense_attention)."""
    if q.dtype not in _DTYPES or q.dim() < 3 or q.shape[-1] not in _FUSED_HEAD_DIMS:
        return None
    ko, vo = _int4_sym_operands(k, q), _int4_sym_operands(v, q)
    if ko is None or vo is None or tuple(k.shape) != tuple(v.shape):
        return None
    Hq, Tq, D = q.shape[-3:]
    Hkv, T = int(k.shape[-3]), int(k.shape[-2])
    if Hq % Hkv != 0:
        return None
    amf_hip.require_device_tensor(q, "int4_sym attention q")
    B = 1
    for d in q.shape[:-3]:
        B *= int(d)
    qc = q.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    mptr, ms = 0, (0, 0, 0, 0)
    m4 = None
    if mask is not None:
        m4 = mask.to(device=q.device, dtype=torch.float32).expand(*q.shape[:-3], Hq, Tq, T)
        m4 = m4.reshape(B, Hq, Tq, T)
        mptr, ms = m4.data_ptr(), tuple(m4.stride())
    wsb = _split_workspace_bytes(B, Hq, Hkv, Tq, T, D)
    if T > 0 and wsb == 0:
        return None  # beyond one split launch: the restoring path takes it
    stream = amf_hip.stream_handle(q.device)
    ws = _scratch(q.device, stream, wsb) if wsb else None
    amf_hip.call("amf_int4_sym_dense_attn", qc.data_ptr(), amf_hip.dtype_tag(q.dtype),
                 ko[0].data_ptr(), ko[1].data_ptr(), vo[0].data_ptr(), vo[1].data_ptr(), mptr,
                 ms[0], ms[1], ms[2], ms[3], out.data_ptr(), amf_hip.dtype_tag(out.dtype), B, Hq,
                 Hkv, Tq, T, D, float(scale), ws.data_ptr() if ws is not None else None, wsb,
                 stream)
    return out


def fallback_fp16_kernel(q: torch.Tensor, k_compressed: Any, v_compressed: Any, *,
                         scale: Optional[float] = None,
                         mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention over decompressed K/V: the reference's signature and result
    (dispatch.py:117-143), computed by the HIP dense-attention kernel.

    q [batch, heads, q_tokens, head_dim]; k/v a CompressedKV or a tensor
    [batch, kv_heads, kv_tokens, head_dim]; scale defaults to 1/sqrt(head_dim);
    mask is additive.  Returns q's shape and dtype."""
    fused = int4_sym_attention(q, k_compressed, v_compressed, scale, mask)
    if fused is not None:
        return fused
    k = _to_tensor(k_compressed, q)
    v = _to_tensor(v_compressed, q)
    return dense_attention(q, k, v, scale, mask)


# ------------------------------------------------------------ paged path --


def _check_buffer(t: torch.Tensor, what: str, dev: torch.device) -> None:
    """A caller buffer the kernel writes through a raw address: a contiguous
    tensor on the launch device, or ValueError before any launch."""
    if not isinstance(t, torch.Tensor) or t.device != dev:
        raise ValueError(f"paged decode: {what} must be a tensor on {dev}, got "
                         f"{getattr(t, 'device', type(t).__name__)}")
    if not t.is_contiguous():
        raise ValueError(f"paged decode: {what} must be contiguous")


def paged_int4_decode(q: torch.Tensor, kv: CompressedKV, block_tables: torch.Tensor,
                      context_lens: torch.Tensor, *, scale: Optional[float] = None,
                      max_context_len: Optional[int] = None, out: Optional[torch.Tensor] = None,
                      out_dtype: Optional[torch.dtype] = None, algo: str = "auto",
                      workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged GQA decode over an INT4 (int4_asym_g32) page pool.

    q [num_seqs, Hq, D] or [num_seqs, Hq, 1, D] (bf16/fp16); kv the
    CompressedKV of a layer's page tensor [2, pool_pages, 16, Hkv, D] (K and V
    planes); block_tables int32 [num_seqs, max_pages] of pool page ids;
    context_lens int32 [num_seqs].  max_context_len (>= every context length)
    sizes the grid and the split-K workspace; when omitted it is the block
    table's capacity, block_tables.shape[1] * 16, so no value is read back
    from the device.  `out` (contiguous [num_seqs, Hq, D] on the pool's
    device, bf16/fp16/fp32) and `workspace` (contiguous, on that device) are
    checked before the launch; a bad one raises ValueError.  algo: "auto"
    (= "mfma"), "mfma" (fp16 PV weights where a chunk's V scales allow),
    "mfma_precise" (bf16 hi/lo PV weights throughout) or "valu"."""
    layout = kv.meta.get("_layout") if isinstance(kv, CompressedKV) else None
    if layout is None or kv.format != FMT_INT4_ASYM_G32 or layout.n_planes != 2:
        raise ValueError("paged decode needs the int4_asym_g32 CompressedKV of a layer page "
                         "tensor [2, pool_pages, 16, kv_heads, head_dim]")
    blob = kv.meta["_blob"]
    dev = blob.device
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("paged decode takes one query token per sequence")
        q3 = q[:, :, 0]
    elif q.dim() == 3:
        q3 = q
    else:
        raise ValueError(f"q must be [seqs, heads, D] or [seqs, heads, 1, D], got {tuple(q.shape)}")
    if q3.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"paged decode: q dtype {q3.dtype} is not bf16/fp16")
    q3 = q3.to(dev).contiguous()
    S, Hq, D = q3.shape
    bt = torch.as_tensor(block_tables, dtype=torch.int32).to(dev).contiguous()
    cl = torch.as_tensor(context_lens, dtype=torch.int32).to(dev).contiguous()
    if bt.dim() != 2 or bt.shape[0] != S or cl.shape != (S,):
        raise ValueError(f"block_tables {tuple(bt.shape)} / context_lens {tuple(cl.shape)} do "
                         f"not match {S} sequences")
    if max_context_len is None:
        max_context_len = int(bt.shape[1]) * layout.block_size
    odt = out_dtype or (out.dtype if out is not None else q3.dtype)
    if odt not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"paged decode: output dtype {odt} is not bf16/fp16/fp32")
    if out is None:
        out = torch.empty(S, Hq, D, dtype=odt, device=dev)
    else:
        _check_buffer(out, "out", dev)
        if tuple(out.shape) != (S, Hq, D) and tuple(out.shape) != (S, Hq, 1, D):
            raise ValueError(f"paged decode: out has shape {tuple(out.shape)}, needs "
                             f"({S}, {Hq}, {D})")
        if out.dtype != odt:
            raise ValueError(f"paged decode: out is {out.dtype}, out_dtype asks for {odt}")
    wsb = amf_hip.decode_workspace_bytes(S, Hq, layout.num_heads, D, max_context_len)
    if workspace is not None:
        _check_buffer(workspace, "workspace", dev)
    stream = amf_hip.stream_handle(dev)
    if workspace is None or workspace.numel() * workspace.element_size() < wsb:
        workspace = _scratch(dev, stream, max(wsb, 4))
    algos = {"auto": amf_hip.DECODE_AUTO, "valu": amf_hip.DECODE_VALU, "mfma": amf_hip.DECODE_MFMA,
             "mfma_precise": amf_hip.DECODE_MFMA_PRECISE}
    amf_hip.call(
        "amf_int4_paged_decode_attn", q3.data_ptr(), amf_hip.dtype_tag(q3.dtype), out.data_ptr(),
        amf_hip.dtype_tag(out.dtype), blob.data_ptr() + layout.code_offset(0),
        blob.data_ptr() + layout.param_offset(0), blob.data_ptr() + layout.code_offset(1),
        blob.data_ptr() + layout.param_offset(1), layout.n_pages, bt.data_ptr(), bt.shape[1],
        cl.data_ptr(), S, Hq, layout.num_heads, D, layout.block_size, int(max_context_len),
        float(scale) if scale else 0.0, workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), algos[algo], None, stream)
    return out.view(q.shape) if q.dim() == 4 else out


def hip_decode_attention(q: torch.Tensor, k: Any, v: Any = None, scale: Optional[float] = None,
                         mask: Optional[torch.Tensor] = None, *,
                         block_tables: Optional[torch.Tensor] = None,
                         context_lens: Optional[torch.Tensor] = None,
                         max_context_len: Optional[int] = None,
                         out: Optional[torch.Tensor] = None,
                         out_dtype: Optional[torch.dtype] = None, algo: str = "auto",
                         workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The gfx950 decode kernel: positional arguments as the reference's
    (q, k, v, scale=None, mask=None); with block_tables/context_lens keywords,
    k is the INT4 page pool (v unused) and the paged GQA kernel runs."""
    if block_tables is not None or context_lens is not None:
        if block_tables is None or context_lens is None:
            raise ValueError("paged decode needs both block_tables and context_lens")
        if mask is not None:
            raise ValueError("paged decode takes no mask (causality is the context length)")
        if v is not None and v is not k:
            raise ValueError("paged decode reads K and V from the one page pool passed as k")
        return paged_int4_decode(q, k, block_tables, context_lens, scale=scale,
                                 max_context_len=max_context_len, out=out, out_dtype=out_dtype,
                                 algo=algo, workspace=workspace)
    res = int4_sym_attention(q, k, v, scale, mask, out_dtype)
    if res is None:
        res = dense_attention(q, _to_tensor(k, q), _to_tensor(v, q), scale, mask, out_dtype)
    if out is not None:
        out.copy_(res)
        return out
    return res


for _storage in (FMT_INT4_SYM, FMT_INT4_BLOCK, FMT_INT4_ASYM_G32, FMT_FP8_E4M3, FMT_FP8_E4M3_PH,
                 FMT_FP16, FMT_BF16):
    for _active in (FMT_FP8_E4M3, FMT_FP16, FMT_BF16):
        register_kernel(GFX950_VERSION, _storage, _active)(hip_decode_attention)


def try_load_cuda_extension(name: str = "axropus_kernels") -> Optional[Any]:
    """The compiled kernel library (libamf_hip.so, ctypes handle), or None when
    no device is present, AXROPUS_DISABLE_CUDA_BUILD is set, or the library
    is missing (reference: dispatch.py:174-230 returns None in the same
    cases).  The name is kept for API compatibility; `name` is ignored."""
    if not torch.cuda.is_available():
        return None
    if os.environ.get("AXROPUS_DISABLE_CUDA_BUILD", "") in ("1", "true", "yes", "on"):
        return None
    try:
        return amf_hip.load()
    except amf_hip.AmfHipUnavailable as exc:
        logger.warning("libamf_hip.so unavailable: %s", exc)
        return None


__all__ = [
    "GFX950_VERSION",
    "KERNEL_DISPATCH",
    "dense_attention",
    "int4_sym_attention",
    "dispatch_kernel",
    "fallback_fp16_kernel",
    "get_current_sm_version",
    "hip_decode_attention",
    "paged_int4_decode",
    "register_kernel",
    "try_load_cuda_extension",
]
