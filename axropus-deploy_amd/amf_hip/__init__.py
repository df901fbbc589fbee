"""amf_hip - ctypes binding of libamf_hip.so (include/amf_hip.h).

The library is the gfx950 implementation of the AMF KV-materialization hot
path.  This module only loads it, declares the C signatures, checks the ABI
version, and turns negative status codes into :class:`AmfHipError`.  Tensors
cross the boundary as plain device addresses (``tensor.data_ptr()``) and the
current HIP stream handle; nothing here computes on the CPU.

Precedent for the ctypes probe pattern: platform/kernels/cuda/bindings.py:9-46
of the reference.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections import OrderedDict
from typing import Optional, Sequence

ABI_VERSION = 3

# status codes
OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_LAUNCH = -3
ERR_WORKSPACE = -4
ERR_FORMAT = -5
ERR_MISMATCH = -6
ERR_RUNTIME = -7

ERRFLAG_BLOCK_RANGE = 1
ERRFLAG_CONTEXT = 2
ERRFLAG_SYNC = 4

# element types (same numbering as the AMFK header dtype tag)
DTYPE_F16 = 0
DTYPE_F32 = 1
DTYPE_BF16 = 2

# codec formats
FMT_FP8_E4M3 = 1
FMT_FP8_E4M3_PH = 2
FMT_INT4_SYM_BLOCK = 3
FMT_INT4_SYM = 4
FMT_INT4_ASYM_G32 = 5

# decode algorithms
DECODE_AUTO = 0
DECODE_VALU = 1
DECODE_MFMA = 2
DECODE_MFMA_PRECISE = 3

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libamf_hip.so")

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_ptr = ctypes.c_void_p
_c_u32 = ctypes.c_uint32
_c_u64 = ctypes.c_uint64
_p_ptr = ctypes.POINTER(ctypes.c_void_p)
_p_u32 = ctypes.POINTER(ctypes.c_uint32)
_p_u64 = ctypes.POINTER(ctypes.c_uint64)

# name -> (restype, argtypes); every symbol declared in include/amf_hip.h.
SIGNATURES = {
    "amf_abi_version": (_c_i32, []),
    "amf_last_error": (ctypes.c_char_p, []),
    "amf_quant_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32]),
    "amf_kv_gather_pages": (
        _c_i32,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "amf_kv_scatter_pages": (
        _c_i32,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "amf_kv_gather_slots": (
        _c_i32,
        [_c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i64, _c_ptr,
         _c_ptr],
    ),
    "amf_kv_scatter_slots": (
        _c_i32,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i64, _c_ptr,
         _c_ptr],
    ),
    "amf_fp8_quant_gather": (
        _c_i32,
        [_c_i32, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i32, _c_i32, _c_i64,
         _c_i32, _c_i32, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr],
    ),
    "amf_fp8_dequant_scatter": (
        _c_i32,
        [_c_i32, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i32,
         _c_i32, _c_i32, _c_ptr, _c_ptr],
    ),
    "amf_int4_quant_gather": (
        _c_i32,
        [_c_i32, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i32, _c_i32, _c_i64,
         _c_i32, _c_i32, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr],
    ),
    "amf_int4_dequant_scatter": (
        _c_i32,
        [_c_i32, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i64, _c_i32, _c_i64, _c_i32,
         _c_i32, _c_i32, _c_ptr, _c_ptr],
    ),
    "amf_int4_decode_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "amf_int4_paged_decode_attn": (
        _c_i32,
        [_c_ptr, _c_i32, _c_ptr, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i32,
         _c_ptr,
         _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_ptr, _c_i64, _c_i32, _c_ptr,
         _c_ptr],
    ),
    "amf_int4_paged_decode_attn_noalloc": (
        _c_i32,
        [_c_ptr, _c_i32, _c_ptr, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i32,
         _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_ptr, _c_ptr],
    ),
    "amf_fnv1a64": (ctypes.c_uint64, [_c_ptr, _c_i64, ctypes.c_uint64]),
    "amf_hash_tokens": (ctypes.c_uint64, [_c_ptr, _c_i64]),
    "amf_dense_attn": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr, _c_i32, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i32,
         _c_i64, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_f32, _c_ptr, _c_i64, _c_ptr],
    ),
    "amf_dense_attn_workspace_bytes": (_c_i64, [_c_i64, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32]),
    "amf_int4_sym_dense_attn": (
        _c_i32,
        [_c_ptr, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_ptr, _c_i32, _c_i64, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_f32, _c_ptr, _c_i64,
         _c_ptr],
    ),
    "amf_direct_kv_init": (_c_ptr, [_c_u64]),
    "amf_direct_kv_free": (None, [_c_ptr]),
    "amf_direct_kv_is_direct_format": (_c_i32, [_c_ptr, _c_u64]),
    "amf_direct_kv_staging": (_c_i32, [_c_ptr, _c_u64, _p_ptr]),
    "amf_direct_kv_save": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_u32, _c_u32, _c_u32, _c_u32, _c_u64, _c_ptr,
         _c_i64, _p_ptr, _p_u64, _c_ptr],
    ),
    "amf_direct_kv_restore": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_u64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_u32, _p_u32, _c_ptr],
    ),
    "amf_direct_kv_save_pages": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_u32, _c_u32, _c_u32, _c_u32,
         _c_u64, _c_ptr, _c_i64, _c_ptr, _c_i64, _p_ptr, _p_u64, _c_ptr, _c_ptr],
    ),
    "amf_direct_kv_restore_pages": (
        _c_i32,
        [_c_ptr, _c_ptr, _c_u64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_u32, _c_ptr,
         _c_i64, _p_u32, _c_ptr, _c_ptr],
    ),
}


class AmfHipError(RuntimeError):
    """A libamf_hip.so call returned a negative status."""

    def __init__(self, func: str, code: int, message: str) -> None:
        super().__init__(f"{func} failed ({code}): {message}")
        self.func = func
        self.code = code
        self.message = message


class AmfHipUnavailable(RuntimeError):
    """libamf_hip.so is missing or does not match this binding."""


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load(path: Optional[str] = None) -> ctypes.CDLL:
    """Load (once) and return the library, with every signature declared."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or os.environ.get("AMF_HIP_LIB", LIB_PATH)
        if not os.path.exists(p):
            raise AmfHipUnavailable(
                f"{p} not found: build it with `make -C axropus-deploy_amd/csrc` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError: symbol missing
            fn.restype = res
            fn.argtypes = args
        got = lib.amf_abi_version()
        if got != ABI_VERSION:
            raise AmfHipUnavailable(f"{p}: ABI version {got}, binding expects {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except (AmfHipUnavailable, OSError, AttributeError):
        return False


def check(func: str, rc: int) -> None:
    if rc != OK:
        msg = load().amf_last_error()
        raise AmfHipError(func, rc, msg.decode() if msg else "")


def call(func: str, *args) -> None:
    """Call a status-returning entry point and raise on failure."""
    check(func, getattr(load(), func)(*args))


# ---------------------------------------------------------------- helpers --


def dtype_tag(dtype) -> int:
    import torch

    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float16:
        return DTYPE_F16
    if dtype == torch.float32:
        return DTYPE_F32
    raise ValueError(f"unsupported dtype {dtype}")


_CUDA_READY = False


def _device_index(device) -> int:
    global _CUDA_READY
    import torch

    if not _CUDA_READY:
        if not torch.cuda.is_initialized():
            torch.cuda.init()
        _CUDA_READY = True
    if isinstance(device, int):
        return device
    idx = getattr(device, "index", None)
    if idx is not None:
        return idx
    dev = torch.device(device)
    return torch.cuda.current_device() if dev.index is None else dev.index


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device` (0 = null stream);
    torch's raw-stream query, without building a Stream object."""
    import torch

    return int(torch._C._cuda_getCurrentRawStream(_device_index(device)))


_TABLES: "OrderedDict[tuple, object]" = OrderedDict()
_TABLES_MAX = 512


def to_device(host, device):
    """Copy a host tensor to `device` through pinned memory, queued on the
    current stream (no host wait for the stream's earlier work)."""
    import torch

    dev = torch.device(device)
    if dev.type != "cuda":
        return host.to(dev)
    return host.pin_memory().to(dev, non_blocking=True)


def address_table(addrs: Sequence[int], device):
    """Device int64 tensor holding `addrs` (a plane table).

    Tables are immutable and cached by content (least recently used dropped
    beyond _TABLES_MAX), so a launch over the same cache or blobs as an
    earlier one costs no host-to-device copy for its tables.  A table handed
    out on a stream other than the one it was made on is recorded on that
    stream, so that dropping it never frees memory a queued kernel still
    reads."""
    import torch

    dev = torch.device(device)
    key = (dev.type, dev.index, tuple(map(int, addrs)))
    sid = stream_handle(dev)
    with _lock:
        hit = _TABLES.get(key)
        if hit is not None:
            _TABLES.move_to_end(key)
    if hit is not None:
        t, streams = hit
        if sid not in streams:
            t.record_stream(torch.cuda.current_stream(dev))
            streams.add(sid)
        return t
    t = to_device(torch.tensor(list(key[2]), dtype=torch.int64), dev)
    with _lock:
        _TABLES[key] = (t, {sid})
        while len(_TABLES) > _TABLES_MAX:
            _TABLES.popitem(last=False)
    return t


def require_device_tensor(t, what: str) -> None:
    if not getattr(t, "is_cuda", False):
        raise RuntimeError(
            f"{what}: the AMF path runs on the GPU through libamf_hip.so; got a tensor on "
            f"{getattr(t, 'device', '?')}"
        )


def quant_workspace_bytes(fmt: int, n_planes: int, planes_per_scale: int, head_dim: int) -> int:
    return int(load().amf_quant_workspace_bytes(fmt, n_planes, planes_per_scale, head_dim))


def decode_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                           max_context_len: int) -> int:
    return int(
        load().amf_int4_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                               max_context_len)
    )
