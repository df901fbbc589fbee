"""codecs/amf_codec.py - FP8 / INT4 KV codecs on the GPU (libamf_hip.so).

Formats and the reference code whose results they reproduce bit for bit:
  fp8_e4m3        FP8E4M3Codec         amf_codec.py:174-222 (per-tensor scale)
  int4_sym        INT4PerChannelCodec  amf_codec.py:292-343
  int4_sym_block  INT4PerBlockCodec    amf_codec.py:345-447 (128-token blocks)
New formats (byte layouts in include/amf_hip.h):
  fp8_e4m3_ph     FP8 with one fp32 scale per (16-token page, head)
  int4_asym_g32   asymmetric INT4, fp16 (scale, zero) per (token, head, 32 dims)
Not implemented here (KeyError from get_codec): fp8_e5m2, int2_sym, nvfp4,
turboquant.

A tensor [..., T, H, D] is handled as planes (the leading dims) of pages of
T-tokens: 16 tokens, or the 128-token block of int4_sym_block; T is zero-padded
to whole pages, which changes no scale.  Per-tensor and per-channel scales span
every plane, as the reference's reductions over the whole tensor do.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Any, Optional

import torch

import amf_hip

from .. import _paged
from .base import (
    FMT_FP8_E4M3,
    FMT_FP8_E4M3_PH,
    FMT_INT4_ASYM_G32,
    FMT_INT4_BLOCK,
    FMT_INT4_SYM,
    Codec,
    CompressedKV,
    register_codec,
)

logger = logging.getLogger(__name__)

_FP8_E4M3_MAX = 448.0


# ---------------------------------------------------------------- sidecar --


@dataclass
class FP8ScaleSidecar:
    """The four fp32 scales that travel with an FP8 blob (the FP8 scale-drift
    fix, amf_codec.py:62-94): restore re-applies them instead of letting vLLM
    recompute scales on the warm batch."""

    k_scale: float
    v_scale: float
    q_scale: float = 1.0
    prob_scale: float = 1.0

    def to_tensor(self) -> torch.Tensor:
        return torch.tensor([self.k_scale, self.v_scale, self.q_scale, self.prob_scale],
                            dtype=torch.float32)

    @classmethod
    def from_tensor(cls, t: torch.Tensor) -> "FP8ScaleSidecar":
        v = [float(x) for x in t.flatten().tolist()]
        return cls(k_scale=v[0], v_scale=v[1], q_scale=v[2] if len(v) > 2 else 1.0,
                   prob_scale=v[3] if len(v) > 3 else 1.0)


# Attribute names vLLM versions and forks use for attention FP8 scales, the
# marker attributes that identify an attention module, and the flags that
# re-enable scale recomputation (amf_codec.py:119-158).
_MARKERS = ("_k_scale", "k_scale", "_kv_scale")
_SCALE_FIELDS = {
    "_k_scale": "k_scale", "_v_scale": "v_scale", "_q_scale": "q_scale",
    "_prob_scale": "prob_scale", "k_scale": "k_scale", "v_scale": "v_scale",
    "q_scale": "q_scale", "prob_scale": "prob_scale", "_k_scale_float": "k_scale",
    "_v_scale_float": "v_scale",
}
_RECOMPUTE_FLAGS = ("calculate_kv_scales", "_calculate_kv_scales",
                    "enable_kv_scales_calculation")


def apply_fp8_scales(model: Any, sidecar: FP8ScaleSidecar) -> None:
    """Write the sidecar's scales into every attention-like module of `model`
    (found by attribute, not class name) and switch scale recomputation off.
    Tensor attributes are filled in place so registered buffers/parameters
    stay the same objects."""
    written = 0
    try:
        modules = list(model.modules())
    except Exception as exc:  # pragma: no cover - duck-typed model
        logger.warning("apply_fp8_scales: cannot list modules: %s", exc)
        return
    for mod in modules:
        if not any(hasattr(mod, m) for m in _MARKERS):
            continue
        for attr, field_name in _SCALE_FIELDS.items():
            if not hasattr(mod, attr):
                continue
            value = getattr(sidecar, field_name)
            try:
                cur = getattr(mod, attr)
                if isinstance(cur, torch.Tensor):
                    cur.data.fill_(value)
                else:
                    setattr(mod, attr, value)
                written += 1
            except (AttributeError, TypeError, RuntimeError):
                pass
        for flag in _RECOMPUTE_FLAGS:
            if hasattr(mod, flag):
                try:
                    setattr(mod, flag, False)
                except (AttributeError, TypeError):
                    pass
    logger.debug("apply_fp8_scales: %d attributes set (k=%.4g v=%.4g)", written,
                 sidecar.k_scale, sidecar.v_scale)


# ------------------------------------------------------------ HIP codecs --

# Floor of the per-tensor FP8 absmax: clamp_min_(1e-8) runs in the tensor's
# own dtype (amf_codec.py:183), so the floor is 1e-8 rounded to that dtype.
_FP8_FLOOR = {
    torch.bfloat16: float(torch.tensor(1e-8, dtype=torch.bfloat16)),
    torch.float16: float(torch.tensor(1e-8, dtype=torch.float16)),
    torch.float32: float(torch.tensor(1e-8, dtype=torch.float32)),
}


def tensor_scale_from_absmax(absmax: float, dtype: torch.dtype) -> float:
    """FP8E4M3Codec's Python-double tensor_scale (amf_codec.py:182-184)."""
    return max(absmax, _FP8_FLOOR[dtype]) / _FP8_E4M3_MAX


class _HipCodec(Codec):
    """Common compress / decompress over dense tensors through the kernels."""

    FORMAT = ""
    RATIO = 0.25

    def memory_ratio(self) -> float:
        return self.RATIO

    def _check_input(self, raw_kv: torch.Tensor) -> None:
        if raw_kv.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise TypeError(f"{type(self).__name__} cannot accept dtype {raw_kv.dtype}")
        if raw_kv.dim() < 3:
            raise ValueError(f"{self.FORMAT} needs [..., tokens, heads, head_dim], got "
                             f"{tuple(raw_kv.shape)}")
        amf_hip.require_device_tensor(raw_kv, f"{self.FORMAT} compress")

    def _page_tokens(self, T: int) -> int:
        """Tokens per page for a dense tensor of T tokens along dim -3.

        int4_sym_block blocks 128 tokens (amf_codec.py:353-370): one page of T
        tokens when T <= 128 (no padding), else 128-token pages.  The
        per-(page, head) and group formats define 16-token pages.  The
        per-tensor and per-channel scales do not depend on paging: 16-token
        pages when 16 divides T, else one page of T tokens up to 256, else
        zero-padded 16-token pages."""
        if self.FORMAT == FMT_INT4_BLOCK:
            return T if 0 < T <= 128 else 128
        if self.FORMAT in (FMT_FP8_E4M3_PH, FMT_INT4_ASYM_G32):
            return 16
        if T % 16 == 0 or T > 256:
            return 16
        return max(T, 1)

    def _flat_rows(self, x: torch.Tensor) -> int:
        """Rows per page when x is compressed as one plane of its D-element
        rows, else 0.  The per-tensor FP8 scale and the per-channel INT4
        scales do not depend on paging, and the codes keep the input's
        memory order either way, so a tensor whose dim -3 is short (e.g.
        [batch, kv_heads, tokens, head_dim]) is cut into pages of about 16K
        elements instead of a few pages of dim -3's length.  The rows per
        page are the largest power of two up to 16384 / D dividing the row
        count, and a page must fill one workgroup pass (2048 elements)."""
        if self.FORMAT not in (FMT_FP8_E4M3, FMT_INT4_SYM) or self._is_page_tensor(x):
            return 0
        D = int(x.shape[-1])
        if D <= 0 or x.numel() == 0:
            return 0
        rows = x.numel() // D
        bs = 1
        while bs * 2 * D <= 16384 and rows % (bs * 2) == 0:
            bs *= 2
        return bs if bs * D >= 2048 else 0

    def _is_page_tensor(self, x: torch.Tensor) -> bool:
        """A layer page tensor [2, nb, bs, H, D] whose pages are exactly the
        dense grouping of [..., T=bs, H, D]: compressed as 2 planes of nb
        pages instead of 2*nb one-page planes (same codes and scales)."""
        if x.dim() != 5 or x.shape[0] != 2:
            return False
        bs = int(x.shape[2])
        if self.FORMAT == FMT_INT4_BLOCK:
            return bs <= 128
        if self.FORMAT in (FMT_FP8_E4M3_PH, FMT_INT4_ASYM_G32):
            return bs == 16
        return True

    def compress(self, raw_kv: torch.Tensor) -> CompressedKV:
        self._check_input(raw_kv)
        x = raw_kv.detach().contiguous()
        flat = self._flat_rows(x)
        if self._is_page_tensor(x):
            _, nb, bs, H, D = x.shape
            view = _paged.planes_view([x[0], x[1]])
            n_pages, page, T = nb, bs, nb * bs
        elif flat:
            # one plane of D-element rows in memory order, `flat` rows a page
            D, H = int(x.shape[-1]), 1
            T = x.numel() // D
            page, n_pages = flat, T // flat
            view = _paged.CacheView([x.data_ptr()], page * D * x.element_size(), n_pages, page,
                                    1, D, x.dtype, x.device, keep=[x])
        else:
            T, H, D = x.shape[-3:]
            page = self._page_tokens(T)
            view, n_pages, _keep = _paged.dense_view(x, page)
        P = len(view.planes)
        layout = _paged.BlobLayout(self.FORMAT, P, n_pages, page, H, D)
        layout.validate()
        blob = torch.empty(layout.total_bytes, dtype=torch.uint8, device=raw_kv.device)
        ws = _paged.quant_gather(layout, view, None, [blob.data_ptr()], P)
        absmax = None
        if ws is not None and self.FORMAT == FMT_FP8_E4M3:
            absmax = float(ws[:1].view(torch.int32).cpu().view(torch.float32))
        return self.wrap_blob(blob, 0, layout, tuple(raw_kv.shape), raw_kv.dtype, absmax, T)

    def wrap_blob(self, storage: torch.Tensor, offset: int, layout: "_paged.BlobLayout",
                  shape: tuple, dtype: torch.dtype, absmax: Optional[float],
                  n_tokens: int, scale: Optional[float] = None) -> CompressedKV:
        """CompressedKV whose tensors are views of storage[offset:] (a blob of
        `layout`).  absmax: the scale group's absmax after a per-tensor FP8
        save (gives the reference's Python-double tensor_scale); scale: that
        tensor_scale when the caller already has it or will set it later (no
        device read either way)."""
        blob = storage.narrow(0, offset, layout.total_bytes)
        data, scales, tensor_scale, meta = self._views(blob, layout, shape, dtype, absmax,
                                                       n_tokens, scale)
        meta.update({"_blob": blob, "_layout": layout, "n_tokens": n_tokens})
        return CompressedKV(format=self.FORMAT, data=data, scales=scales,
                            tensor_scale=tensor_scale, shape=shape, dtype_original=dtype,
                            meta=meta)

    def _code_view(self, blob, layout, n_tokens, dtype, shape):
        """Codes in the input's shape (last dim D, or D/2 packed nibbles): a
        view of the blob unless token padding forces a copy."""
        P, n, bs, H, D = (layout.n_planes, layout.n_pages, layout.block_size, layout.num_heads,
                          layout.head_dim)
        per_tok = D if layout.family == "fp8" else D // 2
        codes = blob.narrow(0, 0, layout.data_bytes).view(P, n * bs, H, per_tok)
        if dtype is not None:
            codes = codes.view(dtype)
        return codes[:, :n_tokens].reshape(*shape[:-1], per_tok)

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        raise NotImplementedError

    def decompress_to(self, compressed: CompressedKV,
                      target_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        blob = compressed.meta.get("_blob")
        layout = compressed.meta.get("_layout")
        if blob is None or layout is None:
            raise ValueError("CompressedKV was not produced by these codecs")
        P, n, bs, H, D = (layout.n_planes, layout.n_pages, layout.block_size, layout.num_heads,
                          layout.head_dim)
        out = torch.empty(P, n, bs, H, D, dtype=target_dtype, device=blob.device)
        view = _paged.planes_view([out[p] for p in range(P)])
        _paged.dequant_scatter(layout, [blob.data_ptr()], P, view, None)
        T = compressed.meta["n_tokens"]
        return out.view(P, n * bs, H, D)[:, :T].reshape(compressed.shape)


class FP8E4M3Codec(_HipCodec):
    """FP8 e4m3fn, one scale for the whole tensor (amf_codec.py:174-222)."""

    FORMAT = FMT_FP8_E4M3
    RATIO = 0.5

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        data = self._code_view(blob, layout, n_tokens, torch.float8_e4m3fn, shape)
        scales = blob.narrow(0, layout.scale_offset, 16).view(torch.float32)
        if scale is not None:
            pass
        elif absmax is not None:
            scale = tensor_scale_from_absmax(absmax, dtype)
        else:
            scale = float(scales[0])
        sidecar = FP8ScaleSidecar(k_scale=scale, v_scale=scale)
        return data, scales, scale, {"sidecar": sidecar}


class FP8PageHeadCodec(_HipCodec):
    """FP8 e4m3fn with one fp32 scale per (16-token page, head)."""

    FORMAT = FMT_FP8_E4M3_PH
    RATIO = 0.5

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        data = self._code_view(blob, layout, n_tokens, torch.float8_e4m3fn, shape)
        stride = _paged._align16(layout.plane_param_bytes) // 4
        fl = blob.narrow(0, layout.scale_offset, layout.scale_bytes).view(torch.float32)
        scales = fl.as_strided((layout.n_planes, layout.n_pages, layout.num_heads),
                               (stride, layout.num_heads, 1))
        return data, scales, 1.0, {"granularity": "page_head", "page_tokens": layout.block_size}


class INT4PerChannelCodec(_HipCodec):
    """Symmetric INT4, one fp16 scale per head_dim channel (amf_codec.py:292-343)."""

    FORMAT = FMT_INT4_SYM
    RATIO = 0.25

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        data = self._code_view(blob, layout, n_tokens, None, shape)
        scales = blob.narrow(0, layout.scale_offset, layout.head_dim * 2).view(torch.float16)
        return data, scales, 1.0, {"zero_point": 0}


class INT4PerBlockCodec(_HipCodec):
    """Symmetric INT4, one fp16 scale per 128-token block (amf_codec.py:345-447)."""

    FORMAT = FMT_INT4_BLOCK
    BLOCK = 128
    RATIO = 0.25

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        data = self._code_view(blob, layout, n_tokens, None, shape)
        stride = _paged._align16(layout.plane_param_bytes) // 2
        hv = blob.narrow(0, layout.scale_offset, layout.scale_bytes).view(torch.float16)
        scales = hv.as_strided((layout.n_planes, layout.n_pages), (stride, 1))
        # [*leading dims, blocks of dim -3] as INT4PerBlockCodec returns them
        # (amf_codec.py:404); a page tensor has one block per (K/V, page).
        lead = 1
        for d in shape[:-3]:
            lead *= int(d)
        n_blocks = layout.n_planes * layout.n_pages // lead
        scales = scales.reshape(*shape[:-3], n_blocks)
        meta = {"block_size": 128, "n_tokens": int(shape[-3]), "n_blocks": n_blocks}
        return data, scales, 1.0, meta


class INT4AsymG32Codec(_HipCodec):
    """Asymmetric INT4, fp16 (scale, zero) per (token, head, 32-dim group);
    head-major pages with dim-major V tiles (include/amf_hip.h)."""

    FORMAT = FMT_INT4_ASYM_G32
    RATIO = 0.3125  # (0.5 code bytes + 4 param bytes / 32) per element, over 2 bytes

    def _views(self, blob, layout, shape, dtype, absmax, n_tokens, scale=None):
        P, n = layout.n_planes, layout.n_pages
        data = blob.narrow(0, 0, layout.data_bytes).view(P, n, layout.code_bytes_per_page)
        stride = _paged._align16(layout.plane_param_bytes) // 4
        iv = blob.narrow(0, layout.scale_offset, layout.scale_bytes).view(torch.int32)
        words = layout.plane_param_bytes // 4 // n
        scales = iv.as_strided((P, n, words), (stride, words, 1))
        meta = {"page_tokens": layout.block_size,
                "layout": "head-major pages; K token-major, V dim-major 8x8 tiles"}
        return data, scales, 1.0, meta


for _codec in (FP8E4M3Codec(), FP8PageHeadCodec(), INT4PerChannelCodec(), INT4PerBlockCodec(),
               INT4AsymG32Codec()):
    register_codec(_codec)


__all__ = [
    "FP8E4M3Codec",
    "FP8PageHeadCodec",
    "FP8ScaleSidecar",
    "INT4AsymG32Codec",
    "INT4PerBlockCodec",
    "INT4PerChannelCodec",
    "apply_fp8_scales",
    "tensor_scale_from_absmax",
]
