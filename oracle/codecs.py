"""CPU restatement of the AMF codecs (test infrastructure only).

Reference formats follow korith_vllm_ext/codecs/amf_codec.py op for op on CPU
torch tensors, because their rounding is defined by that op sequence:
  fp8_e4m3        amf_codec.py:182-222
  int4_sym        amf_codec.py:305-343
  int4_sym_block  amf_codec.py:358-447
  pack / unpack   amf_codec.py:502-539
New formats (no reference counterpart) follow the spec in include/amf_hip.h:
  fp8_e4m3_ph     per-(page, head) fp32 scale
  int4_asym_g32   per-(token, head, 32-dim group) fp16 (scale, zero), with the
                  head-major page layout and dim-major V tiles.
Page tensors are [P, n, bs, H, D] (P planes, n pages); the reference applies
its codecs to one layer's [2, nb, bs, H, D].
"""

from __future__ import annotations

import math
from typing import Dict, Tuple

import numpy as np
import torch

E4M3_MAX = 448.0

# ------------------------------------------------------------------ FP8 ---


def fp8_tensor_compress(x: torch.Tensor) -> Tuple[torch.Tensor, float]:
    """FP8E4M3Codec.compress (amf_codec.py:182-209): one scale for the whole
    tensor; returns (e4m3 codes as uint8, tensor_scale as a Python float)."""
    peak = x.detach().abs().amax().clamp_min_(1e-8)   # in x's dtype, like :183
    scale = float(peak) / E4M3_MAX                      # Python double, :184
    divisor = scale if scale > 1e-12 else 1e-12         # :191 max(scale, 1e-12)
    y = (x.float() / divisor).clamp_(-E4M3_MAX, E4M3_MAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8), scale


def fp8_tensor_decompress(codes: torch.Tensor, scale: float, dtype: torch.dtype) -> torch.Tensor:
    """FP8E4M3Codec.decompress_to (amf_codec.py:211-222)."""
    return (codes.view(torch.float8_e4m3fn).to(torch.float32) * scale).to(dtype)


def fp8_sidecar(scale: float) -> torch.Tensor:
    """FP8ScaleSidecar(k_scale=scale, v_scale=scale).to_tensor() (amf_codec.py:80-84, 200)."""
    return torch.tensor([scale, scale, 1.0, 1.0], dtype=torch.float32)


def fp8_ph_compress(pages: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp8_e4m3_ph: pages [P, n, bs, H, D] -> (codes uint8 same shape, scales
    fp32 [P, n, H]); scale = max(absmax over (bs, D), 1e-8) / 448."""
    x = pages.float()
    peak = x.abs().amax(dim=(2, 4))
    scale = torch.clamp_min(peak, 1e-8) / E4M3_MAX
    y = (x / scale[:, :, None, :, None]).clamp(-E4M3_MAX, E4M3_MAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8), scale


def fp8_ph_decompress(codes: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    v = codes.view(torch.float8_e4m3fn).to(torch.float32)
    return (v * scales[:, :, None, :, None]).to(dtype)


# ------------------------------------------------------- INT4 nibbles ----


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """_pack_int4 (amf_codec.py:502-521): u = q + 8, element 2i in the low
    nibble, odd lengths zero-padded."""
    u = (q.to(torch.int16) + 8).to(torch.uint8)
    if u.shape[-1] % 2:
        u = torch.cat([u, torch.zeros_like(u[..., :1])], dim=-1)
    return (u[..., 1::2] << 4) | u[..., 0::2]


def unpack_int4(packed: torch.Tensor, last: int) -> torch.Tensor:
    """_unpack_int4 (amf_codec.py:524-539) -> int8 in [-8, 7]."""
    lo = (packed & 0x0F).to(torch.int16)
    hi = (packed >> 4).to(torch.int16)
    both = torch.stack([lo, hi], dim=-1).flatten(-2)[..., :last]
    return (both - 8).to(torch.int8)


def pack_nibbles(u: torch.Tensor) -> torch.Tensor:
    """Unsigned 4-bit values -> bytes, element 2i in the low nibble."""
    u = u.to(torch.uint8)
    return (u[..., 1::2] << 4) | u[..., 0::2]


def unpack_nibbles(b: torch.Tensor) -> torch.Tensor:
    return torch.stack([b & 0x0F, b >> 4], dim=-1).flatten(-2)


# ------------------------------------------------------- INT4 symmetric ---


def int4_channel_compress(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """INT4PerChannelCodec.compress (amf_codec.py:305-330): one scale per
    last-dim channel over all other dims.  Returns (packed, fp16 scales [D])."""
    xf = x.float()
    dims = tuple(range(xf.dim() - 1))
    scale = xf.abs().amax(dim=dims).clamp_min(1e-8) / 7.0
    q = torch.round(xf / scale).clamp(-8, 7).to(torch.int8)
    return pack_int4(q), scale.to(torch.float16)


def int4_channel_decompress(packed: torch.Tensor, scales: torch.Tensor, shape, dtype) -> torch.Tensor:
    """INT4PerChannelCodec.decompress_to (amf_codec.py:332-343)."""
    q = unpack_int4(packed, shape[-1]).view(shape)
    return (q.float() * scales.float()).to(dtype)


def int4_block_compress(x: torch.Tensor, block: int = 128) -> Tuple[torch.Tensor, torch.Tensor, Dict]:
    """INT4PerBlockCodec.compress (amf_codec.py:358-408): token axis -3 cut in
    `block`-token blocks (zero padded); one scale per (leading index, block)
    over every head and dim.  Returns (packed, fp16 scales [..., n_blocks], meta)."""
    xf = x.float()
    T, H, D = xf.shape[-3:]
    nb = math.ceil(T / block)
    if nb * block != T:
        pad = torch.zeros(*xf.shape[:-3], nb * block - T, H, D)
        xf = torch.cat([xf, pad], dim=-3)
    blocks = xf.reshape(*xf.shape[:-3], nb, block, H, D)
    scale = blocks.abs().amax(dim=(-3, -2, -1), keepdim=True).clamp_min(1e-8) / 7.0
    q = torch.round(blocks / scale).clamp(-8, 7).to(torch.int8)
    q = q.reshape(*q.shape[:-4], nb * block, H, D)[..., :T, :, :]
    scales = scale.reshape(*scale.shape[:-3]).to(torch.float16)
    return pack_int4(q), scales, {"block_size": block, "n_tokens": T, "n_blocks": nb}


def int4_block_decompress(packed: torch.Tensor, scales: torch.Tensor, shape, meta, dtype) -> torch.Tensor:
    """INT4PerBlockCodec.decompress_to (amf_codec.py:410-447)."""
    q = unpack_int4(packed, shape[-1]).view(shape).float()
    T, H, D = shape[-3:]
    block, nb = meta["block_size"], meta["n_blocks"]
    if nb * block != T:
        q = torch.cat([q, torch.zeros(*q.shape[:-3], nb * block - T, H, D)], dim=-3)
    qb = q.reshape(*q.shape[:-3], nb, block, H, D)
    out = (qb * scales.float().reshape(*scales.shape, 1, 1, 1)).reshape(*q.shape)
    return out[..., :T, :, :].to(dtype)


# ------------------------------------------------- INT4 asymmetric g32 ----


def int4_asym_quantize(pages: torch.Tensor):
    """Group quantizer of int4_asym_g32 on pages [P, n, 16, H, D].

    Returns (u int64 codes [P, n, 16, H, D], scale16, zero16 [P, n, 16, H, G])."""
    x = pages.float()
    P, n, bs, H, D = x.shape
    G = D // 32
    xg = x.reshape(P, n, bs, H, G, 32)
    mn = xg.amin(dim=-1)
    mx = xg.amax(dim=-1)
    scale = torch.clamp_min(mx - mn, 1e-8) / 15.0
    u = torch.round((xg - mn[..., None]) / scale[..., None]).clamp(0, 15).to(torch.int64)
    return u.reshape(P, n, bs, H, D), scale.to(torch.float16), mn.to(torch.float16)


def int4_asym_dequant_f32(u: torch.Tensor, s16: torch.Tensor, z16: torch.Tensor) -> torch.Tensor:
    """fp32 dequantised values q * s + z (unfused multiply then add)."""
    P, n, bs, H, D = u.shape
    G = D // 32
    ug = u.reshape(P, n, bs, H, G, 32).float()
    prod = ug * s16.float()[..., None]
    return (prod + z16.float()[..., None]).reshape(P, n, bs, H, D)


def _param_words(s16: torch.Tensor, z16: torch.Tensor) -> torch.Tensor:
    s = s16.view(torch.int16).to(torch.int64) & 0xFFFF
    z = z16.view(torch.int16).to(torch.int64) & 0xFFFF
    return (s | (z << 16)).to(torch.int64)


def int4_asym_layout(u: torch.Tensor, s16: torch.Tensor, z16: torch.Tensor):
    """Byte layout of int4_asym_g32 (include/amf_hip.h): even planes K, odd V.

    Returns (codes uint8 [P, n, H * 16 * D / 2], params uint32-as-int64
    [P, n, H * 16 * G]); both head-major per page."""
    P, n, bs, H, D = u.shape
    G = D // 32
    words = _param_words(s16, z16)                      # [P, n, bs, H, G]
    codes, params = [], []
    for p in range(P):
        up = u[p]                                       # [n, bs, H, D]
        wp = words[p]                                   # [n, bs, H, G]
        if p % 2 == 0:
            c = pack_nibbles(up.permute(0, 2, 1, 3))    # [n, H, bs, D/2]
            w = wp.permute(0, 2, 1, 3)                  # [n, H, bs, G]
        else:
            # [n, H, D, bs] -> [n, H, D/8, 8 dims, 2 halves, 8 tokens]
            t = up.permute(0, 2, 3, 1).reshape(n, H, D // 8, 8, 2, 8)
            t = t.permute(0, 1, 2, 4, 3, 5)            # [n, H, D/8, half, dim, token]
            c = pack_nibbles(t)                         # [..., 4 bytes]
            w = wp.permute(0, 2, 3, 1)                  # [n, H, G, bs]
        codes.append(c.reshape(n, -1))
        params.append(w.reshape(n, -1))
    return torch.stack(codes), torch.stack(params)


def int4_asym_unlayout(codes: torch.Tensor, params: torch.Tensor, bs: int, H: int, D: int):
    """Inverse of int4_asym_layout -> (u, s16, z16)."""
    P, n = codes.shape[:2]
    G = D // 32
    us, ws = [], []
    for p in range(P):
        c = unpack_nibbles(codes[p].reshape(n, -1)).to(torch.int64)
        w = params[p]
        if p % 2 == 0:
            u = c.reshape(n, H, bs, D).permute(0, 2, 1, 3)
            w = w.reshape(n, H, bs, G).permute(0, 2, 1, 3)
        else:
            t = c.reshape(n, H, D // 8, 2, 8, 8).permute(0, 1, 2, 4, 3, 5)
            u = t.reshape(n, H, D, bs).permute(0, 3, 1, 2)
            w = w.reshape(n, H, G, bs).permute(0, 3, 1, 2)
        us.append(u)
        ws.append(w)
    u = torch.stack(us).contiguous()
    w = torch.stack(ws).contiguous().numpy()
    s16 = torch.from_numpy((w & 0xFFFF).astype(np.uint16).view(np.float16))
    z16 = torch.from_numpy(((w >> 16) & 0xFFFF).astype(np.uint16).view(np.float16))
    return u, s16, z16


def int4_asym_compress(pages: torch.Tensor):
    u, s16, z16 = int4_asym_quantize(pages)
    return int4_asym_layout(u, s16, z16)


def int4_asym_decompress(codes, params, bs, H, D, dtype) -> torch.Tensor:
    u, s16, z16 = int4_asym_unlayout(codes, params, bs, H, D)
    return int4_asym_dequant_f32(u, s16, z16).to(dtype)
