"""Decode-attention oracles (test infrastructure only).

paged_decode_f64: softmax(q k^T * scale) v in float64 over a paged KV pool,
with GQA (query head h reads KV head h // (Hq / Hkv)).  It restates the
math of the reference's fallback (kernels/dispatch.py:117-143: matmul,
softmax, matmul) adding the paging and GQA that its CUDA kernel lacked
(kernels/int4_decode_attention.cu:39-177 walks one dense [T, D] head).

fallback_attention: the reference's own dense fallback in q.dtype
(dispatch.py:117-143), used only to report how far the reference's bf16
path sits from the float64 result.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch


def paged_decode_f64(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                     block_tables: np.ndarray, context_lens: np.ndarray,
                     scale: Optional[float] = None) -> np.ndarray:
    """q [B, Hq, D]; k_pool, v_pool [pool, bs, Hkv, D]; block_tables [B, M];
    context_lens [B] -> out [B, Hq, D] float64."""
    B, Hq, D = q.shape
    bs, Hkv = k_pool.shape[1], k_pool.shape[2]
    R = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx == 0:
            continue
        n = -(-ctx // bs)
        pages = np.asarray(block_tables[b, :n], dtype=np.int64)
        K = k_pool[pages].reshape(n * bs, Hkv, D)[:ctx].astype(np.float64)
        V = v_pool[pages].reshape(n * bs, Hkv, D)[:ctx].astype(np.float64)
        for h in range(Hkv):
            qs = q[b, h * R:(h + 1) * R].astype(np.float64)        # [R, D]
            s = (qs @ K[:, h].T) * scale                            # [R, ctx]
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, h * R:(h + 1) * R] = p @ V[:, h]
    return out


def fallback_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       scale: Optional[float] = None,
                       mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dispatch.py:117-143 semantics: dense [B, H, Tq, D] attention computed in
    q.dtype (matmul -> softmax -> matmul)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    attn = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    if mask is not None:
        attn = attn + mask
    return torch.matmul(torch.softmax(attn, dim=-1), v)


def dense_attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                        scale: Optional[float] = None,
                        mask: Optional[np.ndarray] = None) -> np.ndarray:
    """softmax(q k^T * scale + mask) v in float64 (dispatch.py:117-143 math),
    q [B, Hq, Tq, D], k/v [B, Hkv, T, D] with GQA (query head h reads KV head
    h // (Hq / Hkv)), mask broadcastable to [B, Hq, Tq, T].  T == 0 gives
    zeros (an empty sum); a row of all -inf scores gives NaN."""
    B, Hq, Tq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    R = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, Tq, D), dtype=np.float64)
    if T == 0:
        return out
    kk = np.repeat(k.astype(np.float64), R, axis=1)
    vv = np.repeat(v.astype(np.float64), R, axis=1)
    s = np.einsum("bhqd,bhtd->bhqt", q.astype(np.float64), kk) * scale
    if mask is not None:
        s = s + np.broadcast_to(mask.astype(np.float64), s.shape)
    with np.errstate(invalid="ignore"):
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqt,bhtd->bhqd", p, vv)
