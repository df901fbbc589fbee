"""Shared helpers of the test suite (not collected)."""

from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a 2-byte tensor as a numpy uint16 array (CPU copy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bytes_of(t: torch.Tensor) -> np.ndarray:
    """Raw bytes of a tensor, flattened (CPU copy)."""
    return t.detach().contiguous().view(torch.uint8).cpu().numpy().ravel()


def sentinel_cache(L: int, pool: int, bs: int, H: int, D: int, dtype, device,
                   value: float = -7.25) -> List[torch.Tensor]:
    return [torch.full((2, pool, bs, H, D), value, dtype=dtype, device=device) for _ in range(L)]


def attn_errors(got: np.ndarray, ref: np.ndarray) -> Tuple[float, float]:
    """(max |a - b|, sum |a - b| / sum |b|)."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()) if d.size else 0.0, float(d.sum() / max(np.abs(ref).sum(), 1e-30))


def check_attention(got: np.ndarray, ref: np.ndarray, max_abs: float = 2e-2,
                    mean_rel: float = 1e-2, label: str = "") -> Tuple[float, float]:
    """Asserts max-abs / mean-rel bounds and prints the measured errors."""
    ma, mr = attn_errors(got, ref)
    print(f"attention error{' ' + label if label else ''}: max_abs={ma:.3e} mean_rel={mr:.3e} "
          f"(bounds {max_abs:.0e} / {mean_rel:.0e})", flush=True)
    assert ma <= max_abs and mr <= mean_rel, f"max_abs={ma:.3e} mean_rel={mr:.3e}"
    return ma, mr
