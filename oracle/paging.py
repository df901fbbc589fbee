"""CPU restatement of the page gather / scatter (test infrastructure only).

The reference moves pages with torch advanced indexing:
  gather  k_all[chunk_ids]            compressed_vram_pool.py:491-504,
                                      amf_kv_manager.py:311-318
  scatter k_all[chunk_ids] = src      compressed_vram_pool.py:599-606,
                                      amf_kv_manager.py:505-523
Both are restated on numpy arrays of raw bits (uint16 for bf16/fp16), which
makes them bit copies by construction.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np


def gather(cache: np.ndarray, block_ids: Sequence[int]) -> np.ndarray:
    """cache [P, pool, ...] -> [P, n, ...]: out[:, j] = cache[:, block_ids[j]]."""
    return cache[:, np.asarray(block_ids, dtype=np.int64)]


def scatter(cache: np.ndarray, block_ids: Sequence[int], src: np.ndarray) -> np.ndarray:
    """In-place cache[:, block_ids[j]] = src[:, j]; returns cache."""
    cache[:, np.asarray(block_ids, dtype=np.int64)] = src
    return cache
