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


# ------------------------------------------------------------- token slots --
#
# The connector's token-slot form (korith_vllm_ext/amf_kv_connector.py):
#   slots   AMFReqMeta.make                          :90-115
#   save    flat[:, slots, :, :].clone()              :411-422
#   load    flat_cache[:, slots, ...] = kv_slice      :374-385
#   hash    _prefix_hash (SHA-256, 4-byte LE words)   :64-69
#   align   align_to_block_size                       :72-74


def align_to_block_size(num_tokens: int, block_size: int) -> int:
    """Largest multiple of block_size strictly below num_tokens (floor
    division, so 0 tokens give -block_size)."""
    return ((num_tokens - 1) // block_size) * block_size


def slot_mapping(block_ids: Sequence[int], block_size: int, n_tokens: int) -> list:
    """Token i of the request sits at slot block_ids[i // bs] * bs + i % bs;
    the list is cut to n_tokens with Python slice rules."""
    slots = []
    for b in block_ids:
        for off in range(block_size):
            slots.append(int(b) * block_size + off)
    return slots[:n_tokens]


def gather_slots(cache: np.ndarray, slots: Sequence[int]) -> np.ndarray:
    """cache [P, nb, bs, ...] -> [P, n, ...]: row j = flat slot slots[j]."""
    P, nb, bs = cache.shape[:3]
    flat = cache.reshape(P, nb * bs, *cache.shape[3:])
    return flat[:, np.asarray(slots, dtype=np.int64)]


def scatter_slots(cache: np.ndarray, slots: Sequence[int], src: np.ndarray) -> np.ndarray:
    """In place: flat slot slots[j] of every plane <- src[:, j]; returns cache."""
    bs = cache.shape[2]
    for j, s in enumerate(slots):
        page, off = divmod(int(s), bs)
        cache[:, page, off] = src[:, j]
    return cache


def prefix_hash(tokens: Sequence[int]) -> str:
    """SHA-256 of the tokens packed as unsigned 32-bit little-endian words
    (values taken mod 2**32), first 16 hex digits."""
    import hashlib
    import struct

    data = b"".join(struct.pack("<I", int(t) % (1 << 32)) for t in tokens)
    return hashlib.sha256(data).hexdigest()[:16]
