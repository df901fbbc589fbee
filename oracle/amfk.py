"""AMFK snapshot format and FNV-1a keying (test infrastructure only).

Restates korith_vllm_ext/amf_kv_manager.py:36-134 (constants :38-64, hashes
:69-113, filename :118-134) and the header/table layout of
core/amf_direct_kv.h:35-72: a 56-byte little-endian header
<u32 magic, version, n_layers, n_tokens, n_kv_heads, head_dim, dtype, reserved,
 u64 total_kv_bytes, model_hash, prefix_hash> followed by a 32-byte
<u64 k_off, k_size, v_off, v_size> entry per layer, then the payload.
Pinned by the reference's golden values (platform/tests/test_vllm_amf.py:63-122,
128-162, 350-384; tests/test_direct_kv.py:129-189).
"""

from __future__ import annotations

import struct
from typing import Iterable, List, Sequence, Tuple

# The reference's offset basis (core/amf_store.cpp:27, amf_kv_manager.py:38) is
# 1469598103934665603, not the published FNV-1a basis 14695981039346656037.
FNV_OFFSET = 1469598103934665603
FNV_PRIME = 0x100000001B3
MASK64 = (1 << 64) - 1
AMFK_MAGIC = 0x414D464B
AMFK_VERSION = 1
HEADER = struct.Struct("<8I3Q")
LAYER = struct.Struct("<4Q")


def fnv1a_bytes(data: bytes, h: int = FNV_OFFSET) -> int:
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & MASK64
    return h


def hash_tokens(tokens: Iterable[int]) -> int:
    """One FNV-1a step per token on its 32-bit value (amf_kv_manager.py:75-81)."""
    h = FNV_OFFSET
    for t in tokens:
        h = ((h ^ (int(t) & 0xFFFFFFFF)) * FNV_PRIME) & MASK64
    return h


def hash_tenant(tenant: str) -> int:
    return FNV_OFFSET if not tenant else fnv1a_bytes(tenant.encode("utf-8"))


def float_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def key_filename(model_hash, tenant_hash, prefix_hash, n_ctx, kv_version, rope_base_bits,
                 rope_scale_bits, sampling_hash, rng_hash) -> str:
    return (f"amf_{model_hash:016x}_{tenant_hash:016x}_{prefix_hash:016x}_{n_ctx}_{kv_version}"
            f"_{rope_base_bits}_{rope_scale_bits}_{sampling_hash:016x}_{rng_hash:016x}")


def pack_header(n_layers, n_tokens, n_kv_heads, head_dim, dtype, total, model_hash,
                prefix_hash) -> bytes:
    return HEADER.pack(AMFK_MAGIC, AMFK_VERSION, n_layers, n_tokens, n_kv_heads, head_dim, dtype,
                       0, total, model_hash, prefix_hash)


def layer_table(sizes: Sequence[Tuple[int, int]]) -> List[Tuple[int, int, int, int]]:
    """(k_bytes, v_bytes) per layer -> (k_off, k_size, v_off, v_size), payload
    laid out K0 V0 K1 V1 ... (amf_kv_manager.py:327-333)."""
    out, off = [], 0
    for k, v in sizes:
        out.append((off, k, off + k, v))
        off += k + v
    return out
