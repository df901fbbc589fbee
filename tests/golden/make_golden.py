"""Writes the golden fixtures of this directory (run from the repo root:
`python tests/golden/make_golden.py`).

reference_vectors.json: known answers held by the reference's own tests,
  transcribed as data - FNV-1a goldens (platform/tests/test_vllm_amf.py:
  63-122), the cross-backend file name (:350-384), the AMFK header layout
  (tests/test_direct_kv.py:129-189) and the codec tolerances
  (tests/test_codecs.py:33-41).
codec_golden.json: SHA-256 of the oracle's codes, params and restored cache
  bits for small seeded page tensors of every format and cache dtype.  The CPU
  suite checks that the oracle still reproduces them; the GPU suite checks the
  HIP kernels against them.
"""

from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from oracle import codecs as oc  # noqa: E402
from oracle import gen  # noqa: E402

U64 = (1 << 64) - 1
OFF, PRIME = 1469598103934665603, 1099511628211

CASE = dict(n=6, H=4, D=128)
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
FORMATS = ["fp8_e4m3", "fp8_e4m3_ph", "int4_sym_block", "int4_sym", "int4_asym_g32"]


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def tbytes(t: torch.Tensor) -> bytes:
    return t.contiguous().view(torch.uint8).numpy().tobytes()


def pages_for(fmt: str, dtype: torch.dtype) -> torch.Tensor:
    seed = 1000 + FORMATS.index(fmt) * 10 + list(DTYPES.values()).index(dtype)
    g = torch.Generator().manual_seed(seed)
    return gen.kv_values((2, CASE["n"], 16, CASE["H"], CASE["D"]), CASE["D"], g, True, dtype)


def oracle_case(fmt: str, pages: torch.Tensor, dtype: torch.dtype):
    """(codes bytes, params bytes, restored bits) in the blob's byte order."""
    if fmt == "fp8_e4m3":
        codes, scale = oc.fp8_tensor_compress(pages)
        return tbytes(codes), tbytes(oc.fp8_sidecar(scale)), tbytes(
            oc.fp8_tensor_decompress(codes, scale, dtype))
    if fmt == "fp8_e4m3_ph":
        codes, scales = oc.fp8_ph_compress(pages)
        return tbytes(codes), tbytes(scales), tbytes(oc.fp8_ph_decompress(codes, scales, dtype))
    if fmt == "int4_sym_block":
        pk, sc, meta = oc.int4_block_compress(pages)
        return tbytes(pk), tbytes(sc), tbytes(
            oc.int4_block_decompress(pk, sc, tuple(pages.shape), meta, dtype))
    if fmt == "int4_sym":
        pk, sc = oc.int4_channel_compress(pages)
        return tbytes(pk), tbytes(sc), tbytes(
            oc.int4_channel_decompress(pk, sc, tuple(pages.shape), dtype))
    codes, params = oc.int4_asym_compress(pages)
    words = (params & 0xFFFFFFFF).numpy().astype("<u4").tobytes()
    restored = oc.int4_asym_decompress(codes, params, 16, CASE["H"], CASE["D"], dtype)
    return tbytes(codes.to(torch.uint8)), words, tbytes(restored)


def codec_golden() -> dict:
    out = {"case": CASE, "entries": []}
    for fmt in FORMATS:
        for name, dtype in DTYPES.items():
            c, p, r = oracle_case(fmt, pages_for(fmt, dtype), dtype)
            out["entries"].append({"format": fmt, "dtype": name, "codes": sha(c), "params": sha(p),
                                   "restored": sha(r)})
    return out


def reference_vectors() -> dict:
    h123 = (((((OFF ^ 1) * PRIME) & U64 ^ 2) * PRIME) & U64 ^ 3) * PRIME & U64
    hdr = struct.pack("<IIIIIIII QQQ", 0x414D464B, 1, 80, 85000, 4, 256, 0, 0, 1 << 30,
                      0xDEADBEEFCAFEBABE, 0x0102030405060708)
    return {
        "fnv": {"offset": OFF, "prime": PRIME, "tokens_1_2_3": h123,
                "tokens_0": (OFF ^ 0) * PRIME & U64, "tenant_empty": OFF},
        "float_bits": {"0.0": 0, "1.0": 0x3F800000},
        "filename": {
            "args": [0x1234567890ABCDEF, 0xFEDCBA0987654321, 0xABCDEF0123456789, 65536, 1,
                     struct.unpack("<I", struct.pack("<f", 10000.0))[0],
                     struct.unpack("<I", struct.pack("<f", 1.0))[0], 0, 0],
            "expected": "amf_1234567890abcdef_fedcba0987654321_abcdef0123456789_65536_1_"
                        f"{struct.unpack('<I', struct.pack('<f', 10000.0))[0]}_1065353216_"
                        "0000000000000000_0000000000000000"},
        "amfk_header": {"fields": [0x414D464B, 1, 80, 85000, 4, 256, 0, 0, 1 << 30,
                                   0xDEADBEEFCAFEBABE, 0x0102030405060708],
                        "bytes_hex": hdr.hex(), "size": 56, "layer_entry_size": 32},
        "codec_tolerances": {"fp8_e4m3": 0.05, "int4_sym": 0.20, "int4_sym_block": 0.22},
    }


def main() -> None:
    with open(os.path.join(HERE, "codec_golden.json"), "w") as f:
        json.dump(codec_golden(), f, indent=1)
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(reference_vectors(), f, indent=1)


if __name__ == "__main__":
    main()
