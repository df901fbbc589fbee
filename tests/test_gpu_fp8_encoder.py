"""The e4m3 encoder the FP8 save kernels inline (gfx950's v_cvt_pk_fp8_f32),
checked through libamf_selftest.so:

* against the portable bit-level encoder on every fp32 value the kernels can
  hand it (|x| <= 448, both signs: the kernels clamp each quotient first, as
  amf_codec.py:191 clamps before its float8_e4m3fn cast), on the device;
* against the oracle's table-search encoder (itself pinned against torch's
  float8_e4m3fn cast) on whole binades, every tie point and a random sample.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import e4m3

import amf_hip

LIB = os.path.join(os.path.dirname(amf_hip.LIB_PATH), "libamf_selftest.so")
MAX_REPORT = 8

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    so = ctypes.CDLL(LIB)
    so.amf_selftest_e4m3_sweep.restype = ctypes.c_int
    so.amf_selftest_e4m3_sweep.argtypes = [ctypes.POINTER(ctypes.c_ulonglong),
                                           ctypes.POINTER(ctypes.c_uint32)]
    so.amf_selftest_e4m3_encode.restype = ctypes.c_int
    so.amf_selftest_e4m3_encode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.c_void_p]
    torch.cuda.init()
    return so


def test_kernel_encoder_equals_portable_encoder_on_every_input(lib):
    bad = ctypes.c_ulonglong(0)
    first = (ctypes.c_uint32 * (3 * MAX_REPORT))()
    rc = lib.amf_selftest_e4m3_sweep(ctypes.byref(bad), first)
    assert rc == 0
    report = [tuple(hex(first[3 * k + i]) for i in range(3))
              for k in range(min(bad.value, MAX_REPORT))]
    assert bad.value == 0, report


def _encode(lib, x: np.ndarray) -> np.ndarray:
    xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    out = torch.empty(xd.numel(), dtype=torch.uint8, device="cuda")
    rc = lib.amf_selftest_e4m3_encode(xd.data_ptr(), out.data_ptr(), xd.numel(),
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _binade(lo_bits: int, hi_bits: int) -> np.ndarray:
    return np.arange(lo_bits, hi_bits, dtype=np.uint32).view(np.float32)


def test_kernel_encoder_matches_oracle(lib):
    pos = e4m3.code_values()[:0x7F]
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    near = [mids]
    for k in (1, 2, 3):
        lo, hi = mids.copy(), mids.copy()
        for _ in range(k):
            lo, hi = np.nextafter(lo, np.float32(0)), np.nextafter(hi, np.float32(1000))
        near += [lo, hi]
    codes = pos.astype(np.float32)
    rng = np.random.default_rng(11)
    sample = rng.integers(0, 0x43E00001, size=1_000_000, dtype=np.uint32).view(np.float32)
    small = np.concatenate([*near, codes, sample,
                            np.array([0.0, 448.0, 1e-30, 1e-45], dtype=np.float32)])
    x = np.concatenate([
        small, -small,
        _binade(0x3C000000, 0x3C800000),   # [2^-7, 2^-6): the subnormal codes' top binade
        _binade(0x3A800000, 0x3B000000),   # [2^-10, 2^-9): rounds to 0 or the smallest code
        _binade(0x43800000, 0x43E00001),   # [256, 448]
    ])
    got = _encode(lib, x)
    want = e4m3.encode(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_encode_edge_lengths(lib):
    assert lib.amf_selftest_e4m3_encode(None, None, 0, None) == 0
    assert lib.amf_selftest_e4m3_encode(None, None, -1, None) == -1
    for n in (1, 3, 4, 5, 1023):
        x = np.linspace(-448, 448, n, dtype=np.float32)
        assert np.array_equal(_encode(lib, x), e4m3.encode(x))
