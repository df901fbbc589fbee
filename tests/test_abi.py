"""The C ABI of libamf_hip.so on the CPU: every function include/amf_hip.h
declares is exported and bound by the ctypes layer, the ABI version matches,
the workspace-size queries are consistent, and argument validation returns
the documented status codes with a message (these calls return before any
HIP API call, so no device is needed)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

import amf_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "amf_hip.h")


def header_functions(header: str = HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(amf_\w+)\s*\(", text, flags=re.M))


def header_defines():
    out = {}
    for name, val in re.findall(r"#define\s+(AMF_\w+)\s+\(?(-?\d+)\)?", open(HEADER).read()):
        out[name] = int(val)
    return out


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(amf_hip.LIB_PATH):
        pytest.fail(f"{amf_hip.LIB_PATH} missing: run __graft_entry__.build()")
    return amf_hip.load()


def test_header_declares_the_entry_points():
    fns = header_functions()
    assert {"amf_abi_version", "amf_last_error", "amf_kv_gather_pages", "amf_kv_scatter_pages",
            "amf_fp8_quant_gather", "amf_fp8_dequant_scatter", "amf_int4_quant_gather",
            "amf_int4_dequant_scatter", "amf_int4_paged_decode_attn",
            "amf_int4_decode_workspace_bytes", "amf_quant_workspace_bytes",
            "amf_dense_attn", "amf_dense_attn_workspace_bytes", "amf_int4_sym_dense_attn"} <= fns


def test_every_declared_symbol_is_exported_and_bound(lib):
    fns = header_functions()
    assert fns == set(amf_hip.SIGNATURES), fns ^ set(amf_hip.SIGNATURES)
    raw = ctypes.CDLL(amf_hip.LIB_PATH)
    for f in fns:
        assert hasattr(raw, f), f


def test_selftest_library_exports_its_header():
    """libamf_selftest.so (the encoder checks the GPU tests run) exports what
    include/amf_selftest.h declares, and nothing of it is in the drop-in ABI."""
    path = os.path.join(os.path.dirname(amf_hip.LIB_PATH), "libamf_selftest.so")
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: run __graft_entry__.build()")
    fns = header_functions(os.path.join(ROOT, "include", "amf_selftest.h"))
    assert fns == {"amf_selftest_e4m3_sweep", "amf_selftest_e4m3_encode"}
    assert not fns & header_functions()
    raw = ctypes.CDLL(path)
    for f in fns:
        assert hasattr(raw, f), f


def test_constants_match_header(lib):
    d = header_defines()
    assert lib.amf_abi_version() == d["AMF_ABI_VERSION"] == amf_hip.ABI_VERSION
    for name in ("OK", "DTYPE_F16", "DTYPE_F32", "DTYPE_BF16", "FMT_FP8_E4M3", "FMT_FP8_E4M3_PH",
                 "FMT_INT4_SYM_BLOCK", "FMT_INT4_SYM", "FMT_INT4_ASYM_G32", "DECODE_AUTO",
                 "DECODE_VALU", "DECODE_MFMA", "DECODE_MFMA_PRECISE"):
        assert getattr(amf_hip, name) == d["AMF_" + name], name


def test_workspace_queries(lib):
    d = header_defines()
    assert amf_hip.quant_workspace_bytes(d["AMF_FMT_FP8_E4M3"], 64, 2, 128) == (32 + 32 * 33 * 32) * 4
    assert amf_hip.quant_workspace_bytes(d["AMF_FMT_INT4_SYM"], 4, 4, 128) == 128 * 4
    assert amf_hip.quant_workspace_bytes(d["AMF_FMT_FP8_E4M3_PH"], 64, 1, 128) == 0
    a = amf_hip.decode_workspace_bytes(32, 32, 8, 128, 32768)
    b = amf_hip.decode_workspace_bytes(32, 32, 8, 128, 1024)
    assert a >= b > 0 and a % 16 == 0
    assert amf_hip.decode_workspace_bytes(32, 32, 8, 64, 1024) == 0  # unsupported head_dim


def _rc(lib, fn, *args):
    rc = getattr(lib, fn)(*args)
    return rc, (lib.amf_last_error() or b"").decode()


def _no_device():
    import torch

    return not torch.cuda.is_available()


def test_dense_attn_workspace_bytes(lib):
    """Host-only size query: split partials of (head_dim + 4) fp32 per
    (query row, split); a wave serves up to 4 query heads of a GQA group and
    the splits aim at 2048 waves, one 64-token chunk per split at least; 0
    where the single-pass kernel runs."""
    f = lib.amf_dense_attn_workspace_bytes
    # 128 rows, 4 per wave -> 32 wave rows -> 64 splits of 128 tokens
    assert f(4, 32, 8, 1, 8192, 128) == 128 * 64 * (128 + 4) * 4
    # 32 rows -> 8 wave rows -> 256 splits wanted, 313 chunks -> 157 splits of 128 tokens
    assert f(1, 32, 8, 1, 20000, 128) == 32 * 157 * 132 * 4
    assert f(1, 2, 2, 1, 1, 256) == 2 * 1 * 260 * 4
    # GQA 3: one head per wave; 24 wave rows -> 86 splits wanted, 79 chunks -> 79 splits
    assert f(2, 12, 4, 1, 5000, 64) == 24 * 79 * 68 * 4
    assert f(64, 64, 8, 1, 100, 64) == 4096 * 2 * 68 * 4
    assert f(4, 32, 8, 1, 8192, 80) == 0 and f(4, 32, 8, 1, 0, 128) == 0
    assert f(0, 32, 8, 1, 8192, 128) == 0 and f(1 << 40, 32, 8, 1, 64, 128) == 0
    assert f(4, 32, 7, 1, 8192, 128) == 0  # heads not a multiple: no split path


# Fake addresses below are never dereferenced because every call fails
# validation first; the guard keeps these calls off a machine with a device
# all the same.
@pytest.mark.skipif(not _no_device(), reason="argument-validation calls run on the CPU only")
def test_validation_errors(lib):
    d = header_defines()
    inv, uns, wsp = d["AMF_ERR_INVALID_ARG"], d["AMF_ERR_UNSUPPORTED"], d["AMF_ERR_WORKSPACE"]
    rc, msg = _rc(lib, "amf_kv_gather_pages", None, 4096, None, 8, None, 4096, 2, 1, 4096, None,
                  None)
    assert rc == inv and "null" in msg
    fake = 1 << 20  # never dereferenced: validation fails first
    rc, msg = _rc(lib, "amf_kv_gather_pages", fake, 4096, None, 8, fake, 4096, 2, 1, 4001, None,
                  None)
    assert rc == inv and "multiples of 16" in msg
    rc, msg = _rc(lib, "amf_fp8_dequant_scatter", d["AMF_FMT_FP8_E4M3"], fake, fake, fake, 32768,
                  7, None, 8, 2, 1, 16, 8, 128, None, None)
    assert rc == uns and "dtype" in msg
    rc, msg = _rc(lib, "amf_int4_dequant_scatter", 99, fake, fake, fake, 32768, 2, None, 8, 2, 1,
                  16, 8, 128, None, None)
    assert rc == inv and "INT4" in msg
    rc, msg = _rc(lib, "amf_int4_paged_decode_attn", fake, 2, fake, 2, fake, fake, fake, fake, 8,
                  fake, 4, fake, 1, 32, 8, 64, 16, 64, 0.0, fake, 1 << 20, 0, None, None)
    assert rc == uns and "head_dim" in msg
    rc, msg = _rc(lib, "amf_int4_paged_decode_attn", fake, 2, fake, 2, fake, fake, fake, fake, 8,
                  fake, 4, fake, 1, 24, 8, 128, 16, 64, 0.0, fake, 1 << 20, 0, None, None)
    assert rc == uns and "GQA" in msg
    rc, msg = _rc(lib, "amf_int4_paged_decode_attn", fake, 2, fake, 2, fake, fake, fake, fake, 8,
                  fake, 4, fake, 1, 32, 8, 128, 16, 64, 0.0, None, 0, 0, None, None)
    assert rc == wsp and "workspace" in msg
    rc, msg = _rc(lib, "amf_dense_attn", fake, fake, fake, 2, None, 0, 0, 0, 0, fake, 2, 1, 8, 3,
                  1, 10, 64, 0.0, None, 0, None)
    assert rc == inv and "multiple" in msg
    rc, msg = _rc(lib, "amf_dense_attn", fake, fake, fake, 2, None, 0, 0, 0, 0, fake, 2, 1, 8, 8,
                  1, 10, 512, 0.0, None, 0, None)
    assert rc == uns and "head_dim" in msg
    # INT4_SYM attention: head dims of the split kernel only, and a workspace
    rc, msg = _rc(lib, "amf_int4_sym_dense_attn", fake, 2, fake, fake, fake, fake, None, 0, 0, 0,
                  0, fake, 2, 1, 8, 8, 1, 10, 80, 0.0, None, 0, None)
    assert rc == uns and "head_dim" in msg
    rc, msg = _rc(lib, "amf_int4_sym_dense_attn", fake, 2, fake, fake, fake, fake, None, 0, 0, 0,
                  0, fake, 2, 1, 8, 8, 1, 10, 128, 0.0, None, 0, None)
    assert rc == wsp and "workspace" in msg
    rc, msg = _rc(lib, "amf_int4_sym_dense_attn", fake, 2, fake + 2, fake, fake, fake, None, 0, 0,
                  0, 0, fake, 2, 1, 8, 8, 1, 10, 128, 0.0, fake, 1 << 20, None)
    assert rc == inv and "aligned" in msg


@pytest.mark.skipif(not _no_device(), reason="argument-validation calls run on the CPU only")
def test_python_errors_name_the_call(lib):
    with pytest.raises(amf_hip.AmfHipError) as ei:
        amf_hip.call("amf_kv_scatter_pages", None, 16, None, 16, None, 8, 1, 1, 16, None, None)
    assert ei.value.code == amf_hip.ERR_INVALID_ARG and "amf_kv_scatter_pages" in str(ei.value)
