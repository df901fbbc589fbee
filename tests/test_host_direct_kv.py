"""amf_direct_kv_* validation on the CPU.

Every rejection of a bad blob or bad arguments happens before the first HIP
call (a restore either copies every layer or writes nothing), so these run
without a device: a context made with max_kv_bytes = 0 allocates nothing,
the device addresses passed are never dereferenced, and each case checks the
status code and message.  The blob cases follow the checks of the
reference's restore (core/amf_direct_kv.cu:331-411) plus the layer-range
check it lacks.  Blobs come from the oracle's AMFK header/table."""

from __future__ import annotations

import ctypes
import struct

import pytest

import amf_hip
from oracle import amfk

U64 = ctypes.c_uint64
FAKE = 0x7F0000000000  # a device address that no test dereferences


@pytest.fixture(scope="module")
def lib():
    return amf_hip.load()


@pytest.fixture()
def ctx(lib):
    h = lib.amf_direct_kv_init(0)
    assert h, lib.amf_last_error()
    yield ctypes.c_void_p(h)
    lib.amf_direct_kv_free(ctypes.c_void_p(h))


def _arr(vals):
    return (U64 * max(1, len(vals)))(*vals)


def _blob(sizes, n_tokens=7, payload=None, **hdr):
    table = amfk.layer_table(sizes)
    total = sum(k + v for k, v in sizes)
    h = amfk.pack_header(len(sizes), n_tokens, hdr.get("heads", 8), hdr.get("dim", 128),
                         hdr.get("dtype", 2), total, 1, 2)
    body = b"".join(struct.pack("<4Q", *e) for e in table)
    return h + body + (bytes(total) if payload is None else payload)


def _restore(lib, ctx, blob, k_bytes, v_bytes, ptrs=None):
    n = len(k_bytes)
    ptrs = [FAKE] * n if ptrs is None else ptrs
    nt = ctypes.c_uint32(99)
    rc = lib.amf_direct_kv_restore(ctx, blob, len(blob), _arr(ptrs), _arr(k_bytes), _arr(ptrs),
                                   _arr(v_bytes), n, ctypes.byref(nt), None)
    return rc, lib.amf_last_error().decode(), nt.value


def test_is_direct_format(lib):
    blob = _blob([(16, 16)])
    assert lib.amf_direct_kv_is_direct_format(blob, len(blob)) == 1
    assert lib.amf_direct_kv_is_direct_format(blob, 55) == 0          # shorter than a header
    assert lib.amf_direct_kv_is_direct_format(b"GGUF" + blob[4:], len(blob)) == 0
    assert lib.amf_direct_kv_is_direct_format(None, 100) == 0


def test_init_without_staging_and_free_null(lib):
    h = lib.amf_direct_kv_init(0)
    assert h
    lib.amf_direct_kv_free(ctypes.c_void_p(h))
    lib.amf_direct_kv_free(None)


@pytest.mark.parametrize("case", ["short", "magic", "version", "layers", "table", "k_size",
                                  "v_size", "k_range", "v_range"])
def test_restore_rejects_before_any_copy(lib, ctx, case):
    sizes = [(64, 64), (64, 64)]
    blob = _blob(sizes)
    kb, vb = [64, 64], [64, 64]
    want = amf_hip.ERR_FORMAT
    if case == "short":
        blob, msg = blob[:55], "too small"
    elif case == "magic":
        blob, msg = b"XXXX" + blob[4:], "magic"
    elif case == "version":
        blob, msg = blob[:4] + struct.pack("<I", 2) + blob[8:], "version"
    elif case == "layers":
        kb, vb, msg, want = [64] * 3, [64] * 3, "layer count", amf_hip.ERR_MISMATCH
    elif case == "table":
        blob, msg = blob[:56 + 40], "truncated"
    elif case == "k_size":
        kb, msg, want = [64, 32], "layer 1 size", amf_hip.ERR_MISMATCH
    elif case == "v_size":
        vb, msg, want = [128, 64], "layer 0 size", amf_hip.ERR_MISMATCH
    elif case == "k_range":
        tab = amfk.layer_table(sizes)
        tab[1] = (10 ** 6, 64, tab[1][2], 64)
        blob = blob[:56] + b"".join(struct.pack("<4Q", *e) for e in tab) + blob[56 + 64:]
        msg = "layer 1 K"
    else:  # a payload cut short: V of the last layer runs past its end
        blob, msg = blob[:-1], "layer 1 V"
    rc, err, nt = _restore(lib, ctx, blob, kb, vb)
    assert rc == want and msg in err, (rc, err)
    assert nt == 99  # nothing reported on failure


def test_restore_skips_layers_the_caller_has_no_kv_for(lib, ctx):
    """A layer the caller has no tensors for (SSM) is not validated
    (core/amf_direct_kv.cu:392-393): layer 0's sizes would not match, but it
    is skipped, so the failure reported is layer 1's."""
    blob = _blob([(64, 64), (64, 64)])
    rc, err, _ = _restore(lib, ctx, blob, [0, 32], [0, 64], ptrs=[0, FAKE])
    assert rc == amf_hip.ERR_MISMATCH and "layer 1" in err


def test_restore_null_arguments(lib):
    blob = _blob([(16, 16)])
    rc = lib.amf_direct_kv_restore(None, blob, len(blob), _arr([FAKE]), _arr([16]), _arr([FAKE]),
                                   _arr([16]), 1, None, None)
    assert rc == amf_hip.ERR_INVALID_ARG


def test_save_argument_errors(lib, ctx):
    out, n = ctypes.c_void_p(), U64()
    toks = (ctypes.c_int32 * 3)(1, 2, 3)
    args = [_arr([FAKE]), _arr([16]), _arr([FAKE]), _arr([16])]

    def save(n_layers=1, dtype=2, tokens=toks, n_tokens=3, bo=ctypes.byref(out)):
        return lib.amf_direct_kv_save(ctx, *args, n_layers, 8, 128, dtype, 0, tokens, n_tokens,
                                      bo, ctypes.byref(n), None)

    assert save(n_layers=0) == amf_hip.ERR_INVALID_ARG            # no attention layers
    assert save(dtype=4) == amf_hip.ERR_INVALID_ARG               # dtype tag past fp8
    assert save(tokens=None) == amf_hip.ERR_INVALID_ARG           # tokens missing
    assert save(n_tokens=-1) == amf_hip.ERR_INVALID_ARG
    assert save(bo=None) == amf_hip.ERR_INVALID_ARG


def _restore_pages(lib, ctx, blob, planes, n_pages, page_bytes=4096, staging=FAKE,
                   staging_bytes=1 << 20, stride=None, pool=64, ids=FAKE):
    nt = ctypes.c_uint32(99)
    rc = lib.amf_direct_kv_restore_pages(ctx, blob, len(blob), _arr(planes),
                                         stride or page_bytes, ids, pool, n_pages, page_bytes,
                                         len(planes) // 2, staging, staging_bytes,
                                         ctypes.byref(nt), None, None)
    return rc, lib.amf_last_error().decode(), nt.value


def test_restore_pages_rejections(lib, ctx):
    pb, n = 4096, 3
    sizes = [(n * pb, n * pb)] * 2
    blob = _blob(sizes)
    planes = [FAKE] * 4
    # one of a layer's two planes missing
    rc, err, _ = _restore_pages(lib, ctx, blob, [FAKE, 0, FAKE, FAKE], n)
    assert rc == amf_hip.ERR_INVALID_ARG and "only one" in err
    # staging smaller than two pages
    rc, err, _ = _restore_pages(lib, ctx, blob, planes, n, staging_bytes=2 * pb - 16)
    assert rc == amf_hip.ERR_WORKSPACE
    rc, err, _ = _restore_pages(lib, ctx, blob, planes, n, staging=FAKE + 8)
    assert rc == amf_hip.ERR_WORKSPACE and "aligned" in err
    # geometry
    rc, _, _ = _restore_pages(lib, ctx, blob, planes, n, page_bytes=4088)
    assert rc == amf_hip.ERR_INVALID_ARG
    rc, _, _ = _restore_pages(lib, ctx, blob, planes, n, stride=2048)
    assert rc == amf_hip.ERR_INVALID_ARG
    rc, _, _ = _restore_pages(lib, ctx, blob, planes, 65, ids=None)   # identity past the pool
    assert rc == amf_hip.ERR_INVALID_ARG
    # page count differs from the snapshot's layer sizes
    rc, err, _ = _restore_pages(lib, ctx, blob, planes, n + 1)
    assert rc == amf_hip.ERR_MISMATCH and "layer 0" in err
    # payload cut short
    rc, err, _ = _restore_pages(lib, ctx, blob[:-pb], planes, n)
    assert rc == amf_hip.ERR_FORMAT and "layer 1 V" in err
    # header problems come before sizes
    rc, err, _ = _restore_pages(lib, ctx, b"XXXX" + blob[4:], planes, n + 1)
    assert rc == amf_hip.ERR_FORMAT and "magic" in err


def test_restore_pages_with_no_pages_reports_tokens_only(lib, ctx):
    """n_pages = 0 (AmfKvManager's empty block table) validates the header and
    the layer count, copies nothing and needs no device."""
    blob = _blob([(0, 0), (0, 0)], n_tokens=1234)
    rc, err, nt = _restore_pages(lib, ctx, blob, [FAKE] * 4, 0, staging=0, staging_bytes=0)
    assert rc == amf_hip.OK and nt == 1234, err
    rc, err, _ = _restore_pages(lib, ctx, blob, [FAKE] * 6, 0, staging=0, staging_bytes=0)
    assert rc == amf_hip.ERR_MISMATCH and "layer count" in err


def test_save_pages_argument_errors(lib, ctx):
    out, nb = ctypes.c_void_p(), U64()
    toks = (ctypes.c_int32 * 1)(5)

    def save(planes, n_pages=2, page_bytes=4096, staging_bytes=1 << 20, staging=FAKE):
        return lib.amf_direct_kv_save_pages(ctx, _arr(planes), page_bytes, FAKE, 64, n_pages,
                                            page_bytes, len(planes) // 2, 16, 64, 2, 0, toks, 1,
                                            staging, staging_bytes, ctypes.byref(out),
                                            ctypes.byref(nb), None, None)

    assert save([FAKE, 0]) == amf_hip.ERR_INVALID_ARG
    assert save([FAKE, FAKE], staging_bytes=4096) == amf_hip.ERR_WORKSPACE
    assert save([FAKE, FAKE], staging=0) == amf_hip.ERR_WORKSPACE
    assert save([FAKE, FAKE], page_bytes=100) == amf_hip.ERR_INVALID_ARG
    assert save([FAKE, FAKE], n_pages=-1) == amf_hip.ERR_INVALID_ARG
