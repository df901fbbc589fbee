"""amf_direct_kv_* on the GPU: AMFK blobs byte-exact against the oracle.

Contiguous form (core/amf_direct_kv.cu:158-462 over caller tensors): the
saved blob is the oracle's header + layer table + each layer's K and V
bytes, a layer without KV is recorded as {total, 0, total, 0}, and a restore
puts every byte back.  Paged form (the AMFK manager's path): the blob's
payload is the oracle's page gather of every plane, and a restore through
the two-slot staging ring writes exactly the oracle's scatter, leaving every
other page untouched.  Staging sizes are chosen to force one chunk, many
chunks, chunks that end inside a plane, and more than the 64 segments a
launch carries."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import amf_hip
from oracle import amfk
from oracle import gen

from helpers import sentinel_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _ctx():
    from korith_vllm_ext.amf_direct_kv import AmfDirectKv

    return AmfDirectKv(0)


def _table_bytes(sizes):
    return b"".join(np.array(e, dtype="<u8").tobytes() for e in amfk.layer_table(sizes))


def _raw(t: torch.Tensor) -> bytes:
    return t.contiguous().view(torch.uint8).cpu().numpy().tobytes()


def test_contiguous_save_restore_bytes():
    g = torch.Generator().manual_seed(21)
    shapes = [(33, 4, 64), None, (33, 4, 64), (7, 2, 128)]  # layer 1 has no KV (SSM)
    k = [None if s is None else torch.randn(*s, generator=g).to(torch.bfloat16).to(DEV)
         for s in shapes]
    v = [None if s is None else torch.randn(*s, generator=g).to(torch.bfloat16).to(DEV)
         for s in shapes]
    toks = list(range(40, 73))
    ctx = _ctx()
    blob = bytes(ctx.save(k, v, tokens=toks, n_kv_heads=4, head_dim=64,
                          dtype_tag=amf_hip.DTYPE_BF16, model_hash=0xFEED))
    sizes = [(0, 0) if t is None else (t.numel() * 2, t.numel() * 2) for t in k]
    total = sum(a + b for a, b in sizes)
    want = (amfk.pack_header(4, len(toks), 4, 64, 2, total, 0xFEED, amfk.hash_tokens(toks)) +
            _table_bytes(sizes) +
            b"".join(_raw(t) for kv in zip(k, v) for t in kv if t is not None))
    assert blob == want
    assert ctx.is_direct_format(blob)
    # restore from a host copy (outside the staging buffer) and from staging
    for source in ("bytes", "staging"):
        k2 = [None if t is None else torch.zeros_like(t) for t in k]
        v2 = [None if t is None else torch.zeros_like(t) for t in v]
        if source == "bytes":
            n = ctx.restore(blob, k2, v2)
        else:
            buf = ctx.staging(len(blob))
            buf[:] = blob
            n = ctx.restore(buf, k2, v2)
        torch.cuda.synchronize()
        assert n == len(toks)
        for a, b in zip(k + v, k2 + v2):
            if a is not None:
                assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # a mismatched restore writes nothing
    k3 = [None if t is None else torch.zeros_like(t) for t in k]
    k3[3] = torch.zeros(6, 2, 128, dtype=torch.bfloat16, device=DEV)
    v3 = [None if t is None else torch.zeros_like(t) for t in v]
    with pytest.raises(amf_hip.AmfHipError) as ei:
        ctx.restore(blob, k3, v3)
    assert ei.value.code == amf_hip.ERR_MISMATCH
    torch.cuda.synchronize()
    assert all(t is None or not t.any() for t in k3 + v3)
    ctx.close()


def _paged_case(L, pool, n, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    values = gen.kv_values((L, 2, pool, 16, H, D), D, g, True)
    return values, gen.block_table(pool, n, seed + 1), gen.block_table(pool, n, seed + 2)


@pytest.mark.parametrize("L,pool,n,H,D,slot_pages", [
    (3, 40, 9, 2, 64, 1000),   # one chunk
    (3, 40, 9, 2, 64, 4),      # chunks that end inside planes
    (2, 64, 64, 8, 128, 7),    # 32 KiB pages, odd slot
    (40, 12, 2, 2, 64, 200),   # 80 planes of 2 pages: more than 64 segments per chunk
])
def test_paged_save_restore_match_oracle(L, pool, n, H, D, slot_pages):
    from korith_vllm_ext import _paged

    values, src, dst = _paged_case(L, pool, n, H, D, 31 + L + slot_pages)
    cache = [values[l].to(DEV) for l in range(L)]
    view = _paged.cache_view(cache)
    pb = view.page_bytes
    staging = torch.empty(2 * slot_pages * pb, dtype=torch.uint8, device=DEV)
    toks = list(range(n * 16 - 5))
    ctx = _ctx()
    print(f"paged L={L} pool={pool} n={n} H={H} D={D} slot_pages={slot_pages}", flush=True)
    blob = bytes(ctx.save_pages(view, src.to(DEV), n, staging, tokens=toks, n_kv_heads=16,
                                head_dim=D, dtype_tag=2, model_hash=7))
    plane = n * pb
    want = (amfk.pack_header(L, len(toks), 16, D, 2, 2 * L * plane, 7, amfk.hash_tokens(toks)) +
            _table_bytes([(plane, plane)] * L) +
            b"".join(_raw(values[l][kv][src.long()]) for l in range(L) for kv in range(2)))
    assert blob == want
    target = sentinel_cache(L, pool, 16, H, D, torch.bfloat16, DEV)
    tview = _paged.cache_view(target)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert ctx.restore_pages(blob, tview, dst.to(DEV), n, staging, err) == len(toks)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    for l in range(L):
        want_l = sentinel_cache(1, pool, 16, H, D, torch.bfloat16, "cpu")[0]
        want_l[:, dst.long()] = values[l][:, src.long()]
        assert torch.equal(target[l].cpu().view(torch.int16), want_l.view(torch.int16)), l
    ctx.close()


def test_paged_restore_back_to_back_reuses_staging():
    """Two restores in a row through one context and one staging ring (the
    second's H2D must wait for the first's scatter of the same slot), then a
    save: each result is the oracle's."""
    from korith_vllm_ext import _paged

    L, pool, n, H, D = 4, 48, 20, 2, 64
    values, src, dst = _paged_case(L, pool, n, H, D, 77)
    cache = [values[l].to(DEV) for l in range(L)]
    view = _paged.cache_view(cache)
    staging = torch.empty(2 * 3 * view.page_bytes, dtype=torch.uint8, device=DEV)
    ctx = _ctx()
    blob1 = bytes(ctx.save_pages(view, src.to(DEV), n, staging, tokens=[1, 2], n_kv_heads=16,
                                 head_dim=D, dtype_tag=2))
    blob2 = bytes(ctx.save_pages(view, dst.to(DEV), n, staging, tokens=[3], n_kv_heads=16,
                                 head_dim=D, dtype_tag=2))
    target = sentinel_cache(L, pool, 16, H, D, torch.bfloat16, DEV)
    tview = _paged.cache_view(target)
    ids_a = gen.block_table(pool, n, 5)
    ids_b = gen.block_table(pool, n, 6)
    assert ctx.restore_pages(blob1, tview, ids_a.to(DEV), n, staging) == 2
    assert ctx.restore_pages(blob2, tview, ids_b.to(DEV), n, staging) == 1
    torch.cuda.synchronize()
    for l in range(L):
        want = sentinel_cache(1, pool, 16, H, D, torch.bfloat16, "cpu")[0]
        want[:, ids_a.long()] = values[l][:, src.long()]
        want[:, ids_b.long()] = values[l][:, dst.long()]
        assert torch.equal(target[l].cpu().view(torch.int16), want.view(torch.int16)), l
    ctx.close()
