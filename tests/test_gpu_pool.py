"""CompressedVRAMPool, AmfKvManager and AmfWorkerExtension on the GPU.

Mirrors the reference's pool tests (tests/test_pool.py, tests/
test_fp8_restore.py:80-97) on a HIP device, and checks put_from_vllm ->
restore_to_vllm bit for bit against the oracle for every pool format, AMFK
files byte for byte against the oracle's header/table and page gather, and
stream-ordered reuse of freed slab spans."""

from __future__ import annotations

import os
import time

import numpy as np
import pytest
import torch

from oracle import amfk
from oracle import codecs as oc
from oracle import gen

from helpers import bits, sentinel_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _pool(**kw):
    from korith_vllm_ext.compressed_vram_pool import CompressedVRAMPool

    args = dict(num_layers=4, bytes_per_layer=1 << 18, block_bytes=1 << 13,
                default_format="int4_sym_block", device="cuda")
    args.update(kw)
    return CompressedVRAMPool(**args)


def _fake_kv(layers, tokens, heads=4, head_dim=64):
    return torch.randn(layers, 2, tokens, heads, head_dim, device=DEV)


# -------------------------------------------- tests/test_pool.py on the GPU --


def test_pool_insert_get_delete():
    p = _pool()
    assert p.put_from_raw("abc", _fake_kv(4, 64)) is True
    assert "abc" in p and len(p) == 1
    e = p.get("abc")
    assert e.num_tokens == 64 and e.format == "int4_sym_block"
    assert p.delete("abc") is True and p.get("abc") is None and p.delete("abc") is False


def test_pool_eviction_under_pressure():
    p = _pool()
    for i in range(32):
        p.put_from_raw(f"p{i:02d}", _fake_kv(4, 64))
        time.sleep(0.0005)
    assert p.stats()["evictions"] > 0
    assert p.used_bytes() <= p.capacity_bytes()


def test_pool_reuse_score_protects_valuable_entries():
    p = _pool()
    p.put_from_raw("hot", _fake_kv(4, 32), savings_ms=500.0)
    for _ in range(10):
        p.get("hot")
    cold = _fake_kv(4, 32)
    for i in range(20):
        p.put_from_raw(f"cold{i}", cold, savings_ms=0.0)
    assert "hot" in p


def test_pool_restore_to_tensor_roundtrip():
    p = _pool()
    kv = _fake_kv(4, 64)
    p.put_from_raw("a", kv)
    r = p.restore_to_tensor("a", target_dtype=torch.float32)
    assert r.shape == kv.shape
    assert (r - kv).norm().item() / kv.norm().item() < 0.30
    assert p.restore_to_tensor("missing") is None


def test_pool_stats_map_and_errors():
    from korith_vllm_ext.compressed_vram_pool import _ExternalBlockRef

    p = _pool()
    p.put_from_raw("a", _fake_kv(4, 32))
    p.get("a")
    p.get("not_here")
    s = p.stats()
    assert s["hits"] >= 1 and s["misses"] >= 1 and s["inserts"] == 1
    table = {42: [None] * 4}
    assert p.map_into_vllm("a", 42, table)
    assert all(isinstance(r, _ExternalBlockRef) and r.is_external for r in table[42])
    with pytest.raises(ValueError):
        p.put_from_raw("bad", torch.randn(2, 3, device=DEV))
    tiny = _pool(num_layers=1, bytes_per_layer=1024, block_bytes=1024)
    assert tiny.put_from_raw("huge", torch.randn(1, 2, 1024, 8, 128, device=DEV)) is False


def test_pool_fp8_sidecar_per_layer():
    """tests/test_fp8_restore.py:80-97, plus the Python-double tensor_scale
    of every layer equal to the codec's."""
    from korith_vllm_ext.codecs import FP8ScaleSidecar

    p = _pool(num_layers=2, default_format="fp8_e4m3")
    kv = torch.randn(2, 2, 64, 4, 64, device=DEV)
    assert p.put_from_raw("p", kv, format="fp8_e4m3")
    e = p.get("p")
    assert len(e.blobs) == 2
    for l, blob in enumerate(e.blobs):
        sc = blob.meta["sidecar"]
        assert isinstance(sc, FP8ScaleSidecar) and sc.k_scale > 0
        _, want = oc.fp8_tensor_compress(kv[l].cpu())
        assert blob.tensor_scale == want == e.blocks[l].tensor_scale


# ------------------------------------------------- vLLM paths, bit-exact --

FORMATS = ["int4_sym_block", "fp8_e4m3", "fp8_e4m3_ph", "int4_sym", "int4_asym_g32"]


def _want_pages(fmt, pages, dtype):
    """Oracle restore of one layer's gathered pages [2, n, bs, H, D]."""
    if fmt == "int4_sym_block":
        pk, sc, meta = oc.int4_block_compress(pages)
        return oc.int4_block_decompress(pk, sc, tuple(pages.shape), meta, dtype)
    if fmt == "fp8_e4m3":
        c, s = oc.fp8_tensor_compress(pages)
        return oc.fp8_tensor_decompress(c, s, dtype)
    if fmt == "fp8_e4m3_ph":
        c, s = oc.fp8_ph_compress(pages)
        return oc.fp8_ph_decompress(c, s, dtype)
    if fmt == "int4_sym":
        pk, sc = oc.int4_channel_compress(pages)
        return oc.int4_channel_decompress(pk, sc, tuple(pages.shape), dtype)
    c, pr = oc.int4_asym_compress(pages)
    return oc.int4_asym_decompress(c, pr, pages.shape[2], pages.shape[3], pages.shape[4], dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", FORMATS)
def test_vllm_roundtrip_bitexact(fmt, dtype):
    L, pool_pages, n, H, D = 3, 48, 20, 8, 128
    g = torch.Generator().manual_seed(FORMATS.index(fmt))
    values = gen.kv_values((L, 2, pool_pages, 16, H, D), D, g, True, dtype)
    cache = [values[l].to(DEV) for l in range(L)]
    src = gen.block_table(pool_pages, n, 1).tolist()
    dst = gen.block_table(pool_pages, n, 2).tolist()
    p = _pool(num_layers=L, bytes_per_layer=8 << 20, block_bytes=1 << 16, default_format=fmt)
    assert p.put_from_vllm("k", cache, src, n * 16 - 5)
    target = sentinel_cache(L, pool_pages, 16, H, D, dtype, DEV)
    assert p.restore_to_vllm("k", target, dst) == n * 16 - 5
    torch.cuda.synchronize()
    for l in range(L):
        want = sentinel_cache(1, pool_pages, 16, H, D, dtype, "cpu")[0]
        want[:, torch.tensor(dst)] = _want_pages(fmt, values[l][:, torch.tensor(src)], dtype)
        assert np.array_equal(bits(target[l]), bits(want)), (fmt, l)
    # restore_to_tensor of a vLLM entry: [L, 2, n, bs, H, D]
    r = p.restore_to_tensor("k", target_dtype=dtype)
    assert r.shape == (L, 2, n, 16, H, D)
    assert np.array_equal(bits(r[1]), bits(_want_pages(fmt, values[1][:, torch.tensor(src)],
                                                       dtype)))
    # partial restore: a shorter block table and fewer layers
    target2 = sentinel_cache(2, pool_pages, 16, H, D, dtype, DEV)
    assert p.restore_to_vllm("k", target2, dst[:7]) == n * 16 - 5
    torch.cuda.synchronize()
    want = sentinel_cache(1, pool_pages, 16, H, D, dtype, "cpu")[0]
    want[:, torch.tensor(dst[:7])] = _want_pages(fmt, values[1][:, torch.tensor(src)],
                                                 dtype)[:, :7]
    assert np.array_equal(bits(target2[1]), bits(want))
    assert p.restore_to_vllm("nope", target, dst) == 0


def test_failed_per_tensor_fp8_save_is_a_miss():
    """A per-tensor FP8 save whose layer absmax comes back non-finite (what
    the single-read kernel writes for a scale group whose wait gave up) is
    dropped on first lookup: get() misses, restore_to_vllm restores nothing
    and returns 0, and the entry's spans are free again."""
    L, pool_pages, n, H, D = 2, 32, 8, 2, 64
    g = torch.Generator().manual_seed(17)
    cache = [gen.kv_values((2, pool_pages, 16, H, D), D, g, True).to(DEV) for _ in range(L)]
    p = _pool(num_layers=L, bytes_per_layer=1 << 20, block_bytes=1 << 12,
              default_format="fp8_e4m3")
    assert p.put_from_vllm("bad", cache, list(range(n)), n * 16)
    host, ev = p._index["bad"].pending_absmax
    ev.synchronize()
    host.view(torch.float32)[1] = float("inf")   # layer 1's save "gave up"
    target = sentinel_cache(L, pool_pages, 16, H, D, torch.bfloat16, DEV)
    before = p.stats()["misses"]
    assert p.restore_to_vllm("bad", target, list(range(n))) == 0
    assert p.get("bad") is None and "bad" not in p
    assert p.stats()["misses"] == before + 2
    assert all(a.free_blocks() == a.n_blocks for a in p._alloc)
    torch.cuda.synchronize()
    assert all(bool((t == -7.25).all()) for t in target)
    # a good save of the same key afterwards is a normal hit
    assert p.put_from_vllm("bad", cache, list(range(n)), n * 16)
    assert p.restore_to_vllm("bad", target, list(range(n))) == n * 16


def test_vllm_one_byte_cache_is_stored_raw():
    L, pool_pages, n = 2, 16, 6
    cache = [torch.randint(0, 256, (2, pool_pages, 16, 2, 64), dtype=torch.uint8, device=DEV)
             .view(torch.float8_e4m3fn) for _ in range(L)]
    p = _pool(num_layers=L, bytes_per_layer=1 << 20, block_bytes=1 << 12)
    assert p.put_from_vllm("r", cache, list(range(3, 3 + n)), n * 16)
    assert p.get("r").format == "raw"
    target = [torch.zeros_like(c) for c in cache]
    assert p.restore_to_vllm("r", target, list(range(n))) == n * 16
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(target[l][:, :n].view(torch.uint8),
                           cache[l][:, 3:3 + n].view(torch.uint8))


def test_4d_cache_layers_and_geometry_check():
    g = torch.Generator().manual_seed(3)
    cache = [gen.kv_values((12, 16, 2, 64), 64, g, False).to(DEV) for _ in range(2)]
    p = _pool(num_layers=2, bytes_per_layer=1 << 20, block_bytes=1 << 12,
              default_format="fp8_e4m3_ph")
    assert p.put_from_vllm("x", cache, [1, 5, 7], 48)
    target = [torch.zeros_like(c) for c in cache]
    assert p.restore_to_vllm("x", target, [0, 2, 4]) == 48
    torch.cuda.synchronize()
    pages = torch.stack([cache[0].cpu()[[1, 5, 7]]] * 2)
    want = oc.fp8_ph_decompress(*oc.fp8_ph_compress(pages), torch.bfloat16)
    assert torch.equal(target[0].cpu()[[0, 2, 4]], want[0])
    with pytest.raises(ValueError):
        p.restore_to_vllm("x", [torch.zeros(12, 16, 4, 64, dtype=torch.bfloat16, device=DEV)],
                          [0])
    with pytest.raises(ValueError):
        p.put_from_vllm("y", cache, [0, 12], 32)  # block id outside the cache


def test_freed_span_reuse_waits_for_side_stream_restore():
    """A restore enqueued on a side stream still reads a span when its entry is
    deleted and the span is re-filled from the default stream: the refill waits
    for the restore's event, so the restore sees the old data."""
    L, pool_pages, n, H, D = 2, 4096, 2048, 8, 128
    g = torch.Generator(device="cuda").manual_seed(9)
    a = [torch.randn(2, pool_pages, 16, H, D, generator=g, device=DEV).to(torch.bfloat16)
         for _ in range(L)]
    b = [torch.randn(2, pool_pages, 16, H, D, generator=g, device=DEV).to(torch.bfloat16)
         for _ in range(L)]
    p = _pool(num_layers=L, bytes_per_layer=160 << 20, block_bytes=1 << 20,
              default_format="fp8_e4m3_ph")
    ids = list(range(n))
    assert p.put_from_vllm("a", a, ids, n * 16)
    torch.cuda.synchronize()
    target = [torch.zeros_like(t) for t in a]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(4):
            p.restore_to_vllm("a", target, ids)
    p.delete("a")
    assert p.put_from_vllm("b", b, ids, n * 16)     # same span, default stream
    torch.cuda.synchronize()
    ref = [torch.zeros_like(t) for t in a]
    q = _pool(num_layers=L, bytes_per_layer=160 << 20, block_bytes=1 << 20,
              default_format="fp8_e4m3_ph")
    q.put_from_vllm("a", a, ids, n * 16)
    q.restore_to_vllm("a", ref, ids)
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(target[l], ref[l])


def test_compaction_keeps_entries_restorable():
    p = _pool(num_layers=2, bytes_per_layer=1 << 20, block_bytes=1 << 13,
              default_format="int4_asym_g32")
    g = torch.Generator().manual_seed(4)
    vals = {k: gen.kv_values((2, 2, 8, 16, 2, 64), 64, g, True) for k in "abc"}
    for k, v in vals.items():
        assert p.put_from_vllm(k, [v[l].to(DEV) for l in range(2)], list(range(8)), 128)
    p.delete("a")
    before = {k: p.restore_to_tensor(k, torch.bfloat16) for k in "bc"}
    p._compact_slabs()
    assert p._alloc[0].runs()[0][0] == sum(b.span_blocks for e in p._index.values()
                                           for b in e.blocks if b.layer_id == 0)
    for k in "bc":
        after = p.restore_to_tensor(k, torch.bfloat16)
        assert torch.equal(after, before[k])


def test_entry_blob_views_follow_their_spans():
    """entry.blobs are built on first access: views made before a compaction
    are re-cut to the moved spans, views made after it start at the new
    offsets, and every view decodes to what restore_to_tensor returns."""
    from korith_vllm_ext.codecs import FP8ScaleSidecar, get_codec

    p = _pool(num_layers=2, bytes_per_layer=1 << 20, block_bytes=1 << 13,
              default_format="fp8_e4m3")
    g = torch.Generator().manual_seed(6)
    vals = {k: gen.kv_values((2, 2, 8, 16, 2, 64), 64, g, True) for k in "abc"}
    for k, v in vals.items():
        assert p.put_from_vllm(k, [v[l].to(DEV) for l in range(2)], list(range(8)), 128)
    e_b = p._index["b"]
    assert e_b.blobs[0].tensor_scale == 0.0            # built before its scale resolved
    p.delete("a")
    p._compact_slabs()
    codec = get_codec("fp8_e4m3")
    for k in "bc":
        e = p.get(k)                                    # resolves the per-tensor scales
        want = p.restore_to_tensor(k, torch.bfloat16)
        for l in range(2):
            blk, blob = e.blocks[l], e.blobs[l]
            assert blob.data.data_ptr() == p._slabs[l].data_ptr() + blk.data_offset
            assert blob.tensor_scale == blk.tensor_scale > 0
            assert isinstance(blob.meta["sidecar"], FP8ScaleSidecar)
            assert blob.meta is blk.meta
            assert torch.equal(codec.decompress_to(blob, torch.bfloat16), want[l])
    assert len(e.blobs) == 2 and e.blobs[-1] is e.blobs[1]
    assert [b.data.data_ptr() for b in e.blobs[0:2]] == [b.data.data_ptr() for b in e.blobs]
    with pytest.raises(IndexError):
        e.blobs[2]


# ------------------------------------------------------------- AMFK files --


class _Engine:
    def __init__(self, caches):
        self.gpu_cache = caches


class _Cfg:
    max_model_len = 8192


def test_amfk_save_restore_bytes_and_pages(tmp_path):
    from korith_vllm_ext.amf_kv_manager import AmfKvManager

    L, pool_pages, n, H, D = 3, 40, 9, 2, 64
    g = torch.Generator().manual_seed(6)
    values = gen.kv_values((L, 2, pool_pages, 16, H, D), D, g, False)
    cache = [values[l].to(DEV) for l in range(L)]
    mgr = AmfKvManager(_Engine(cache), str(tmp_path), _Cfg(), model_hash=0xABC,
                       tenant_id="t1")
    toks = list(range(100, 100 + n * 16 - 3))
    src = gen.block_table(pool_pages, n, 3).tolist()
    assert mgr.save_kv_state(toks, src)
    key = mgr.compute_amf_key(toks)
    data = mgr._kv_filename(key).read_bytes()
    plane = n * 16 * H * D * 2
    hdr = amfk.pack_header(L, len(toks), 16, D, 2, 2 * L * plane, 0xABC, amfk.hash_tokens(toks))
    tab = b"".join(np.array(e, dtype="<u8").tobytes()
                   for e in amfk.layer_table([(plane, plane)] * L))
    payload = b"".join(values[l][kv][torch.tensor(src)].contiguous().view(torch.uint8)
                       .numpy().tobytes() for l in range(L) for kv in range(2))
    assert data == hdr + tab + payload
    assert mgr._tok_filename(key).read_bytes() == np.asarray(toks, "<i4").tobytes()
    # restore into another cache at other pages
    target = sentinel_cache(L, pool_pages, 16, H, D, torch.bfloat16, DEV)
    mgr2 = AmfKvManager(_Engine(target), str(tmp_path), _Cfg(), model_hash=0xABC,
                        tenant_id="t1")
    dst = gen.block_table(pool_pages, n, 4).tolist()
    assert mgr2.restore_kv_state(toks, dst) == len(toks)
    for l in range(L):
        want = sentinel_cache(1, pool_pages, 16, H, D, torch.bfloat16, "cpu")[0]
        want[:, torch.tensor(dst)] = values[l][:, torch.tensor(src)]
        assert torch.equal(target[l].cpu(), want)
    with pytest.raises(ValueError):
        mgr2.restore_kv_state(toks, dst[:4])        # page count differs from the file
    assert mgr2.stats()["hits"] == 1


# ------------------------------------------------------- worker extension --


class _Runner:
    def __init__(self, caches):
        self.kv_caches = caches
        self.model_config = _Cfg()


class _Worker:
    def __init__(self, caches):
        self.model_runner = _Runner(caches)


@pytest.mark.parametrize("mode", ["pool_fp8", "pool_int4", "raw", "disk"])
def test_worker_extension_roundtrip(mode, tmp_path, monkeypatch):
    from korith_vllm_ext.amf_worker_ext import AmfWorkerExtension

    for k in ("KORITH_VRAM_POOL_GB", "KORITH_VRAM_CACHE_GB", "KORITH_VRAM_POOL_QUANT"):
        monkeypatch.delenv(k, raising=False)
    if mode.startswith("pool"):
        monkeypatch.setenv("KORITH_VRAM_POOL_GB", "0.25")
        monkeypatch.setenv("KORITH_VRAM_POOL_QUANT", mode[5:])
    elif mode == "raw":
        monkeypatch.setenv("KORITH_VRAM_CACHE_GB", "0.25")
    else:
        monkeypatch.setenv("KORITH_AMF_PATH", str(tmp_path))

    class Worker(_Worker, AmfWorkerExtension):
        pass

    g = torch.Generator().manual_seed(8)
    values = gen.kv_values((2, 2, 32, 16, 2, 128), 128, g, True)
    caches = [values[l].to(DEV) for l in range(2)]
    w = Worker(caches)
    toks = list(range(5, 5 + 80))
    assert w.amf_save_kv(toks, [3, 4, 9, 10, 11], len(toks)) is True
    for c in caches:
        c.fill_(0.0)
    assert w.amf_restore_kv(toks, [20, 21, 22, 23, 24]) == len(toks)
    assert w.amf_restore_kv([1, 2], [0]) == 0
    torch.cuda.synchronize()
    got = caches[1][:, 20:25].cpu()
    src = values[1][:, [3, 4, 9, 10, 11]]
    if mode in ("raw", "disk"):
        assert torch.equal(got, src)
    else:
        fmt = {"pool_fp8": "fp8_e4m3_ph", "pool_int4": "int4_sym_block"}[mode]
        assert torch.equal(got, _want_pages(fmt, src, torch.bfloat16))
    assert isinstance(w.amf_kv_stats(), dict)
