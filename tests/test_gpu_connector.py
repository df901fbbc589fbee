"""Token-slot kernels, the pool's slot paths and AMFKVConnector on the GPU.

The connector's save stores flat[:, slots] of every layer as the dense
[L, 2, T, H, D] entry put_from_raw makes, and its load writes
decompress(entry)[:, :n] to flat_cache[:, slots[:n]]
(korith_vllm_ext/amf_kv_connector.py:345-385, 411-483).  Every check here is
bit for bit against the oracle's slot gather / scatter and codecs."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import codecs as oc
from oracle import gen, paging

from helpers import bits, bytes_of

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
FORMATS = ["fp8_e4m3", "int4_sym_block", "fp8_e4m3_ph", "int4_sym", "int4_asym_g32"]


def _pool(**kw):
    from korith_vllm_ext.compressed_vram_pool import CompressedVRAMPool

    args = dict(num_layers=4, bytes_per_layer=8 << 20, block_bytes=1 << 14,
                default_format="fp8_e4m3", device="cuda")
    args.update(kw)
    return CompressedVRAMPool(**args)


def _u16(t: torch.Tensor) -> np.ndarray:
    return bits(t) if t.element_size() == 2 else t.detach().cpu().contiguous().numpy()


def _want_dense(fmt: str, dense: torch.Tensor, dtype) -> torch.Tensor:
    """Oracle decompression of one dense layer [2, T, H, D] as put_from_raw
    stores it (pages of 16 tokens for the paged formats, zero padded)."""
    if fmt == "fp8_e4m3":
        c, s = oc.fp8_tensor_compress(dense)
        return oc.fp8_tensor_decompress(c, s, dtype)
    if fmt == "int4_sym":
        pk, sc = oc.int4_channel_compress(dense)
        return oc.int4_channel_decompress(pk, sc, tuple(dense.shape), dtype)
    if fmt == "int4_sym_block":
        pk, sc, meta = oc.int4_block_compress(dense)
        return oc.int4_block_decompress(pk, sc, tuple(dense.shape), meta, dtype)
    _, T, H, D = dense.shape
    n = -(-T // 16)
    pages = torch.zeros(2, n * 16, H, D, dtype=dense.dtype)
    pages[:, :T] = dense
    pages = pages.view(2, n, 16, H, D)
    if fmt == "fp8_e4m3_ph":
        out = oc.fp8_ph_decompress(*oc.fp8_ph_compress(pages), dtype)
    else:
        c, pr = oc.int4_asym_compress(pages)
        out = oc.int4_asym_decompress(c, pr, 16, H, D, dtype)
    return out.reshape(2, n * 16, H, D)[:, :T]


def _slots_of(blocks, bs, n):
    return paging.slot_mapping(blocks, bs, n)


def _from_bits(a: np.ndarray, dtype) -> torch.Tensor:
    """A tensor of `dtype` holding the raw bits of a numpy array."""
    if a.dtype == np.uint8:
        return torch.from_numpy(np.ascontiguousarray(a)).view(dtype)
    if a.dtype == np.float32:
        return torch.from_numpy(np.ascontiguousarray(a))
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def _blob_regions(p, e):
    """The written bytes of each layer blob of entry e: codes, then the
    shared params or each plane's params (alignment padding left out)."""
    lay = e.layout
    out = []
    for b in e.blocks:
        slab = p._slabs[b.layer_id]
        parts = [bytes_of(slab.narrow(0, b.data_offset, lay.data_bytes))]
        if lay.family != "raw":
            if lay.shared_params:
                parts.append(bytes_of(slab.narrow(0, b.data_offset + lay.scale_offset,
                                                  lay.shared_param_bytes)))
            else:
                for pl in range(lay.n_planes):
                    parts.append(bytes_of(slab.narrow(0, b.data_offset + lay.param_offset(pl),
                                                      lay.plane_param_bytes)))
        out.append(np.concatenate(parts))
    return out


# ------------------------------------------------------------ slot kernels --

# (H, D, dtype, block_size, layout): layout "5d" = [2, nb, bs, H, D];
# "nb2" = [nb, 2, bs, H, D] (page stride twice the page); "flat" = [2, S, H, D]
SLOT_GEOMS = [
    (2, 64, torch.bfloat16, 16, "5d"),     # 256-byte rows: 16 lanes per row
    (8, 128, torch.bfloat16, 16, "5d"),    # 2 KiB rows: a wave per row, two trips
    (1, 32, torch.float16, 16, "nb2"),     # 64-byte rows: 4 lanes per row
    (3, 32, torch.float32, 16, "nb2"),     # 384-byte rows: 24 of 32 lanes busy
    (4, 64, torch.bfloat16, 1, "flat"),    # one-token pages
]


def _make_cache(H, D, dtype, bs, layout, nb, seed, value=None):
    g = torch.Generator().manual_seed(seed)
    shape = {"5d": (2, nb, bs, H, D), "nb2": (nb, 2, bs, H, D), "flat": (2, nb, H, D)}[layout]
    if value is None:
        x = (torch.randn(*shape, generator=g) * 4).to(dtype)
    else:
        x = torch.full(shape, value, dtype=dtype)
    return x


def _planes(x, layout):
    """The [2, nb, bs, H, D] view (numpy-side order) of a cache tensor."""
    if layout == "nb2":
        return x.transpose(0, 1)
    if layout == "flat":
        return x.unsqueeze(2)
    return x


@pytest.mark.parametrize("geom", SLOT_GEOMS, ids=lambda g: f"{g[0]}x{g[1]}-{g[2]}-bs{g[3]}-{g[4]}")
def test_slot_gather_scatter_bitexact(geom):
    from korith_vllm_ext import _paged

    H, D, dtype, bs, layout = geom
    nb = 40 if bs > 1 else 640
    x = _make_cache(H, D, dtype, bs, layout, nb, seed=H * D)
    dx = x.to(DEV)
    view = _paged.planes_view([_planes(dx, layout)[0], _planes(dx, layout)[1]])
    S = nb * bs
    rng = np.random.default_rng(H + D)
    src_slots = rng.permutation(S)[:301].tolist()
    dst_slots = rng.permutation(S)[:301].tolist()
    n = len(src_slots)
    out = torch.empty(2, n, H, D, dtype=dtype, device=DEV)
    _paged.gather_slots(view, _paged.SlotMap(src_slots), n,
                        [out[0].data_ptr(), out[1].data_ptr()], H * D * out.element_size())
    torch.cuda.synchronize()
    want = paging.gather_slots(_u16(_planes(x, layout)), src_slots)
    assert np.array_equal(_u16(out), want)

    target = _make_cache(H, D, dtype, bs, layout, nb, seed=0, value=-3.5).to(DEV)
    tview = _paged.planes_view([_planes(target, layout)[0], _planes(target, layout)[1]])
    _paged.scatter_slots([out[0].data_ptr(), out[1].data_ptr()], H * D * out.element_size(),
                         tview, _paged.SlotMap(dst_slots), n)
    torch.cuda.synchronize()
    want_t = paging.scatter_slots(
        _u16(_planes(_make_cache(H, D, dtype, bs, layout, nb, 0, value=-3.5), layout)).copy(),
        dst_slots, want)
    assert np.array_equal(_u16(_planes(target, layout).contiguous()), want_t)


def test_slot_out_of_range_is_skipped_and_flagged():
    """Slot ids outside [0, pool_slots) are skipped by the kernel's own range
    check and reported in err_flag; the other rows still move."""
    import amf_hip
    from korith_vllm_ext import _paged

    H, D, nb, bs = 2, 64, 8, 16
    x = torch.randn(2, nb, bs, H, D).to(torch.bfloat16).to(DEV)
    view = _paged.cache_view([x])
    slots = _paged.SlotMap([3, nb * bs, 7, -1, 100])
    out = torch.zeros(2, 5, H, D, dtype=torch.bfloat16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    _paged.gather_slots(view, slots, 5, [out[0].data_ptr(), out[1].data_ptr()], H * D * 2,
                        err_flag=flag)
    torch.cuda.synchronize()
    assert flag.item() == amf_hip.ERRFLAG_BLOCK_RANGE
    flat = x.view(2, nb * bs, H, D)
    for j, s in enumerate([3, None, 7, None, 100]):
        if s is None:
            assert torch.count_nonzero(out[:, j]).item() == 0
        else:
            assert torch.equal(out[:, j], flat[:, s])


# ------------------------------------------------------- pool slot paths --


@pytest.mark.parametrize("fmt", FORMATS + ["raw"])
def test_put_from_slots_matches_put_from_raw(fmt):
    """Page-ordered slots (quantized straight from the cache pages), the same
    rows through a flat one-token-page view (slot gather, then put_from_raw)
    and put_from_raw of the oracle's gathered rows give the same entry bytes,
    and the entry decompresses to the oracle's values."""
    L, nb, H, D = 3, 48, 2, 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(FORMATS.index(fmt) if fmt in FORMATS else 9)
    vals = gen.kv_values((L, 2, nb, 16, H, D), D, g, True, dtype)
    if fmt == "raw":
        vals = torch.randint(0, 256, (L, 2, nb, 16, H, D), generator=g, dtype=torch.uint8) \
            .view(torch.float8_e4m3fn)
        dtype = torch.float8_e4m3fn
    cache = [vals[l].to(DEV) for l in range(L)]
    blocks = gen.block_table(nb, 9, 5).tolist()
    slots = _slots_of(blocks, 16, 9 * 16)
    p = _pool(num_layers=L, default_format=fmt if fmt != "raw" else "fp8_e4m3")
    assert p.put_from_slots("paged", cache, torch.tensor(slots))
    flat = [c.view(2, nb * 16, 1, H, D) for c in cache]
    assert p.put_from_slots("flat", flat, slots)
    dense = torch.stack([_from_bits(paging.gather_slots(
        vals[l].view(torch.uint8).numpy() if fmt == "raw" else _u16(vals[l]), slots), dtype)
        for l in range(L)])
    assert p.put_from_raw("raw_path", dense.to(DEV))
    torch.cuda.synchronize()
    entries = [p.get(k) for k in ("paged", "flat", "raw_path")]
    assert entries[0].format == ("raw" if fmt == "raw" else fmt)
    assert all(e.layout == entries[0].layout for e in entries)
    assert all(e.num_tokens == 9 * 16 for e in entries)

    ref = _blob_regions(p, entries[2])
    for e in entries[:2]:
        for a, b in zip(_blob_regions(p, e), ref):
            assert np.array_equal(a, b)
    if fmt == "raw":
        return
    for tdt in (torch.bfloat16, torch.float32):
        got = p.restore_to_tensor("paged", target_dtype=tdt)
        assert got.shape == (L, 2, 9 * 16, H, D)
        for l in range(L):
            assert torch.equal(got[l].cpu(), _want_dense(fmt, dense[l], tdt))


@pytest.mark.parametrize("fmt", FORMATS)
def test_restore_to_slots_paths(fmt):
    """restore_to_slots writes decompress(entry)[:, :n] to the slots, n =
    min(tokens, slots), for page-ordered slots (codec kernel into the pages),
    unordered slots (dense buffer + slot kernel), fewer slots than tokens and
    a layer offset; untouched rows keep the sentinel."""
    L, nb, H, D, T = 3, 40, 4, 64, 144
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(30 + FORMATS.index(fmt))
    dense = gen.kv_values((L, 2, T, H, D), D, g, True, dtype)
    p = _pool(num_layers=L, default_format=fmt)
    assert p.put_from_raw("e", dense.to(DEV), format=fmt)
    rng = np.random.default_rng(FORMATS.index(fmt))
    cases = {
        "pages": _slots_of(gen.block_table(nb, 9, 7).tolist(), 16, T),
        "unordered": rng.permutation(nb * 16)[:T].tolist(),
        "short": _slots_of(gen.block_table(nb, 5, 8).tolist(), 16, 80),
        "ragged": rng.permutation(nb * 16)[:37].tolist(),
    }
    want_l = [_want_dense(fmt, dense[l], dtype) for l in range(L)]
    for name, slots in cases.items():
        target = [torch.full((2, nb, 16, H, D), -7.25, dtype=dtype, device=DEV)
                  for _ in range(L)]
        assert p.restore_to_slots("e", target, torch.tensor(slots)) == T
        torch.cuda.synchronize()
        n = min(T, len(slots))
        for l in range(L):
            want = np.full((2, nb, 16, H, D), 0, np.uint16)
            want[:] = bits(torch.tensor(-7.25, dtype=dtype))
            paging.scatter_slots(want, slots[:n], bits(want_l[l][:, :n]))
            assert np.array_equal(bits(target[l]), want), (name, l)
    one = [torch.full((2, nb, 16, H, D), -7.25, dtype=dtype, device=DEV)]
    slots = cases["pages"]
    assert p.restore_to_slots("e", one, slots, first_layer=2) == T
    torch.cuda.synchronize()
    want = np.full((2, nb, 16, H, D), bits(torch.tensor(-7.25, dtype=dtype)), np.uint16)
    paging.scatter_slots(want, slots, bits(want_l[2]))
    assert np.array_equal(bits(one[0]), want)
    assert p.restore_to_slots("missing", one, slots) == 0
    with pytest.raises(ValueError):
        p.restore_to_slots("e", one, [nb * 16])
    with pytest.raises(ValueError):
        p.restore_to_slots("e", [torch.zeros(2, nb, 16, H, 32, dtype=dtype, device=DEV)], slots)


# --------------------------------------------------------------- connector --


def _connector(fmt, load_stream, L, H, D):
    from korith_vllm_ext.amf_kv_connector import AMFKVConnector, KVConnectorRole

    extra = dict(num_layers=L, num_kv_heads=H, head_dim=D, bytes_per_layer=8 << 20,
                 default_format=fmt, min_prefix_tokens=64, load_stream=load_stream)
    cfg = SimpleNamespace(cache_config=SimpleNamespace(block_size=16),
                          kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra))
    return AMFKVConnector(cfg, KVConnectorRole.WORKER)


def _sched(new_reqs):
    cached = SimpleNamespace(req_ids=[], resumed_req_ids=set(), num_computed_tokens=[],
                             new_block_ids=[])
    return SimpleNamespace(scheduled_new_reqs=new_reqs, scheduled_cached_reqs=cached,
                           num_scheduled_tokens={})


def _forward(caches, shape_fn):
    layers = {f"model.layers.{l}.self_attn.attn": SimpleNamespace(kv_cache=[shape_fn(c)])
              for l, c in enumerate(caches)}
    return SimpleNamespace(attn_metadata=object(), no_compile_layers=layers, virtual_engine=0)


@pytest.mark.parametrize("load_stream", ["side", "current"])
@pytest.mark.parametrize("fmt", ["fp8_e4m3", "int4_sym_block", "int4_asym_g32"])
def test_connector_cold_save_then_warm_load(fmt, load_stream):
    """A cold prefill's save_kv_layer / wait_for_save, then a warm request's
    start_load_kv / wait_for_layer_load through the scheduler metadata; the
    warm request's pages hold the oracle's decompression of the cold
    request's rows, read on the forward stream right after each layer's
    wait."""
    from korith_vllm_ext.amf_kv_connector import AMFReqMeta

    L, nb, H, D = 4, 64, 2, 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(77)
    vals = gen.kv_values((L, 2, nb, 16, H, D), D, g, True, dtype)
    caches = [vals[l].to(DEV) for l in range(L)]
    c = _connector(fmt, load_stream, L, H, D)
    prompt = list(range(5000, 5000 + 150))
    cold_blocks = gen.block_table(nb, 10, 11).tolist()

    c.update_state_after_alloc(SimpleNamespace(request_id="cold"), None, 0)
    meta = c.build_connector_meta(_sched([SimpleNamespace(
        req_id="cold", prompt_token_ids=prompt, block_ids=(cold_blocks,))]))
    assert meta.requests[0].is_store
    c.bind_connector_metadata(meta)
    fwd = _forward(caches, lambda t: t)
    c.start_load_kv(fwd)
    for name, layer in fwd.no_compile_layers.items():
        c.wait_for_layer_load(name)
        c.save_kv_layer(name, layer.kv_cache[0], None)
    c.wait_for_save()
    c.clear_connector_metadata()
    saved = meta.requests[0]
    assert saved.prefix_hash in c._pool and saved.prefix_hash in c._known_hashes

    n_hit, is_async = c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=prompt), 0)
    assert (n_hit, is_async) == (paging.align_to_block_size(149, 16), False)
    warm_blocks = gen.block_table(nb, 10, 12).tolist()
    warm = SimpleNamespace(request_id="warm")
    c.update_state_after_alloc(warm, None, n_hit)
    meta2 = c.build_connector_meta(_sched([SimpleNamespace(
        req_id="warm", prompt_token_ids=prompt, block_ids=(warm_blocks,))]))
    assert not meta2.requests[0].is_store
    c.bind_connector_metadata(meta2)
    targets = [torch.full_like(t, -7.25) for t in caches]
    fwd2 = _forward(targets, lambda t: t)
    c.start_load_kv(fwd2)
    seen = []
    for name in fwd2.no_compile_layers:
        c.wait_for_layer_load(name)
        seen.append(fwd2.no_compile_layers[name].kv_cache[0].clone())  # forward stream
    c.wait_for_save()
    torch.cuda.synchronize()

    want_meta = AMFReqMeta.make("w", "", prompt, warm_blocks, 16, False)
    save_slots = saved.slot_mapping.tolist()
    load_slots = want_meta.slot_mapping.tolist()
    n = min(len(save_slots), len(load_slots))
    for l in range(L):
        dense = _from_bits(paging.gather_slots(_u16(vals[l]), save_slots), dtype)
        want = np.full((2, nb, 16, H, D), bits(torch.tensor(-7.25, dtype=dtype)), np.uint16)
        paging.scatter_slots(want, load_slots[:n], bits(_want_dense(fmt, dense, dtype)[:, :n]))
        assert np.array_equal(bits(seen[l]), want), l
        assert np.array_equal(bits(targets[l]), want), l


def test_connector_flat_caches_and_misses():
    """[2, slots, H * D] caches (one-token pages through the slot kernels),
    a load whose entry is gone (a logged miss that leaves the cache alone)
    and layers beyond the entry's."""
    L, nb, H, D = 2, 32, 2, 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(5)
    vals = gen.kv_values((L, 2, nb, 16, H, D), D, g, True, dtype)
    flat = [vals[l].reshape(2, nb * 16, H * D).to(DEV) for l in range(L)]
    c = _connector("fp8_e4m3_ph", "side", L, H, D)
    prompt = list(range(100))
    blocks = [3, 30, 7, 1, 12, 9, 20]
    meta = c.build_connector_meta(_sched([SimpleNamespace(req_id="a", prompt_token_ids=prompt,
                                                          block_ids=(blocks,))]))
    c.bind_connector_metadata(meta)
    for l in range(L):
        c.save_kv_layer(f"model.layers.{l}.attn", flat[l], None)
    c.wait_for_save()
    req = meta.requests[0]
    slots = req.slot_mapping.tolist()

    c.update_state_after_alloc(SimpleNamespace(request_id="b"), None, 80)
    warm_blocks = [0, 2, 4, 6, 8, 10, 11]
    meta2 = c.build_connector_meta(_sched([SimpleNamespace(req_id="b", prompt_token_ids=prompt,
                                                           block_ids=(warm_blocks,))]))
    c.bind_connector_metadata(meta2)
    targets = [torch.zeros_like(t) for t in flat] + [torch.zeros_like(flat[0])]
    fwd = SimpleNamespace(attn_metadata=object(), no_compile_layers={
        f"model.layers.{l}.attn": SimpleNamespace(kv_cache=targets[l]) for l in range(L + 1)})
    c.start_load_kv(fwd)
    for name in fwd.no_compile_layers:
        c.wait_for_layer_load(name)
    torch.cuda.synchronize()
    load_slots = meta2.requests[0].slot_mapping.tolist()
    for l in range(L):
        dense = _from_bits(paging.gather_slots(_u16(vals[l]), slots), dtype)
        want = np.zeros((2, nb, 16, H, D), np.uint16)
        paging.scatter_slots(want, load_slots, bits(_want_dense("fp8_e4m3_ph", dense, dtype)))
        assert np.array_equal(bits(targets[l].view(2, nb, 16, H, D)), want)
    assert torch.count_nonzero(targets[L]).item() == 0   # no layer 2 in the entry

    c._pool.delete(req.prefix_hash)
    c.update_state_after_alloc(SimpleNamespace(request_id="c"), None, 80)
    c.bind_connector_metadata(c.build_connector_meta(_sched([SimpleNamespace(
        req_id="c", prompt_token_ids=prompt, block_ids=(warm_blocks,))])))
    again = [torch.zeros_like(t) for t in flat]
    c.start_load_kv(SimpleNamespace(attn_metadata=object(), no_compile_layers={
        f"model.layers.{l}.attn": SimpleNamespace(kv_cache=again[l]) for l in range(L)}))
    torch.cuda.synchronize()
    assert all(torch.count_nonzero(t).item() == 0 for t in again)
    # the missed load's blocks go back to vLLM for recomputation (once), and
    # the scheduler no longer reports the evicted prefix as a hit
    n_valid = paging.align_to_block_size(len(prompt), 16) // 16
    assert c.get_block_ids_with_load_errors() == set(warm_blocks[:n_valid])
    assert c.get_block_ids_with_load_errors() == set()
    assert req.prefix_hash not in c._known_hashes
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=prompt), 0) == (0, False)


@pytest.mark.parametrize("fmt,bs", [("fp8_e4m3_ph", 32), ("int4_asym_g32", 64),
                                    ("int4_sym_block", 128), ("fp8_e4m3", 1)])
def test_slot_paths_other_block_sizes(fmt, bs, monkeypatch):
    """vLLM blocks of 32, 64, 128 tokens or one token: slots in aligned runs
    of the entry's page length go through the codec kernels directly (the slot
    kernel is never called), and the results match the oracle."""
    from korith_vllm_ext import _paged

    L, H, D = 2, 2, 64
    S = 4096
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(bs)
    vals = gen.kv_values((L, 2, S // bs, bs, H, D), D, g, True, dtype)
    cache = [vals[l].to(DEV) for l in range(L)]
    page = 128 if fmt == "int4_sym_block" else 16
    T = 512
    blocks = gen.block_table(S // max(bs, page), T // max(bs, page), 3).tolist()
    if bs >= page:
        slots = _slots_of(blocks, bs, T)
    else:  # one-token blocks: runs of `page` slots at page-aligned places
        slots = _slots_of(blocks, page, T)

    def no_slot_kernel(*a, **k):
        raise AssertionError("slot kernel used on an aligned slot list")

    monkeypatch.setattr(_paged, "scatter_slots", no_slot_kernel)
    monkeypatch.setattr(_paged, "gather_slots", no_slot_kernel)
    p = _pool(num_layers=L, default_format=fmt)
    assert p.put_from_slots("k", cache, slots)
    got = p.restore_to_tensor("k", target_dtype=dtype)
    want_l = []
    for l in range(L):
        dense = _from_bits(paging.gather_slots(_u16(vals[l]), slots), dtype)
        want_l.append(_want_dense(fmt, dense, dtype))
        assert torch.equal(got[l].cpu(), want_l[l])
    dst_blocks = gen.block_table(S // max(bs, page), T // max(bs, page), 4).tolist()
    dst = _slots_of(dst_blocks, bs if bs >= page else page, T)
    target = [torch.full_like(c, -7.25) for c in cache]
    assert p.restore_to_slots("k", target, dst) == T
    torch.cuda.synchronize()
    for l in range(L):
        want = np.full(tuple(target[l].shape), bits(torch.tensor(-7.25, dtype=dtype)), np.uint16)
        paging.scatter_slots(want, dst, bits(want_l[l]))
        assert np.array_equal(bits(target[l]), want), l
