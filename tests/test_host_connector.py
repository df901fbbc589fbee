"""AMFKVConnector host logic on the CPU: prefix hashing, block alignment,
slot mappings, scheduler-side metadata and the no-GPU behaviour, against the
oracle's restatements of korith_vllm_ext/amf_kv_connector.py."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import paging


def _conn(role=None, **extra):
    from korith_vllm_ext.amf_kv_connector import AMFKVConnector, KVConnectorRole

    cfg = SimpleNamespace(
        cache_config=SimpleNamespace(block_size=extra.pop("block_size", 16)),
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra),
    )
    return AMFKVConnector(cfg, role or KVConnectorRole.WORKER)


def test_prefix_hash_and_align_match_oracle():
    from korith_vllm_ext.amf_kv_connector import _prefix_hash, align_to_block_size

    rng = np.random.default_rng(0)
    for n in (0, 1, 7, 64, 300):
        toks = rng.integers(-(1 << 33), 1 << 33, size=n).tolist()
        assert _prefix_hash(toks) == paging.prefix_hash(toks)
    big = [1 << 70, -(1 << 65) - 3, 7]                 # beyond int64: the word-by-word route
    assert _prefix_hash(big) == paging.prefix_hash(big)
    for n in range(-3, 70):
        for bs in (1, 4, 16):
            assert align_to_block_size(n, bs) == paging.align_to_block_size(n, bs)


@pytest.mark.parametrize("n_tokens", [0, 1, 16, 17, 40, 64])
def test_req_meta_slots_match_oracle(n_tokens):
    from korith_vllm_ext.amf_kv_connector import AMFReqMeta

    blocks = [9, 3, 12, 0]
    toks = list(range(100, 100 + n_tokens))
    m = AMFReqMeta.make("r", "h", toks, blocks, 16, True)
    valid = paging.align_to_block_size(n_tokens, 16)
    assert m.num_tokens == valid
    assert m.slot_mapping.tolist() == paging.slot_mapping(blocks, 16, valid)
    assert m.token_ids.tolist() == toks[:valid]


def test_slot_map_page_structure():
    from korith_vllm_ext._paged import SlotMap

    slots = paging.slot_mapping([5, 2, 7], 16, 48)
    sm = SlotMap(torch.tensor(slots))
    assert sm.page_ids(48, 16) == [5, 2, 7]
    assert sm.page_ids(32, 16) == [5, 2]
    assert sm.page_ids(40, 16) is None          # partial page
    assert sm.page_ids(48, 8) == [10, 11, 4, 5, 14, 15]
    assert sm.page_ids(48, 32) is None          # block 5 is not 32-aligned
    swapped = list(slots)
    swapped[3], swapped[4] = swapped[4], swapped[3]
    assert SlotMap(swapped).page_ids(48, 16) is None
    shifted = [s + 1 for s in slots]
    assert SlotMap(shifted).page_ids(48, 16) is None
    sm.check(8 * 16)
    with pytest.raises(ValueError):
        sm.check(7 * 16)
    with pytest.raises(ValueError):
        SlotMap([-1, 3]).check(100)


def test_layer_index():
    from korith_vllm_ext.amf_kv_connector import _layer_index

    assert _layer_index("model.layers.0.self_attn") == 0
    assert _layer_index("model.layers.27.self_attn.attn") == 27
    assert _layer_index("model.decoder.layers.x.attn") is None
    assert _layer_index("lm_head") is None


def _new_req(req_id, tokens, blocks):
    return SimpleNamespace(req_id=req_id, prompt_token_ids=tokens, block_ids=(blocks,))


def _sched_out(new=(), cached_ids=(), resumed=(), computed=(), new_blocks=(), scheduled=None):
    cached = SimpleNamespace(req_ids=list(cached_ids), resumed_req_ids=set(resumed),
                             num_computed_tokens=list(computed),
                             new_block_ids=list(new_blocks))
    return SimpleNamespace(scheduled_new_reqs=list(new), scheduled_cached_reqs=cached,
                           num_scheduled_tokens=scheduled or {})


def test_scheduler_metadata_store_load_and_resumed():
    from korith_vllm_ext.amf_kv_connector import AMFConnectorMetadata, KVConnectorRole

    c = _conn(KVConnectorRole.SCHEDULER)
    toks = list(range(1000, 1000 + 70))
    # no pool without a GPU: a hit comes only from the known-hash set
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=toks), 0) == (0, False)
    n_check = paging.align_to_block_size(len(toks) - 1, 16)
    h = paging.prefix_hash(toks[:n_check])
    c._known_hashes.add(h)
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=toks), 0) == \
        (n_check, False)
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=toks), n_check) == \
        (0, False)
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=toks[:63]), 0) == \
        (0, False)                                   # below min_prefix_tokens

    load = SimpleNamespace(request_id="L", all_token_ids=toks)
    c.update_state_after_alloc(load, None, 0)
    assert not c._requests_need_load
    c.update_state_after_alloc(load, None, n_check)
    resumed = SimpleNamespace(request_id="R", all_token_ids=toks + [1, 2, 3])
    c.update_state_after_alloc(resumed, None, 16)
    out = _sched_out(new=[_new_req("L", toks, [4, 5, 6, 7, 8]),
                          _new_req("S", toks[:40], [1, 2, 3])],
                     cached_ids=["X", "R"], resumed=["R"], computed=[0, 32],
                     new_blocks=[None, ([10, 11, 12, 13],)], scheduled={"R": 20})
    meta = c.build_connector_meta(out)
    assert isinstance(meta, AMFConnectorMetadata) and not c._requests_need_load
    by_id = {r.request_id: r for r in meta.requests}
    assert set(by_id) == {"L", "S", "R"}
    assert not by_id["L"].is_store and by_id["S"].is_store and not by_id["R"].is_store
    assert by_id["L"].prefix_hash == h
    assert by_id["L"].slot_mapping.tolist() == paging.slot_mapping(
        [4, 5, 6, 7, 8], 16, paging.align_to_block_size(70, 16))
    n_s = paging.align_to_block_size(39, 16)
    assert by_id["S"].prefix_hash == paging.prefix_hash(toks[:n_s])
    r_toks = (toks + [1, 2, 3])[:52]
    assert by_id["R"].prefix_hash == paging.prefix_hash(
        r_toks[:paging.align_to_block_size(51, 16)])
    assert by_id["R"].slot_mapping.tolist() == paging.slot_mapping(
        [10, 11, 12, 13], 16, paging.align_to_block_size(52, 16))
    # a load the scheduler accepted but did not schedule trips the check
    c.update_state_after_alloc(load, None, 16)
    with pytest.raises(AssertionError):
        c.build_connector_meta(_sched_out())


def test_worker_without_gpu_is_inert():
    """Without a GPU the pool cannot be made: loads do nothing, saves drop
    their layers (reference: amf_kv_connector.py:188-197, 334-335, 440-443)."""
    from korith_vllm_ext.amf_kv_connector import AMFConnectorMetadata, AMFReqMeta

    if torch.cuda.is_available():
        pytest.skip("checks the no-GPU behaviour")
    c = _conn()
    meta = AMFConnectorMetadata([AMFReqMeta.make("s", "h", list(range(40)), [0, 1, 2], 16, True)])
    c.bind_connector_metadata(meta)
    c.start_load_kv(SimpleNamespace(attn_metadata=object(), no_compile_layers={}))
    c.save_kv_layer("model.layers.0.attn", torch.zeros(2, 4, 16, 2, 64), None)
    assert "h" in c._save_layers
    c.wait_for_save()
    assert c._pool is None and not c._save_layers
    c.wait_for_layer_load("model.layers.0.attn")
    c.clear_connector_metadata()
    assert not c.has_connector_metadata()
    assert type(c).requires_piecewise_for_cudagraph({}) is True


def test_bad_load_stream_option():
    with pytest.raises(ValueError):
        _conn(load_stream="sideways")
    assert _conn()._side_load is False                  # the forward's stream by default
    assert _conn(load_stream="side")._side_load is True


def test_load_launch_groups():
    """Consecutive layers of one geometry share a launch; on a side stream the
    first layer is a launch of its own."""
    from korith_vllm_ext.amf_kv_connector import _layer_groups

    a = torch.zeros(2, 4, 16, 2, 64)
    b = torch.zeros(2, 4, 16, 2, 128)
    layers = [(i, f"l{i}", a) for i in range(4)] + [(4, "l4", b), (6, "l6", b), (7, "l7", b)]
    ids = lambda groups: [[i for i, _, _ in g] for g in groups]
    assert ids(_layer_groups(layers, False)) == [[0, 1, 2, 3], [4], [6, 7]]
    assert ids(_layer_groups(layers, True)) == [[0], [1, 2, 3], [4], [6, 7]]
    assert _layer_groups([], True) == []


def test_token_pages_recut():
    from korith_vllm_ext import _paged

    x = torch.zeros(2, 8, 32, 2, 64, dtype=torch.bfloat16)
    v = _paged.cache_view([x])
    r = _paged.token_pages(v, 16)
    assert (r.block_size, r.pool_pages, r.page_stride) == (16, 16, 16 * 2 * 64 * 2)
    assert r.planes == v.planes
    assert _paged.token_pages(v, 32) is v
    assert _paged.token_pages(v, 512) is None          # fewer rows than one page
    nb2 = torch.zeros(8, 2, 32, 2, 64, dtype=torch.bfloat16)
    pv = _paged.planes_view([nb2[:, 0], nb2[:, 1]])
    assert _paged.token_pages(pv, 32) is pv            # padded pages: only their own length
    assert _paged.token_pages(pv, 16) is None
