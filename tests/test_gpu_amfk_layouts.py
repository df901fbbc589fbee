"""AmfKvManager behaviour of the reference's mock-CacheEngine suite
(platform/tests/test_vllm_amf.py:167-291) on a HIP device, in the old vLLM
layout [2, n_blocks, n_kv_heads, block_size, head_dim] the suite uses (a
block is still one contiguous run, so pages move as the same bytes), plus
the AMFK bytes of that layout against the oracle's header and table."""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import amfk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


class _Engine:
    def __init__(self, caches):
        self.gpu_cache = caches


class _Cfg:
    max_model_len = 4096
    num_attention_layers = 4


def _engine(n_layers=4, n_blocks=8, n_kv_heads=2, block_size=16, head_dim=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    return _Engine([torch.randn(2, n_blocks, n_kv_heads, block_size, head_dim, generator=g)
                    .to(torch.float16).to(DEV) for _ in range(n_layers)])


def _manager(store, engine=None):
    from korith_vllm_ext.amf_kv_manager import AmfKvManager

    return AmfKvManager(engine or _engine(), str(store), _Cfg(), model_hash=0xDEAD,
                        tenant_id="test")


def test_save_files_magic_version(tmp_path):
    mgr = _manager(tmp_path)
    assert mgr.save_kv_state(list(range(100)), [0, 1, 2, 3])
    kv = list(Path(tmp_path).glob("*.kv"))
    assert len(kv) == 1 and len(list(Path(tmp_path).glob("*.tok"))) == 1
    data = kv[0].read_bytes()
    magic, version = struct.unpack_from("<II", data, 0)
    assert magic == 0x414D464B and version == 1


def test_snapshot_restore_stats_and_misses(tmp_path):
    mgr = _manager(tmp_path)
    toks = list(range(80))
    assert not mgr.has_snapshot(toks)
    assert mgr.restore_kv_state(toks, [0]) == 0
    assert mgr.save_kv_state(toks, [0, 1])
    assert mgr.has_snapshot(toks)
    assert mgr.restore_kv_state(toks, [0, 1]) == len(toks)
    s = mgr.stats()
    assert s["hits"] == 1 and s["saves"] == 1
    assert mgr.save_kv_state(list(range(1, 81)), [0])
    assert len(list(Path(tmp_path).glob("*.kv"))) == 2


def test_old_layout_bytes_and_round_trip(tmp_path):
    """Header n_kv_heads = shape[-3] (here the head count), payload = the
    blocks' bytes in block-table order, restore puts them back bit for bit."""
    L, nb, H, bs, D = 3, 12, 2, 16, 32
    eng = _engine(L, nb, H, bs, D, seed=4)
    mgr = _manager(tmp_path, eng)
    toks = list(range(500, 500 + 3 * bs))
    src = [7, 2, 10]
    assert mgr.save_kv_state(toks, src)
    data = mgr._kv_filename(mgr.compute_amf_key(toks)).read_bytes()
    plane = len(src) * H * bs * D * 2
    hdr = amfk.pack_header(L, len(toks), H, D, 0, 2 * L * plane, 0xDEAD, amfk.hash_tokens(toks))
    tab = b"".join(np.array(e, dtype="<u8").tobytes()
                   for e in amfk.layer_table([(plane, plane)] * L))
    payload = b"".join(eng.gpu_cache[l][kv][torch.tensor(src)].contiguous().view(torch.uint8)
                       .cpu().numpy().tobytes() for l in range(L) for kv in range(2))
    assert data == hdr + tab + payload
    target = _Engine([torch.zeros_like(c) for c in eng.gpu_cache])
    dst = [0, 11, 5]
    assert _manager(tmp_path, target).restore_kv_state(toks, dst) == len(toks)
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(target.gpu_cache[l][:, dst], eng.gpu_cache[l][:, src])
        rest = [b for b in range(nb) if b not in dst]
        assert torch.count_nonzero(target.gpu_cache[l][:, rest]).item() == 0
