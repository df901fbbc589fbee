"""Pool allocator, AMFK manager miss paths and keys on the CPU (no device
work): the slab allocator's first-fit / coalescing / fence bookkeeping, the
pool refusing a CPU device, AMFK header validation, and the key helpers
against the oracle's FNV."""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from korith_vllm_ext.amf_kv_manager import (
    AmfKvManager,
    AmfKVManager,
    amf_float_bits,
    amf_hash_model,
    amf_hash_tenant_id,
    amf_hash_tokens,
    amf_key_filename,
)
from korith_vllm_ext.amf_worker_ext import prefix_key
from korith_vllm_ext.compressed_vram_pool import CompressedVRAMPool, _SlabAllocator
from oracle import amfk


class FakeEvent:
    def __init__(self, done=False):
        self.done = done

    def query(self):
        return self.done


def test_allocator_first_fit_and_coalesce():
    a = _SlabAllocator(10)
    s1, f1 = a.alloc(3)
    s2, _ = a.alloc(4)
    s3, _ = a.alloc(3)
    assert (s1, s2, s3) == (0, 3, 7) and a.alloc(1) is None and f1 == []
    a.free(s2, 4, [FakeEvent()])
    assert a.runs() == [(3, 4)]
    assert a.alloc(5) is None
    got = a.alloc(2)
    assert got[0] == 3 and len(got[1]) == 1          # the span's fence travels with it
    a.free(0, 3)
    a.free(7, 3)
    assert a.runs() == [(0, 3), (5, 5)]
    a.free(3, 2)
    assert a.runs() == [(0, 10)] and a.free_blocks() == 10
    with pytest.raises(ValueError):
        a.free(2, 2)


def test_allocator_prunes_completed_fences():
    """Merged runs keep their fences (duplicates dropped); once a run holds
    many, the completed ones are queried out, the pending ones kept."""
    a = _SlabAllocator(8)
    s, _ = a.alloc(4)
    t, _ = a.alloc(4)
    done, pending = FakeEvent(done=True), FakeEvent(done=False)
    a.free(s, 4, [done, done])
    a.free(t, 4, [pending])
    start, fences = a.alloc(8)
    assert start == 0 and fences == [done, pending]
    a.free(0, 8, [FakeEvent(done=True) for _ in range(9)] + [pending])
    _, fences = a.alloc(8)
    assert fences == [pending]
    a.free(0, 8)
    a.reset(5)
    assert a.runs() == [(5, 3)]


def test_pool_requires_a_gpu_device():
    with pytest.raises(RuntimeError):
        CompressedVRAMPool(num_layers=2, bytes_per_layer=1 << 16, block_bytes=1 << 12,
                           device="cpu")


def test_keys_match_oracle_fnv():
    toks = list(range(1000)) + [-1, 2**31 - 1]
    assert amf_hash_tokens(toks) == amfk.hash_tokens(toks)
    assert amf_hash_tokens([]) == amfk.FNV_OFFSET
    assert amf_hash_tenant_id("") == amfk.FNV_OFFSET
    assert amf_hash_tenant_id("nebius") == amfk.hash_tenant("nebius")
    assert amf_float_bits(1.0) == 0x3F800000
    assert amf_key_filename(1, 2, 3, 4096, 1, 0, 0, 0, 0) == amfk.key_filename(
        1, 2, 3, 4096, 1, 0, 0, 0, 0)
    assert prefix_key("abc") == "abc" and prefix_key(255) == f"{255:016x}"
    assert prefix_key([1, 2, 3]) == f"{amfk.hash_tokens([1, 2, 3]):016x}"
    assert AmfKVManager is AmfKvManager


def test_hash_model_file(tmp_path):
    p = tmp_path / "m.bin"
    data = np.random.default_rng(0).integers(0, 256, 100_000, dtype=np.uint8).tobytes()
    p.write_bytes(data)
    assert amf_hash_model(str(p)) == amfk.fnv1a_bytes(data)
    assert amf_hash_model(str(tmp_path / "missing")) == 0


class _Engine:
    def __init__(self, n_layers):
        self.gpu_cache = [torch.zeros(2, 4, 16, 2, 64, dtype=torch.bfloat16)
                          for _ in range(n_layers)]


class _Cfg:
    max_model_len = 4096


def _write(mgr, tokens, payload: bytes):
    mgr._kv_filename(mgr.compute_amf_key(tokens)).write_bytes(payload)


def test_manager_restore_miss_paths(tmp_path):
    mgr = AmfKvManager(_Engine(2), str(tmp_path), _Cfg())
    toks = [5, 6, 7]
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # no file
    _write(mgr, toks, b"\x00" * 20)
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # too small
    hdr = amfk.pack_header(2, 3, 16, 64, 2, 0, 0, 0)
    _write(mgr, toks, b"XXXX" + hdr[4:])
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # magic
    _write(mgr, toks, hdr[:4] + struct.pack("<I", 9) + hdr[8:])
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # version
    _write(mgr, toks, amfk.pack_header(3, 3, 16, 64, 2, 0, 0, 0))
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # layer count
    _write(mgr, toks, hdr + b"\x00" * 10)
    assert mgr.restore_kv_state(toks, [0, 1]) == 0                         # table cut
    assert mgr.stats()["misses"] == 6 and mgr.stats()["hits"] == 0
    # an empty block table restores nothing but is a hit, as the reference
    tab = b"".join(struct.pack("<4Q", 0, 0, 0, 0) for _ in range(2))
    _write(mgr, toks, hdr + tab)
    assert mgr.restore_kv_state(toks, []) == 3 and mgr.stats()["hits"] == 1
    assert mgr.has_snapshot(toks) and not mgr.has_snapshot([1])


@pytest.mark.parametrize("size", [1000, (8 << 20) + 12345, (21 << 20) + 7])
@pytest.mark.parametrize("threads", ["1", "4"])
def test_snapshot_file_io_round_trip(tmp_path, monkeypatch, size, threads):
    """Chunked positional reads of a snapshot file (the AMFK tier's file
    side) move exactly the file's bytes, with one thread or a pool, for sizes
    below, at and past several chunks; a read past the end raises."""
    from korith_vllm_ext import amf_kv_manager as m

    monkeypatch.setenv("KORITH_AMF_IO_THREADS", threads)
    data = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8)
    path = tmp_path / "snap.kv"
    data.tofile(path)
    back = bytearray(size + 16)
    with open(path, "rb") as f:
        m._read_file_into(f.fileno(), memoryview(back), size)
    assert np.array_equal(np.frombuffer(bytes(back[:size]), dtype=np.uint8), data)
    with open(path, "rb") as f, pytest.raises(OSError):
        m._read_file_into(f.fileno(), memoryview(bytearray(size + 100)), size + 100)


@pytest.mark.parametrize("size", [1000, (8 << 20) + 12345, (21 << 20) + 7])
@pytest.mark.parametrize("threads", ["1", "4"])
@pytest.mark.parametrize("blob_delta", [0, -5, 4096])
def test_snapshot_file_write(tmp_path, monkeypatch, size, threads, blob_delta):
    """A save's file side: the file allocated at the expected size and filled
    through a mapping by the pool, or, when the blob's size differs from the
    expected one (or with one thread, or below two chunks), written by one
    call; the file holds exactly the blob either way, also over an older,
    longer file of the same name."""
    from korith_vllm_ext import amf_kv_manager as m

    monkeypatch.setenv("KORITH_AMF_IO_THREADS", threads)
    n = size + blob_delta
    blob = np.random.default_rng(size + n).integers(0, 256, n, dtype=np.uint8)
    path = tmp_path / "snap.kv.tmp"
    path.write_bytes(b"\x55" * (size + 8192))
    out = m._SnapshotFile(path, size)
    try:
        out.write(memoryview(blob.tobytes()))
    finally:
        out.close()
    assert np.array_equal(np.fromfile(path, dtype=np.uint8), blob)


def test_snapshot_file_close_without_write(tmp_path, monkeypatch):
    """A save that fails before its blob exists still closes the file and
    its mapping."""
    from korith_vllm_ext import amf_kv_manager as m

    monkeypatch.setenv("KORITH_AMF_IO_THREADS", "4")
    out = m._SnapshotFile(tmp_path / "snap.kv.tmp", 16 << 20)
    out.close()
    assert (tmp_path / "snap.kv.tmp").stat().st_size == 16 << 20


def test_snapshot_file_write_without_fallocate(tmp_path, monkeypatch):
    """Where the file system cannot allocate ahead (posix_fallocate fails),
    the save's file side falls back to one write of the whole blob."""
    from korith_vllm_ext import amf_kv_manager as m

    def refuse(fd, off, n):
        raise OSError(95, "Operation not supported")

    monkeypatch.setenv("KORITH_AMF_IO_THREADS", "4")
    monkeypatch.setattr(m.os, "posix_fallocate", refuse)
    size = (12 << 20) + 3
    blob = np.random.default_rng(5).integers(0, 256, size, dtype=np.uint8)
    path = tmp_path / "snap.kv.tmp"
    out = m._SnapshotFile(path, size)
    try:
        out.write(memoryview(blob.tobytes()))
    finally:
        out.close()
    assert np.array_equal(np.fromfile(path, dtype=np.uint8), blob)
