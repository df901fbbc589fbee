"""amf_kv_manager.py - AMFK disk snapshots of vLLM's paged KV cache.

API and file format of the reference (korith_vllm_ext/amf_kv_manager.py:
36-543): a snapshot is `<key>.kv` (56-byte AMFK header, one 32-byte
(k_off, k_size, v_off, v_size) entry per layer, then the payload K0 V0 K1
V1 ...) plus `<key>.tok` (the prompt as little-endian int32), named by the
9-field AMF key.  Files written here and by the reference are byte-identical
for the same cache contents, including the header's n_kv_heads field, which
the reference fills from shape[-3] of a gathered [n_blocks, block_size, H, D]
page stack, i.e. with block_size (amf_kv_manager.py:336-338).

Data movement (libamf_hip.so amf_direct_kv_save_pages / _restore_pages):
  save    the pages of every layer are gathered into one slot of a two-slot
          device staging ring while the other slot is copied D2H into the
          context's pinned blob (header and layer table written natively),
          and the blob is written to the file in one call;
  restore the file is read straight into the pinned staging buffer; the
          header and layer table are validated natively before any copy, then
          H2D copies of one slot overlap the page scatter of the other.
Pinned and device staging are kept across calls.  The reference gathers per
layer with advanced indexing and copies through pageable memory and Python
bytes objects (:311-368, 488-523).
"""

from __future__ import annotations

import ctypes
import logging
import mmap
import os
import struct
import threading
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Any, List, Optional, Sequence

import numpy as np
import torch

import amf_hip

from . import _paged
from .amf_direct_kv import AmfDirectKv, staging_bytes_for

logger = logging.getLogger(__name__)

# Snapshot files are read into the pinned staging buffer in chunks on a small
# thread pool (positional reads release the GIL and share the file), so the
# file side is not one single-threaded copy; KORITH_AMF_IO_THREADS sets the
# pool size (1: one read or write call).  Concurrent write() calls to one file
# serialize on its inode lock and measured slower (25 MB to /dev/shm: 6.1-6.6
# ms with 8 threads against 4.5-4.6 ms), so a save allocates the file
# (posix_fallocate) on the pool while the pages are gathered and copied to the
# host, maps it, and copies the blob in on the pool (page faults of a mapped
# file run in parallel).
_IO_CHUNK = 4 << 20
_io_lock = threading.Lock()
_io_pool: Optional[ThreadPoolExecutor] = None


def _io_threads() -> int:
    try:
        n = int(os.environ.get("KORITH_AMF_IO_THREADS", "8"))
    except ValueError:
        n = 8
    return max(1, min(n, 32))


def _pool() -> ThreadPoolExecutor:
    global _io_pool
    with _io_lock:
        if _io_pool is None:
            _io_pool = ThreadPoolExecutor(max_workers=_io_threads(), thread_name_prefix="amfk-io")
        return _io_pool


def _chunks(size: int) -> List[tuple]:
    return [(off, min(_IO_CHUNK, size - off)) for off in range(0, size, _IO_CHUNK)]


def _pread_all(fd: int, buf: memoryview, off: int, n: int) -> None:
    done = 0
    while done < n:
        got = os.preadv(fd, [buf[off + done:off + n]], off + done)
        if got <= 0:
            raise OSError(f"short read at byte {off + done}")
        done += got


def _read_file_into(fd: int, buf: memoryview, size: int) -> None:
    """Bytes [0, size) of the open file `fd` into buf[0:size]."""
    if _io_threads() == 1 or size < 2 * _IO_CHUNK:
        _pread_all(fd, buf, 0, size)
        return
    for f in [_pool().submit(_pread_all, fd, buf, off, n) for off, n in _chunks(size)]:
        f.result()


def _write_all(fd: int, data: memoryview) -> None:
    done = 0
    while done < len(data):
        done += os.write(fd, data[done:])


class _SnapshotFile:
    """A snapshot file of a known size, created and allocated ahead of its
    bytes (on the IO pool, while the device side runs), then filled through a
    shared mapping by the pool; files where that fails are written by one
    write() call instead."""

    def __init__(self, path: Path, size: int):
        self.path, self.size = path, size
        self.fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
        self._ready = None
        if _io_threads() > 1 and size >= 2 * _IO_CHUNK:
            self._ready = _pool().submit(self._allocate)

    def _allocate(self) -> Optional[mmap.mmap]:
        try:
            os.posix_fallocate(self.fd, 0, self.size)
            return mmap.mmap(self.fd, self.size, flags=mmap.MAP_SHARED,
                             prot=mmap.PROT_READ | mmap.PROT_WRITE)
        except (OSError, ValueError):
            return None

    def write(self, blob: memoryview) -> None:
        mm = self._ready.result() if self._ready is not None else None
        if mm is None or len(blob) != self.size:
            if mm is not None:
                mm.close()
            os.ftruncate(self.fd, 0)
            os.lseek(self.fd, 0, os.SEEK_SET)
            _write_all(self.fd, blob)
            return
        try:
            dst = ctypes.addressof(ctypes.c_char.from_buffer(mm))
            src = int(np.frombuffer(blob, dtype=np.uint8).ctypes.data)
            # ctypes.memmove releases the GIL: one page-aligned piece per pool
            # thread, copied in parallel
            step = -(-self.size // _io_threads())
            step = -(-step // mmap.PAGESIZE) * mmap.PAGESIZE
            for f in [_pool().submit(ctypes.memmove, dst + off, src + off,
                                     min(step, self.size - off))
                      for off in range(0, self.size, step)]:
                f.result()
            del dst
        finally:
            mm.close()

    def close(self) -> None:
        if self._ready is not None and not self._ready.done():
            mm = self._ready.result()
            if mm is not None:
                mm.close()
        os.close(self.fd)



_FNV_OFFSET: int = 1469598103934665603
_FNV_PRIME: int = 1099511628211
_U64_MASK: int = (1 << 64) - 1

_AMFK_MAGIC: int = 0x414D464B  # "AMFK"
_AMFK_VERSION: int = 1
_HEADER_FMT = "<IIIIIIII QQQ"
_HEADER_SIZE = struct.calcsize(_HEADER_FMT)
_LAYER_FMT = "<QQQQ"
_LAYER_SIZE = struct.calcsize(_LAYER_FMT)
assert _HEADER_SIZE == 56 and _LAYER_SIZE == 32

# AMF dtype tags (core/amf_direct_kv.h AmfKvDtype).
_DTYPE_TAG = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}


# ------------------------------------------------------------------ keys --


def _fnv1a_bytes(data: bytes, h: int = _FNV_OFFSET) -> int:
    """FNV-1a over bytes from hash h (libamf_hip.so's amf_fnv1a64)."""
    buf = bytes(data)
    return int(amf_hip.load().amf_fnv1a64(buf, len(buf), h & _U64_MASK))


def amf_hash_tokens(token_ids: Sequence[int]) -> int:
    """Prefix hash: one FNV-1a step per token on its 32-bit value
    (reference: amf_kv_manager.py:75-81; amf_hash_tokens of the C ABI)."""
    arr = np.asarray([int(t) & 0xFFFFFFFF for t in token_ids], dtype=np.uint32)
    return int(amf_hip.load().amf_hash_tokens(arr.ctypes.data, arr.size))


def amf_hash_tenant_id(tenant_id: str) -> int:
    """FNV-1a over the UTF-8 tenant string; "" hashes to the offset basis."""
    if not tenant_id:
        return _FNV_OFFSET
    return _fnv1a_bytes(tenant_id.encode("utf-8"))


def amf_hash_model(model_path: str) -> int:
    """FNV-1a over a model file's bytes, 0 if it does not exist (reference:
    amf_kv_manager.py:84-103).  Reads 16 MiB at a time."""
    path = Path(model_path)
    if not path.exists():
        return 0
    lib = amf_hip.load()
    h = _FNV_OFFSET
    buf = bytearray(16 << 20)
    mv = memoryview(buf)
    with open(path, "rb") as f:
        while True:
            n = f.readinto(mv)
            if not n:
                break
            h = int(lib.amf_fnv1a64((ctypes.c_char * n).from_buffer(buf), n, h))
    return h


def amf_float_bits(v: float) -> int:
    """IEEE-754 single-precision bit pattern of v."""
    return struct.unpack("<I", struct.pack("<f", v))[0]


def amf_key_filename(model_hash: int, tenant_hash: int, prefix_hash: int, n_ctx: int,
                     kv_version: int, rope_base_bits: int, rope_scale_bits: int,
                     sampling_hash: int, rng_hash: int) -> str:
    """The store's entry base name (AmfStore entry_basename(); reference:
    amf_kv_manager.py:118-134)."""
    return (f"amf_{model_hash:016x}_{tenant_hash:016x}_{prefix_hash:016x}"
            f"_{n_ctx}_{kv_version}_{rope_base_bits}_{rope_scale_bits}"
            f"_{sampling_hash:016x}_{rng_hash:016x}")


# --------------------------------------------------------------- manager --


def _kv_planes(layer: torch.Tensor):
    """(K, V) page arrays of a layer: stacked [2, nb, ...] or one array used
    for both (reference: amf_kv_manager.py:302-313)."""
    if layer.dim() == 5 and layer.shape[0] == 2:
        return layer[0], layer[1]
    return layer, layer


class AmfKvManager:
    """AMFK snapshot save / restore of vLLM's GPU KV cache.

    cache_engine: any object with `gpu_cache`, a list of per-layer tensors
    ([2, num_blocks, block_size, H, D] or [num_blocks, block_size, H, D]).
    Other arguments as the reference (amf_kv_manager.py:155-199)."""

    def __init__(self, cache_engine: Any, amf_store_path: str, model_config: Any, *,
                 model_hash: int = 0, tenant_id: str = "__shared__", kv_version: int = 1,
                 rope_base: float = 10000.0, rope_scale: float = 1.0, sampling_hash: int = 0,
                 rng_hash: int = 0) -> None:
        self._cache_engine = cache_engine
        self._store_path = Path(amf_store_path)
        self._model_config = model_config
        self._model_hash = model_hash
        self._tenant_hash = amf_hash_tenant_id(tenant_id)
        self._kv_version = kv_version
        self._rope_base_bits = amf_float_bits(rope_base)
        self._rope_scale_bits = amf_float_bits(rope_scale)
        self._sampling_hash = sampling_hash
        self._rng_hash = rng_hash
        self._store_path.mkdir(parents=True, exist_ok=True)
        self._hits = 0
        self._misses = 0
        self._saves = 0
        self._restore_ms = 0.0
        self._direct: Optional[AmfDirectKv] = None
        self._staging: Optional[torch.Tensor] = None

    # ---------------------------------------------------------- staging --

    def _direct_ctx(self) -> AmfDirectKv:
        if self._direct is None:
            self._direct = AmfDirectKv(0)
        return self._direct

    def _device_staging(self, device, payload_bytes: int, page_bytes: int) -> torch.Tensor:
        """The two-slot device ring, reused while it is large enough and on
        the same device."""
        want = staging_bytes_for(payload_bytes, page_bytes)
        st = self._staging
        if st is None or st.device != device or st.numel() < want:
            self._staging = torch.empty(want, dtype=torch.uint8, device=device)
        return self._staging

    # -------------------------------------------------------------- keys --

    def compute_amf_key(self, prompt_tokens: Sequence[int], n_ctx: Optional[int] = None) -> dict:
        return {
            "model_hash": self._model_hash,
            "tenant_hash": self._tenant_hash,
            "prefix_hash": amf_hash_tokens(prompt_tokens),
            "n_ctx": n_ctx or getattr(self._model_config, "max_model_len", 0),
            "kv_version": self._kv_version,
            "rope_base_bits": self._rope_base_bits,
            "rope_scale_bits": self._rope_scale_bits,
            "sampling_hash": self._sampling_hash,
            "rng_hash": self._rng_hash,
        }

    def _stem(self, key: dict) -> str:
        return amf_key_filename(**key)

    def _kv_filename(self, key: dict) -> Path:
        return self._store_path / (self._stem(key) + ".kv")

    def _tok_filename(self, key: dict) -> Path:
        return self._store_path / (self._stem(key) + ".tok")

    def has_snapshot(self, prompt_tokens: Sequence[int]) -> bool:
        return self._kv_filename(self.compute_amf_key(prompt_tokens)).exists()

    # -------------------------------------------------------------- save --

    def save_kv_state(self, prompt_tokens: Sequence[int], block_table: List[int], *,
                      saved_ms: float = 0.0) -> bool:
        """Write the snapshot of `block_table`'s pages (every page when the
        table is empty) of every layer; True on success."""
        t0 = time.monotonic()
        key = self.compute_amf_key(prompt_tokens)
        kv_path = self._kv_filename(key)
        gpu_cache = self._cache_engine.gpu_cache
        n_layers = len(gpu_cache)
        if n_layers == 0:
            logger.warning("[AMF_VLLM] save: no GPU cache layers")
            return False
        view = _paged.cache_view(gpu_cache)
        amf_hip.require_device_tensor(gpu_cache[0], "AmfKvManager.save_kv_state")
        n_tokens = len(prompt_tokens)
        if block_table:
            _paged.check_block_ids(block_table, view.pool_pages, unique=False)
            n_blocks, ids = len(block_table), list(block_table)
        else:
            n_blocks, ids = view.pool_pages, None
        page_bytes = view.page_bytes
        k0 = _kv_planes(gpu_cache[0])[0]
        staging = self._device_staging(view.device, 2 * n_layers * n_blocks * page_bytes,
                                       page_bytes)
        # the blob: header, layer table, then K and V pages of each layer with KV
        kv_layers = sum(1 for l in range(view.n_layers) if view.planes[2 * l])
        size = (_HEADER_SIZE + _LAYER_SIZE * view.n_layers
                + 2 * kv_layers * n_blocks * page_bytes)
        tmp_path = kv_path.with_suffix(".kv.tmp")
        try:
            out = _SnapshotFile(tmp_path, size)
        except OSError as exc:
            logger.warning("[AMF_VLLM] save: cannot create %s: %s", tmp_path, exc)
            return False
        try:
            try:
                blob = self._direct_ctx().save_pages(
                    view, _paged._device_ids(ids, view.device), n_blocks, staging,
                    tokens=prompt_tokens,
                    n_kv_heads=int(k0.shape[-3]),  # the reference's shape[-3] of the page stack
                    head_dim=int(k0.shape[-1]), dtype_tag=_DTYPE_TAG.get(view.dtype, 0),
                    model_hash=key["model_hash"])
                out.write(blob)
            finally:
                out.close()
            os.replace(tmp_path, kv_path)
        except OSError as exc:
            logger.warning("[AMF_VLLM] save: write failed: %s", exc)
            tmp_path.unlink(missing_ok=True)
            return False
        except BaseException:
            tmp_path.unlink(missing_ok=True)
            raise
        try:
            toks = np.asarray([int(t) for t in prompt_tokens], dtype="<i4")
            self._tok_filename(key).write_bytes(toks.tobytes())
        except OSError as exc:
            logger.warning("[AMF_VLLM] save: tok write failed: %s", exc)
        self._saves += 1
        logger.info("[AMF_VLLM] save: %d layers, %d tokens, %.1f MB in %.0f ms", n_layers,
                    n_tokens, len(blob) / (1 << 20), (time.monotonic() - t0) * 1e3)
        return True

    # ----------------------------------------------------------- restore --

    def restore_kv_state(self, prompt_tokens: Sequence[int], block_table: List[int]) -> int:
        """Load the snapshot of prompt_tokens into the pages `block_table` of
        every layer; the snapshot's token count, or 0 on a miss or an
        incompatible file (reference: amf_kv_manager.py:406-533)."""
        t0 = time.monotonic()
        key = self.compute_amf_key(prompt_tokens)
        kv_path = self._kv_filename(key)
        if not kv_path.exists():
            self._misses += 1
            return 0
        try:
            with open(kv_path, "rb") as f:
                size = os.fstat(f.fileno()).st_size
                if size < _HEADER_SIZE:
                    logger.warning("[AMF_VLLM] restore: blob too small (%d bytes)", size)
                    self._misses += 1
                    return 0
                head = f.read(_HEADER_SIZE)
                (magic, version, n_layers_snap, n_tokens, _heads, _dim, _dtype, _res, _total,
                 _mh, _ph) = struct.unpack_from(_HEADER_FMT, head, 0)
                if magic != _AMFK_MAGIC:
                    logger.warning("[AMF_VLLM] restore: wrong magic 0x%08X (expected AMFK)",
                                   magic)
                    self._misses += 1
                    return 0
                if version != _AMFK_VERSION:
                    logger.warning("[AMF_VLLM] restore: version mismatch (got=%d, want=%d)",
                                   version, _AMFK_VERSION)
                    self._misses += 1
                    return 0
                gpu_cache = self._cache_engine.gpu_cache
                if n_layers_snap != len(gpu_cache):
                    logger.warning("[AMF_VLLM] restore: layer count mismatch (snap=%d, ctx=%d)",
                                   n_layers_snap, len(gpu_cache))
                    self._misses += 1
                    return 0
                if size < _HEADER_SIZE + n_layers_snap * _LAYER_SIZE:
                    logger.warning("[AMF_VLLM] restore: blob truncated (layer table missing)")
                    self._misses += 1
                    return 0
                if block_table:
                    # the whole file into the pinned staging buffer; layer
                    # entries and sizes are validated natively before any copy
                    view = _paged.cache_view(gpu_cache)
                    amf_hip.require_device_tensor(gpu_cache[0], "AmfKvManager.restore_kv_state")
                    _paged.check_block_ids(block_table, view.pool_pages, unique=False)
                    ctx = self._direct_ctx()
                    blob = ctx.staging(size)
                    _read_file_into(f.fileno(), blob, size)
        except OSError as exc:
            logger.warning("[AMF_VLLM] restore: read failed: %s", exc)
            self._misses += 1
            return 0
        if block_table:
            tbl_end = _HEADER_SIZE + n_layers_snap * _LAYER_SIZE
            staging = self._device_staging(view.device, size - tbl_end, view.page_bytes)
            try:
                ctx.restore_pages((ctypes.addressof(ctypes.c_ubyte.from_buffer(blob)), size),
                                  view, _paged._device_ids(block_table, view.device),
                                  len(block_table), staging)
            except amf_hip.AmfHipError as exc:
                if exc.code in (amf_hip.ERR_FORMAT, amf_hip.ERR_MISMATCH):
                    raise ValueError(exc.message) from exc
                raise
        self._hits += 1
        self._restore_ms = (time.monotonic() - t0) * 1e3
        logger.info("[AMF_VLLM] restore: %d layers, %d tokens, %.1f ms", len(gpu_cache),
                    n_tokens, self._restore_ms)
        return int(n_tokens)

    def stats(self) -> dict:
        return {"hits": self._hits, "misses": self._misses, "saves": self._saves,
                "restore_ms": self._restore_ms}


# The name the vLLM integration imports (and the spelling used elsewhere).
AmfKVManager = AmfKvManager

__all__ = [
    "AmfKVManager",
    "AmfKvManager",
    "amf_float_bits",
    "amf_hash_model",
    "amf_hash_tenant_id",
    "amf_hash_tokens",
    "amf_key_filename",
]
