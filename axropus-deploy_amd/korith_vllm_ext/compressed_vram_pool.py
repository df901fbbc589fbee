"""compressed_vram_pool.py - compressed multi-prefix KV residency in HBM.

Same API and bookkeeping as the reference (korith_vllm_ext/
compressed_vram_pool.py:76-892): one byte slab per layer cut into fixed-size
slab blocks, entries keyed by prefix hash, one contiguous span of slab blocks
per (entry, layer), reuse-score eviction, an RLock around the index.

What runs differently on the GPU:

* The slab is the only copy.  put_from_vllm quantizes straight from vLLM's
  paged cache into each layer's span with ONE fused gather+quantize launch for
  all layers (amf_*_quant_gather); restore_to_vllm dequantizes straight from
  the spans into the cache pages with ONE fused dequantize+scatter launch
  (amf_*_dequant_scatter).  The reference gathers with advanced indexing,
  stacks, compresses, keeps the compressed tensors AND copies them into the
  slab (:481-560, 731-757), then decompresses to a temporary and scatters in
  512-block chunks (:562-608).  Entry.blobs here are views of the slab.
* No host synchronisation on save or restore.  The per-tensor FP8 scale the
  reference reads back with float() (amf_codec.py:183) is copied to pinned
  memory asynchronously and resolved when the entry is next looked up.
* Span reuse is stream-ordered: every launch that reads or writes an entry's
  spans records an event; freed spans keep those events and a later
  allocation makes its stream wait on them, so a span is never overwritten
  while a restore on another stream still reads it.
* Already-quantized 1-byte caches (fp8 / int8 / uint8) are stored as raw page
  bytes (format "raw").  The reference switches them to fp8_e4m3, whose
  compress then rejects the 1-byte dtype (amf_codec.py:186-188).

There is no CPU fallback: the pool needs a HIP device and libamf_hip.so.
"""

from __future__ import annotations

import collections.abc
import logging
import math
import threading
import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

import amf_hip

from . import _paged
from .codecs import (
    FMT_FP8_E4M3,
    FMT_FP8_E4M3_PH,
    FMT_INT4_ASYM_G32,
    FMT_INT4_BLOCK,
    FMT_INT4_SYM,
    FMT_RAW,
    CompressedKV,
    get_codec,
)
from .codecs.amf_codec import FP8ScaleSidecar, tensor_scale_from_absmax

logger = logging.getLogger(__name__)

POOL_FORMATS = (FMT_FP8_E4M3, FMT_FP8_E4M3_PH, FMT_INT4_BLOCK, FMT_INT4_SYM, FMT_INT4_ASYM_G32,
                FMT_RAW)


def _is_already_compressed(dtype: torch.dtype) -> bool:
    """1-byte cache dtypes (fp8 / int8 / uint8), stored raw rather than
    quantized again (reference: compressed_vram_pool.py:55-74)."""
    one_byte = {torch.int8, torch.uint8}
    for name in ("float8_e4m3fn", "float8_e5m2", "float8_e4m3fnuz", "float8_e5m2fnuz"):
        if hasattr(torch, name):
            one_byte.add(getattr(torch, name))
    return dtype in one_byte


# --------------------------------------------------------------- records --


@dataclass
class CompressedBlock:
    """One layer's span of an entry (reference: compressed_vram_pool.py:84-99).
    data_offset / scale_offset are byte offsets into the layer slab."""

    layer_id: int
    block_id: int
    format: str
    num_tokens: int
    num_heads: int
    head_dim: int
    data_offset: int
    data_bytes: int
    scale_offset: int
    scale_bytes: int
    tensor_scale: float
    meta: Dict[str, Any] = field(default_factory=dict)
    span_blocks: int = 1


@dataclass
class PoolEntry:
    """A cached prefix: one CompressedBlock and one slab-view CompressedKV per
    layer (reference: compressed_vram_pool.py:102-123)."""

    prefix_hash: str
    num_layers: int
    num_tokens: int
    format: str
    blocks: List[CompressedBlock]
    blobs: Sequence[CompressedKV]  # per layer, built on first access

    created_ns: int = 0
    last_hit_ns: int = 0
    hit_count: int = 0
    avg_savings_ms: float = 0.0
    # launch bookkeeping (not part of the reference record)
    layout: Optional[_paged.BlobLayout] = None
    cache_dtype: Optional[torch.dtype] = None
    # last launch that touched the entry's spans, per stream (stream id -> event)
    fences: Dict[int, torch.cuda.Event] = field(default_factory=dict)
    # per stream id, the fence events that stream has already been ordered
    # after (held, so a later fence is never mistaken for one of them)
    waited: Dict[int, List[torch.cuda.Event]] = field(default_factory=dict)
    pending_absmax: Optional[Tuple[torch.Tensor, torch.cuda.Event]] = None

    def nbytes(self) -> int:
        return sum(b.data_bytes + b.scale_bytes for b in self.blocks)


class _EntryBlobs(collections.abc.Sequence):
    """An entry's per-layer CompressedKV views of its slab spans, each built
    on first access.  The save and restore launches work from the entry's
    blocks and layout, so a save of L layers no longer builds L sets of
    tensor views that only a later caller of entry.blobs reads."""

    __slots__ = ("_make", "_items")

    def __init__(self, n: int, make) -> None:
        self._make = make
        self._items: List[Optional[CompressedKV]] = [None] * n

    def __len__(self) -> int:
        return len(self._items)

    def __getitem__(self, l):
        if isinstance(l, slice):
            return [self[i] for i in range(*l.indices(len(self._items)))]
        n = len(self._items)
        if not -n <= l < n:
            raise IndexError(l)
        l = l % n
        blob = self._items[l]
        if blob is None:
            blob = self._items[l] = self._make(l)
        return blob

    def __setitem__(self, l: int, blob: CompressedKV) -> None:
        self._items[l] = blob

    def built(self, l: int) -> bool:
        return self._items[l] is not None


# ------------------------------------------------------------ allocator --


class _SlabAllocator:
    """First-fit allocator of contiguous slab-block runs of one layer.

    Free space is a sorted list of runs [start, length, fences]; a run's
    fences are the events of the launches that last touched its blocks.
    alloc() returns the lowest-address run start of the requested length (the
    reference's sorted free-list scan, :700-729) together with the fences the
    new user must wait on; free() returns a span with its fence and merges
    neighbours."""

    def __init__(self, n_blocks: int) -> None:
        self.n_blocks = n_blocks
        self._runs: List[List[Any]] = [[0, n_blocks, []]] if n_blocks > 0 else []

    def free_blocks(self) -> int:
        return sum(r[1] for r in self._runs)

    def runs(self) -> List[Tuple[int, int]]:
        return [(r[0], r[1]) for r in self._runs]

    def alloc(self, n: int) -> Optional[Tuple[int, list]]:
        for i, run in enumerate(self._runs):
            start, length, fences = run
            if length >= n:
                if length == n:
                    self._runs.pop(i)
                else:
                    run[0] = start + n
                    run[1] = length - n
                return start, list(fences)
        return None

    def free(self, start: int, n: int, fences: Sequence = ()) -> None:
        fences = _prune(fences) if fences else []
        i = 0
        while i < len(self._runs) and self._runs[i][0] < start:
            i += 1
        prev = self._runs[i - 1] if i > 0 else None
        nxt = self._runs[i] if i < len(self._runs) else None
        if prev is not None and prev[0] + prev[1] > start:
            raise ValueError(f"double free of slab blocks at {start}")
        if nxt is not None and start + n > nxt[0]:
            raise ValueError(f"double free of slab blocks at {start}")
        if prev is not None and prev[0] + prev[1] == start:
            prev[1] += n
            prev[2] = _prune(prev[2] + fences)
            if nxt is not None and prev[0] + prev[1] == nxt[0]:
                prev[1] += nxt[1]
                prev[2] = _prune(prev[2] + nxt[2])
                self._runs.pop(i)
        elif nxt is not None and start + n == nxt[0]:
            nxt[0] = start
            nxt[1] += n
            nxt[2] = _prune(nxt[2] + fences)
        else:
            self._runs.insert(i, [start, n, fences])

    def reset(self, used_prefix: int) -> None:
        """Everything at or after `used_prefix` becomes one free run."""
        fences = _prune([f for r in self._runs for f in r[2]])
        n = self.n_blocks - used_prefix
        self._runs = [[used_prefix, n, fences]] if n > 0 else []


_PRUNE_QUERY_AT = 8  # fences a run may hold before completed ones are queried out


def _prune(fences: list) -> list:
    """Drop duplicates, and once the list is long, events that have completed
    (non-blocking query).  Waiting on a completed event costs nothing, while
    a query is a runtime call per event: short lists are kept as they are."""
    out, seen = [], set()
    for e in fences:
        if e is None or id(e) in seen:
            continue
        seen.add(id(e))
        out.append(e)
    if len(out) >= _PRUNE_QUERY_AT:
        out = [e for e in out if not e.query()]
    return out


# ----------------------------------------------------------------- pool --


class CompressedVRAMPool:
    """Compressed multi-prefix KV pool resident in HBM.

    Args (reference: compressed_vram_pool.py:126-154):
        num_layers:      number of transformer layers (= number of slabs).
        bytes_per_layer: slab bytes per layer.
        block_bytes:     slab block size (allocation unit).
        default_format:  codec used when a call names none (any of
                         POOL_FORMATS except "raw").
        device:          a HIP device ("cuda", "cuda:N"); a CPU device raises.
        reuse_alpha..delta: eviction score weights on age, 1/hits, size and
                         per-hit savings.
    """

    def __init__(
        self,
        num_layers: int,
        bytes_per_layer: int = 1 << 30,
        block_bytes: int = 1 << 17,
        *,
        default_format: str = "int4_sym_block",
        device: "str | torch.device" = "cuda",
        reuse_alpha: float = 0.3,
        reuse_beta: float = 0.4,
        reuse_gamma: float = 0.1,
        reuse_delta: float = 0.2,
    ) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(
                "CompressedVRAMPool keeps its slabs in GPU memory and runs its codecs through "
                f"libamf_hip.so; device {device} is not a HIP device")
        if not torch.cuda.is_available():
            raise amf_hip.AmfHipUnavailable("CompressedVRAMPool needs a HIP device")
        amf_hip.load()
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if default_format not in POOL_FORMATS or default_format == FMT_RAW:
            get_codec(default_format)  # KeyError for unknown names, as the reference
            raise KeyError(f"format {default_format!r} has no pool kernel")
        if block_bytes <= 0 or block_bytes % 256:
            raise ValueError("block_bytes must be a positive multiple of 256")
        self.num_layers = num_layers
        self.bytes_per_layer = bytes_per_layer
        self.block_bytes = block_bytes
        self.default_format = default_format
        self.device = device

        self._blocks_per_layer = bytes_per_layer // block_bytes
        self._slabs: List[torch.Tensor] = [
            torch.empty(self._blocks_per_layer * block_bytes, dtype=torch.uint8, device=device)
            for _ in range(num_layers)
        ]
        # slab base addresses (slabs never move), read on every launch
        self._slab_ptr: List[int] = [t.data_ptr() for t in self._slabs]
        self._alloc = [_SlabAllocator(self._blocks_per_layer) for _ in range(num_layers)]

        self._index: Dict[str, PoolEntry] = {}
        self._lock = threading.RLock()
        self._alpha, self._beta = reuse_alpha, reuse_beta
        self._gamma, self._delta = reuse_gamma, reuse_delta

        self._stat_hits = 0
        self._stat_misses = 0
        self._stat_inserts = 0
        self._stat_evictions = 0
        self._stat_bytes_stored = 0
        self._stat_bytes_evicted = 0
        logger.info("CompressedVRAMPool: layers=%d slab=%.2f GiB blocks=%d device=%s",
                    num_layers, bytes_per_layer / (1 << 30), self._blocks_per_layer, device)

    # ---------------------------------------------------------- queries --

    def __len__(self) -> int:
        with self._lock:
            return len(self._index)

    def __contains__(self, prefix_hash: str) -> bool:
        with self._lock:
            return prefix_hash in self._index

    def capacity_bytes(self) -> int:
        return self.num_layers * self.bytes_per_layer

    def used_bytes(self) -> int:
        with self._lock:
            return sum(e.nbytes() for e in self._index.values())

    def num_prefixes(self) -> int:
        return len(self._index)

    def stats(self) -> Dict[str, Any]:
        with self._lock:
            return {
                "hits": self._stat_hits,
                "misses": self._stat_misses,
                "inserts": self._stat_inserts,
                "evictions": self._stat_evictions,
                "bytes_stored": self._stat_bytes_stored,
                "bytes_evicted": self._stat_bytes_evicted,
                "num_prefixes": self.num_prefixes(),
                "used_bytes": self.used_bytes(),
                "capacity_bytes": self.capacity_bytes(),
            }

    def get(self, prefix_hash: str) -> Optional[PoolEntry]:
        """Look up a prefix; a hit updates its recency and hit count."""
        with self._lock:
            entry = self._index.get(prefix_hash)
            if entry is None or not self._resolve_scales(entry):
                self._stat_misses += 1
                return None
            entry.last_hit_ns = time.monotonic_ns()
            entry.hit_count += 1
            self._stat_hits += 1
            return entry

    # ------------------------------------------------------- vLLM paths --

    def put_from_vllm(self, prefix_hash: str, gpu_cache: list, block_table: List[int],
                      n_tokens: int, *, format: Optional[str] = None,
                      savings_ms: float = 0.0) -> bool:
        """Save the pages `block_table` of every layer of vLLM's cache
        (per-layer [2, num_blocks, block_size, H, D] or [num_blocks,
        block_size, H, D]) in `format`; False if no room after eviction
        (reference: compressed_vram_pool.py:434-560)."""
        fmt = format or self.default_format
        if len(gpu_cache) == 0 or len(block_table) == 0:
            return False
        view = _paged.cache_view(gpu_cache)
        self._check_device(view.device)
        _paged.check_block_ids(block_table, view.pool_pages, unique=False)
        if _is_already_compressed(view.dtype):
            fmt = FMT_RAW
        layout = self._layout(fmt, len(block_table), view.block_size, view.num_heads,
                              view.head_dim, view.dtype)
        shape = (2, len(block_table), view.block_size, view.num_heads, view.head_dim)
        return self._insert(prefix_hash, fmt, layout, view, block_table, n_tokens, shape,
                            view.dtype, savings_ms)

    def restore_to_vllm(self, prefix_hash: str, gpu_cache: list, block_table: List[int]) -> int:
        """Write the entry's pages into vLLM's cache pages `block_table` (the
        first min(len(block_table), saved pages) of them, for the first
        min(len(gpu_cache), saved layers) layers); returns the saved token
        count, 0 on a miss (reference: compressed_vram_pool.py:562-608)."""
        entry = self.get(prefix_hash)
        if entry is None:
            return 0
        with self._lock:
            layers = min(len(gpu_cache), entry.num_layers)
            if layers == 0:
                return entry.num_tokens
            view = _paged.cache_view(gpu_cache[:layers])
            self._check_device(view.device)
            lay = entry.layout
            if (view.block_size, view.num_heads, view.head_dim) != \
                    (lay.block_size, lay.num_heads, lay.head_dim):
                raise ValueError(
                    f"cache pages [{view.block_size}, {view.num_heads}, {view.head_dim}] do not "
                    f"match the entry's [{lay.block_size}, {lay.num_heads}, {lay.head_dim}]")
            n = min(len(block_table), lay.n_pages)
            if n > 0:
                ids = list(block_table[:n])
                _paged.check_block_ids(ids, view.pool_pages, unique=False)
                if entry.format == FMT_RAW and view.dtype.itemsize != lay.elem_bytes:
                    raise ValueError(f"raw entry of {lay.elem_bytes}-byte elements cannot fill a "
                                     f"{view.dtype} cache")
                bases = [self._slab_ptr[b.layer_id] + b.data_offset
                         for b in entry.blocks[:layers]]
                self._wait(entry)
                if entry.format == FMT_RAW:
                    ins = [base + lay.code_offset(p) for base in bases for p in range(2)]
                    _paged.scatter_pages(ins, lay.code_bytes_per_page, view, ids, n)
                else:
                    _paged.dequant_scatter(lay, bases, 2, view, ids, n_pages=n)
                self._fence(entry)
            return entry.num_tokens

    # -------------------------------------------------------- raw paths --

    def put_from_raw(self, prefix_hash: str, raw_kv: torch.Tensor, *,
                     format: Optional[str] = None, savings_ms: float = 0.0) -> bool:
        """Insert a dense KV tensor: [L, 2, T, H, D], [L, 2, nb, bs, H, D]
        (read as T = nb*bs) or [nb, bs, H, D] (one layer, K = V).  Each layer
        [2, T, H, D] is compressed as the format's codec compresses it.
        False if no room after eviction; ValueError on other shapes
        (reference: compressed_vram_pool.py:255-377)."""
        fmt = format or self.default_format
        x = raw_kv
        if x.dim() == 5 and x.shape[1] == 2:
            pass
        elif x.dim() == 6 and x.shape[1] == 2:
            L, _, nb, bs, H, D = x.shape
            x = x.reshape(L, 2, nb * bs, H, D)
        elif x.dim() == 4:
            nb, bs, H, D = x.shape
            one = x.reshape(1, nb * bs, H, D)
            x = torch.stack([one, one], dim=1)
        else:
            raise ValueError(
                f"put_from_raw: unsupported shape {tuple(raw_kv.shape)}. "
                "Expected [L,2,T,H,D], [L,2,nb,bs,H,D], or [nb,bs,H,D].")
        if x.device != self.device:
            x = x.to(self.device)
        if _is_already_compressed(x.dtype):
            fmt = FMT_RAW
        L, _, T, H, D = x.shape
        if L > self.num_layers:
            raise ValueError(f"{L} layers exceed the pool's {self.num_layers}")
        page = self._dense_page(fmt, T)
        n_pages = max(1, -(-T // page))
        Tp = n_pages * page
        x = x.contiguous()
        if Tp != T:
            pad = torch.zeros(L, 2, Tp, H, D, dtype=x.dtype, device=x.device)
            pad[:, :, :T].copy_(x)
            x = pad
        view = _paged.planes_view([x[l, kv].view(n_pages, page, H, D)
                                   for l in range(L) for kv in range(2)])
        layout = self._layout(fmt, n_pages, page, H, D, x.dtype)
        return self._insert(prefix_hash, fmt, layout, view, None, T, (2, T, H, D), raw_kv.dtype,
                            savings_ms, keep=x)

    def _dense_page(self, fmt: str, T: int) -> int:
        """Tokens per page of a dense [2, T, H, D] layer entry in `fmt`."""
        if fmt == FMT_RAW:
            return 16 if T % 16 == 0 else T
        if fmt not in POOL_FORMATS:
            get_codec(fmt)
            raise KeyError(f"format {fmt!r} has no pool kernel")
        return get_codec(fmt)._page_tokens(T)

    def promote_from_raw(self, prefix_hash: str, raw_kv: torch.Tensor, *,
                         format: Optional[str] = None) -> bool:
        """Alias of put_from_raw (reference: compressed_vram_pool.py:420-428)."""
        return self.put_from_raw(prefix_hash, raw_kv, format=format)

    def restore_to_tensor(self, prefix_hash: str,
                          target_dtype: torch.dtype = torch.float16) -> Optional[torch.Tensor]:
        """The entry decompressed to [num_layers, *layer shape] in target_dtype,
        or None on a miss (reference: compressed_vram_pool.py:379-398)."""
        entry = self.get(prefix_hash)
        if entry is None:
            return None
        with self._lock:
            lay = entry.layout
            L = entry.num_layers
            bases = [self._slab_ptr[b.layer_id] + b.data_offset for b in entry.blocks]
            shape = tuple(entry.blobs[0].shape)
            T = entry.blobs[0].meta["n_tokens"]
            self._wait(entry)
            if entry.format == FMT_RAW:
                out = torch.empty(L, 2, lay.n_pages, lay.block_size, lay.num_heads, lay.head_dim,
                                  dtype=entry.cache_dtype, device=self.device)
                ins = [base + lay.code_offset(p) for base in bases for p in range(2)]
                view = _paged.planes_view([out[l, kv] for l in range(L) for kv in range(2)])
                _paged.scatter_pages(ins, lay.code_bytes_per_page, view, None, lay.n_pages)
            else:
                out = torch.empty(L, 2, lay.n_pages, lay.block_size, lay.num_heads, lay.head_dim,
                                  dtype=target_dtype, device=self.device)
                view = _paged.planes_view([out[l, kv] for l in range(L) for kv in range(2)])
                _paged.dequant_scatter(lay, bases, 2, view, None)
            self._fence(entry)
        flat = out.view(L, 2, lay.n_pages * lay.block_size, lay.num_heads, lay.head_dim)
        res = flat[:, :, :T].reshape(L, *shape)
        return res.to(target_dtype) if res.dtype != target_dtype else res

    # ------------------------------------------------- token-slot paths --

    def put_from_slots(self, prefix_hash: str, gpu_cache: list, slot_mapping, *,
                       format: Optional[str] = None, savings_ms: float = 0.0) -> bool:
        """Save the token rows `slot_mapping` (slot = block * block_size +
        offset) of every layer of vLLM's cache as a dense [L, 2, T, H, D]
        entry, T = len(slot_mapping): the entry put_from_raw makes from
        stack([flat(layer)[:, slots] for layer]), which is what the
        connector's save_kv_layer + wait_for_save store (reference:
        amf_kv_connector.py:411-422, 446-483).

        Slots that come in aligned runs as long as the format's dense pages
        (whole vLLM blocks of that length, or of any multiple of it when the
        cache's pages are unpadded) are quantized straight from the cache (one
        launch for all layers); any other mapping is first gathered into a
        dense buffer by the slot kernel."""
        fmt = format or self.default_format
        if len(gpu_cache) == 0:
            return False
        view = _paged.cache_view(gpu_cache)
        self._check_device(view.device)
        slots = _paged.SlotMap.of(slot_mapping)
        T = slots.n
        if T == 0:
            return False
        slots.check(view.pool_pages * view.block_size)
        if _is_already_compressed(view.dtype):
            fmt = FMT_RAW
        L, H, D = view.n_layers, view.num_heads, view.head_dim
        if L > self.num_layers:
            raise ValueError(f"{L} layers exceed the pool's {self.num_layers}")
        page = self._dense_page(fmt, T)
        pview = _paged.token_pages(view, page)
        ids = slots.page_ids_on(T, page, view.device) if pview is not None else None
        if ids is not None:
            layout = self._layout(fmt, T // page, page, H, D, view.dtype)
            return self._insert(prefix_hash, fmt, layout, pview, ids, T, (2, T, H, D),
                                view.dtype, savings_ms)
        staging = torch.empty(L, 2, T, H, D, dtype=view.dtype, device=view.device)
        outs = [staging[l, kv].data_ptr() for l in range(L) for kv in range(2)]
        _paged.gather_slots(view, slots, T, outs, H * D * staging.element_size())
        return self.put_from_raw(prefix_hash, staging, format=fmt, savings_ms=savings_ms)

    def restore_to_slots(self, prefix_hash: str, gpu_cache: list, slot_mapping, *,
                         first_layer: int = 0) -> int:
        """restore_entry_to_slots for the entry under prefix_hash; returns its
        token count, 0 on a miss."""
        entry = self.get(prefix_hash)
        if entry is None:
            return 0
        self.restore_entry_to_slots(entry, gpu_cache, slot_mapping, first_layer=first_layer)
        return entry.num_tokens

    def restore_entry_to_slots(self, entry: PoolEntry, gpu_cache: list, slot_mapping, *,
                               first_layer: int = 0) -> int:
        """Write layers first_layer .. first_layer + len(gpu_cache) - 1 of
        `entry` into the token rows `slot_mapping` of the caches gpu_cache
        (flat(cache)[:, slots[:n]] = decompress(blob)[:, :n] with n = min(entry
        tokens, len(slots)); reference: amf_kv_connector.py:345-385).  Returns
        n, or 0 when the entry has left the pool.

        Slots in aligned runs as long as the entry's pages are written by the
        codec kernel straight into the cache; otherwise the layers are
        decompressed into a dense buffer and moved by the slot kernel (a raw
        entry is moved by the slot kernel directly)."""
        with self._lock:
            if self._index.get(entry.prefix_hash) is not entry:
                return 0
            layers = min(len(gpu_cache), entry.num_layers - first_layer)
            if first_layer < 0 or layers <= 0:
                return 0
            view = _paged.cache_view(gpu_cache[:layers])
            self._check_device(view.device)
            lay = entry.layout
            H, D = lay.num_heads, lay.head_dim
            if (view.num_heads, view.head_dim) != (H, D):
                raise ValueError(f"cache rows [{view.num_heads}, {view.head_dim}] do not match "
                                 f"the entry's [{H}, {D}]")
            if entry.format == FMT_RAW and view.dtype.itemsize != lay.elem_bytes:
                raise ValueError(f"raw entry of {lay.elem_bytes}-byte elements cannot fill a "
                                 f"{view.dtype} cache")
            slots = _paged.SlotMap.of(slot_mapping)
            T = entry.blobs[0].meta["n_tokens"]
            n = min(T, slots.n)
            if n == 0:
                return 0
            slots.check(view.pool_pages * view.block_size, n)
            bases = [self._slab_ptr[b.layer_id] + b.data_offset
                     for b in entry.blocks[first_layer:first_layer + layers]]
            P = lay.block_size
            row = H * D * view.dtype.itemsize
            self._wait(entry)
            pview = _paged.token_pages(view, P)
            ids = slots.page_ids_on(n, P, view.device) if pview is not None else None
            if ids is not None and entry.format == FMT_RAW:
                ins = [base + lay.code_offset(p) for base in bases for p in range(2)]
                _paged.scatter_pages(ins, lay.code_bytes_per_page, pview, ids, n // P)
            elif ids is not None:
                _paged.dequant_scatter(lay, bases, 2, pview, ids, n_pages=n // P)
            elif entry.format == FMT_RAW:
                ins = [base + lay.code_offset(p) for base in bases for p in range(2)]
                _paged.scatter_slots(ins, row, view, slots, n)
            else:
                pages = -(-n // P)
                staging = torch.empty(2 * layers, pages, P, H, D, dtype=view.dtype,
                                      device=view.device)
                planes = [staging[i] for i in range(2 * layers)]
                _paged.dequant_scatter(lay, bases, 2, _paged.planes_view(planes), None,
                                       n_pages=pages)
                _paged.scatter_slots([t.data_ptr() for t in planes], row, view, slots, n)
            self._fence(entry)
            return n

    def delete(self, prefix_hash: str) -> bool:
        with self._lock:
            entry = self._index.pop(prefix_hash, None)
            if entry is None:
                return False
            self._release_entry(entry)
            return True

    def clear(self) -> None:
        with self._lock:
            for entry in list(self._index.values()):
                self._release_entry(entry)
            self._index.clear()

    # --------------------------------------------------------- internals --

    def _check_device(self, dev: torch.device) -> None:
        if dev != self.device:
            raise ValueError(f"KV cache on {dev}, pool on {self.device}")

    def _layout(self, fmt: str, n_pages: int, bs: int, H: int, D: int,
                dtype: torch.dtype) -> _paged.BlobLayout:
        if fmt == FMT_RAW:
            lay = _paged.BlobLayout(FMT_RAW, 2, n_pages, bs, H, D, dtype.itemsize)
        else:
            if fmt not in POOL_FORMATS:
                get_codec(fmt)
                raise KeyError(f"format {fmt!r} has no pool kernel")
            if dtype not in (torch.float16, torch.bfloat16, torch.float32):
                raise TypeError(f"{fmt} cannot accept dtype {dtype}")
            lay = _paged.BlobLayout(fmt, 2, n_pages, bs, H, D)
        lay.validate()
        return lay

    def _blocks_for(self, layout: _paged.BlobLayout) -> int:
        return max(1, math.ceil(layout.total_bytes / self.block_bytes))

    def _insert(self, prefix_hash, fmt, layout, view, block_ids, n_tokens, shape, dtype,
                savings_ms, keep=None) -> bool:
        L = len(view.planes) // 2
        need = self._blocks_for(layout)
        with self._lock:
            if prefix_hash in self._index:
                self._release_entry(self._index.pop(prefix_hash))
            spans = self._allocate(L, need)
            if spans is None:
                logger.warning("CompressedVRAMPool: no room for %s (%d x %d slab blocks, %s)",
                               prefix_hash[:12], L, need, fmt)
                return False
            # the layers' spans mostly carry the same events: wait once each
            stream = torch.cuda.current_stream(self.device)
            seen = set()
            for _, fences in spans:
                for ev in fences:
                    if id(ev) not in seen:
                        seen.add(id(ev))
                        stream.wait_event(ev)
            bases = [self._slab_ptr[l] + start * self.block_bytes
                     for l, (start, _) in enumerate(spans)]
            pending = None
            if fmt == FMT_RAW:
                outs = [b + layout.code_offset(p) for b in bases for p in range(2)]
                _paged.gather_pages(view, block_ids, outs, layout.code_bytes_per_page,
                                    layout.n_pages)
            else:
                ws = _paged.quant_gather(layout, view, block_ids, bases, 2)
                if fmt == FMT_FP8_E4M3:
                    host = torch.empty(L, dtype=torch.int32, pin_memory=True)
                    host.copy_(ws[:L].view(torch.int32), non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(torch.cuda.current_stream(self.device))
                    pending = (host, ev)
            codec = None if fmt == FMT_RAW else get_codec(fmt)
            T = shape[1] * shape[2] if len(shape) == 5 else shape[1]  # tokens per plane
            # tensor_scale: 1.0 for every format but per-tensor FP8, whose
            # scale arrives with pending_absmax (0.0 until then)
            scale0 = 0.0 if pending is not None else 1.0
            blocks = [CompressedBlock(
                layer_id=l, block_id=start, format=fmt, num_tokens=n_tokens,
                num_heads=layout.num_heads, head_dim=layout.head_dim,
                data_offset=start * self.block_bytes, data_bytes=layout.data_bytes,
                scale_offset=start * self.block_bytes + layout.scale_offset,
                scale_bytes=layout.scale_bytes, tensor_scale=scale0,
                meta={"_layout": layout, "n_tokens": T}, span_blocks=need)
                for l, (start, _) in enumerate(spans)]
            slabs = self._slabs

            def make_blob(l: int) -> CompressedKV:
                # Reads the block's current offset (compaction moves spans)
                # and scale; the blob shares the block's meta dict.
                blk = blocks[l]
                if codec is None:
                    data = slabs[l].narrow(0, blk.data_offset, layout.data_bytes).view(dtype)
                    return CompressedKV(format=FMT_RAW, data=data.view(shape), scales=None,
                                        tensor_scale=1.0, shape=shape, dtype_original=dtype,
                                        meta=blk.meta)
                blob = codec.wrap_blob(slabs[l], blk.data_offset, layout, shape, dtype, None, T,
                                       scale=blk.tensor_scale if fmt == FMT_FP8_E4M3 else None)
                blk.meta.update(blob.meta)
                blob.meta = blk.meta
                return blob

            # (per-tensor FP8 entries always carry pending_absmax here, so
            # blk.tensor_scale is 0.0 until resolved, then the scale)
            blobs = _EntryBlobs(L, make_blob)
            now = time.monotonic_ns()
            entry = PoolEntry(prefix_hash=prefix_hash, num_layers=L, num_tokens=n_tokens,
                              format=fmt, blocks=blocks, blobs=blobs, created_ns=now,
                              last_hit_ns=now, hit_count=0, avg_savings_ms=savings_ms,
                              layout=layout, cache_dtype=dtype, pending_absmax=pending)
            self._fence(entry)
            self._index[prefix_hash] = entry
            self._stat_inserts += 1
            self._stat_bytes_stored += entry.nbytes()
            return True

    def _resolve_scales(self, entry: PoolEntry) -> bool:
        """Per-tensor FP8: turn the asynchronously copied absmax into the
        reference's Python-double tensor_scale and FP8ScaleSidecar.

        A non-finite layer absmax means the save failed (the single-read
        kernel writes +inf for a scale group whose cross-workgroup wait gave
        up, and a cache holding inf has no usable FP8 scale either): the
        entry is dropped and its spans freed, and False is returned so that
        the lookup is a miss instead of a restore of inf/NaN pages."""
        if entry.pending_absmax is None:
            return True
        host, ev = entry.pending_absmax
        ev.synchronize()
        vals = host.view(torch.float32).tolist()
        if not all(math.isfinite(v) for v in vals):
            logger.warning("CompressedVRAMPool: per-tensor FP8 save of %s failed (non-finite "
                           "absmax in layer %d); entry dropped", entry.prefix_hash[:12],
                           next(l for l, v in enumerate(vals) if not math.isfinite(v)))
            entry.pending_absmax = None
            if self._index.get(entry.prefix_hash) is entry:
                self._index.pop(entry.prefix_hash)
            self._release_entry(entry)
            return False
        blobs = entry.blobs
        for l, blk in enumerate(entry.blocks):
            scale = tensor_scale_from_absmax(vals[l], entry.cache_dtype)
            blk.tensor_scale = scale
            # blk.meta is the blob's meta once the blob exists
            blk.meta["sidecar"] = FP8ScaleSidecar(k_scale=scale, v_scale=scale)
            if not isinstance(blobs, _EntryBlobs) or blobs.built(l):
                blobs[l].tensor_scale = scale
        entry.pending_absmax = None
        return True

    def _fence(self, entry: PoolEntry) -> None:
        """Record the current stream's last launch on the entry's spans (one
        event per stream, so restores queued on several streams all hold the
        spans until they finish)."""
        stream = torch.cuda.current_stream(self.device)
        ev = torch.cuda.Event()
        ev.record(stream)
        entry.fences[int(stream.cuda_stream)] = ev

    def _wait(self, entry: PoolEntry) -> None:
        """Order this stream after the entry's launches on other streams (its
        save may have run elsewhere)."""
        sid = amf_hip.stream_handle(self.device)
        done = entry.waited.get(sid, ())
        others = [ev for s, ev in entry.fences.items()
                  if s != sid and not any(ev is d for d in done)]
        if others:
            stream = torch.cuda.current_stream(self.device)
            for ev in others:
                stream.wait_event(ev)
            entry.waited[sid] = [ev for s, ev in entry.fences.items() if s != sid]

    def _allocate(self, L: int, need: int) -> Optional[List[Tuple[int, list]]]:
        """One span of `need` slab blocks on each of the first L layers,
        evicting by reuse score while a layer has no room; on failure every
        span taken so far is returned (reference: compressed_vram_pool.py:
        664-698)."""
        spans: List[Tuple[int, list]] = []
        for l in range(L):
            got = self._alloc[l].alloc(need)
            while got is None:
                if not self._evict_one():
                    for rl, (start, fences) in enumerate(spans):
                        self._alloc[rl].free(start, need, fences)
                    return None
                got = self._alloc[l].alloc(need)
            spans.append(got)
        return spans

    def _reuse_score(self, entry: PoolEntry) -> float:
        """Eviction score, higher = evicted first (reference: :612-626)."""
        age_s = max(0.0, (time.monotonic_ns() - entry.last_hit_ns) / 1e9)
        hits = max(1, entry.hit_count)
        size_mb = entry.nbytes() / (1 << 20)
        savings = max(0.0, entry.avg_savings_ms)
        return (self._alpha * age_s + self._beta / hits + self._gamma * size_mb
                - self._delta * savings)

    def _evict_one(self) -> bool:
        if not self._index:
            return False
        worst = max(self._index, key=lambda h: self._reuse_score(self._index[h]))
        entry = self._index.pop(worst)
        nbytes = entry.nbytes()
        self._release_entry(entry)
        self._stat_evictions += 1
        self._stat_bytes_evicted += nbytes
        logger.debug("CompressedVRAMPool evicted %s (%d bytes)", worst[:12], nbytes)
        return True

    def _release_entry(self, entry: PoolEntry) -> None:
        fences = _prune(list(entry.fences.values()))
        for b in entry.blocks:
            self._alloc[b.layer_id].free(b.block_id, b.span_blocks, fences)

    def _allocate_with_compaction(self, L: int, need: int):
        """Allocation with slab compaction as the last resort (reference:
        :764-783)."""
        spans = self._allocate(L, need)
        if spans is not None:
            return spans
        self._compact_slabs()
        return self._allocate(L, need)

    def _compact_slabs(self) -> None:
        """Move every live span to the front of its slab (stream-ordered device
        copies) and rebuild the entries' slab views (reference: :785-819)."""
        with self._lock:
            stream = torch.cuda.current_stream(self.device)
            for entry in self._index.values():
                self._wait(entry)
            # Free runs keep the fences of the entries released into them (a
            # restore of an evicted entry may still be reading there on a
            # side stream): the copies below overwrite free space, so they
            # wait for those launches too.
            for alloc in self._alloc:
                for _, _, fences in alloc._runs:
                    for ev in fences:
                        stream.wait_event(ev)
            for l in range(self.num_layers):
                live = sorted((b.block_id, b, e) for e in self._index.values()
                              for b in e.blocks if b.layer_id == l)
                nxt = 0
                for _, blk, entry in live:
                    if blk.block_id != nxt:
                        src = self._slabs[l].narrow(0, blk.block_id * self.block_bytes,
                                                    blk.span_blocks * self.block_bytes).clone()
                        self._slabs[l].narrow(0, nxt * self.block_bytes, src.numel()).copy_(src)
                        blk.block_id = nxt
                        blk.data_offset = nxt * self.block_bytes
                        blk.scale_offset = blk.data_offset + entry.layout.scale_offset
                        self._rewrap(entry, blk)
                    nxt += blk.span_blocks
                self._alloc[l].reset(nxt)
            for entry in self._index.values():
                ev = torch.cuda.Event()
                ev.record(stream)
                entry.fences = {int(stream.cuda_stream): ev}

    def _rewrap(self, entry: PoolEntry, blk: CompressedBlock) -> None:
        if isinstance(entry.blobs, _EntryBlobs) and not entry.blobs.built(blk.layer_id):
            return  # built later from the block's new offset
        old = entry.blobs[blk.layer_id]
        if entry.format == FMT_RAW:
            data = self._slabs[blk.layer_id].narrow(0, blk.data_offset, blk.data_bytes)
            old.data = data.view(entry.cache_dtype).view(old.shape)
            return
        codec = get_codec(entry.format)
        new = codec.wrap_blob(self._slabs[blk.layer_id], blk.data_offset, entry.layout, old.shape,
                              entry.cache_dtype, None, old.meta["n_tokens"],
                              scale=old.tensor_scale)
        new.tensor_scale = old.tensor_scale
        if "sidecar" in old.meta:
            new.meta["sidecar"] = old.meta["sidecar"]
        entry.blobs[blk.layer_id] = new
        blk.meta = new.meta

    # -------------------------------------------------- vLLM block table --

    def map_into_vllm(self, prefix_hash: str, vllm_seq_id: int, vllm_block_table: Any) -> bool:
        """Write one opaque external reference per layer span into
        vllm_block_table[vllm_seq_id] (reference: :823-866)."""
        entry = self._index.get(prefix_hash)
        if entry is None:
            return False
        try:
            table = vllm_block_table[vllm_seq_id]
            for idx, block in enumerate(entry.blocks):
                ref = _ExternalBlockRef(block)
                if idx < len(table):
                    table[idx] = ref
                else:
                    table.append(ref)
            return True
        except Exception as exc:  # duck-typed vLLM structure
            logger.warning("map_into_vllm: seq=%s: %s", vllm_seq_id, exc)
            return False


@dataclass
class _ExternalBlockRef:
    """Opaque reference to a pool span for vLLM's block table; is_external
    tells the allocator to leave it alone (reference: :869-886)."""

    block: CompressedBlock
    is_external: bool = True

    def __repr__(self) -> str:
        return (f"<ExternalBlockRef layer={self.block.layer_id} block={self.block.block_id} "
                f"fmt={self.block.format}>")


__all__ = ["CompressedBlock", "CompressedVRAMPool", "PoolEntry", "POOL_FORMATS"]
