"""amf_kv_connector.py - the AMF pool as a vLLM v1 KV connector.

Mirrors korith_vllm_ext/amf_kv_connector.py of the reference (a
KVConnectorBase_V1 for vLLM v0.19): on a cold prefill, save_kv_layer notes
each layer's KV and wait_for_save stores the request's prefix in the
CompressedVRAMPool; on a warm hit, start_load_kv writes the pool entry into
vLLM's paged buffer at the request's slots.

    LLM(model=..., kv_transfer_config={
        "kv_connector": "AMFKVConnector",
        "kv_connector_module_path": "korith_vllm_ext.amf_kv_connector",
        "kv_role": "kv_both",
        "kv_connector_extra_config": {"num_layers": 28, "num_kv_heads": 2, "head_dim": 64,
                                      "bytes_per_layer": 8388608,
                                      "default_format": "fp8_e4m3",
                                      "min_prefix_tokens": 64}})

Device work (the reference runs codec.decompress_to + flat_cache[:, slots] =
kv per request and layer, and flat[:, slots].clone() + torch.stack +
put_from_raw on save):

* save: save_kv_layer keeps a reference to the layer's cache (no copy);
  wait_for_save stores each prefix with CompressedVRAMPool.put_from_slots,
  which quantizes the request's pages of every layer in one launch (or
  gathers unordered slots with the slot kernel first).  The entry is the
  one the reference's stack + put_from_raw makes.
* load: start_load_kv queues the restore of every hit request into its
  slots on a load stream, in launches of 1, 1, 2, 4, 8, ... consecutive
  layers, each followed by an event; wait_for_layer_load(layer) makes the
  forward's stream wait for its launch's event only, so layer l's attention
  runs while later layers are still being restored.  extra_config "load_stream": "current" queues the loads
  on the forward's own stream instead (the reference's ordering).

The scheduler-side logic (prefix hash, block alignment, metadata) follows
the reference line for line in behaviour, including its quirks:
align_to_block_size(n, bs) is (n - 1) // bs * bs (it drops a whole block
when n is a multiple of bs), the hash covers align_to_block_size(len - 1)
tokens while a request's slots cover align_to_block_size(len) tokens, and
the scheduler's pool only answers membership for entries of its own
process.

With vLLM installed the connector derives from vLLM's KVConnectorBase_V1;
without it, from a local class with the same metadata hooks, so the
connector can be driven directly (tests, embedding without vLLM).
"""

from __future__ import annotations

import enum
import hashlib
import logging
import weakref
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, Any, Dict, List, Optional, Tuple

import numpy as np
import torch

import amf_hip

from ._paged import SlotMap

try:
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (
        KVConnectorBase_V1,
        KVConnectorMetadata,
        KVConnectorRole,
    )
except ImportError:  # vLLM is an optional dependency of this module

    class KVConnectorRole(enum.Enum):
        SCHEDULER = 0
        WORKER = 1

    class KVConnectorMetadata:
        """Per-step metadata the scheduler hands the workers."""

    class KVConnectorBase_V1:
        """The part of vLLM's KVConnectorBase_V1 the connector relies on."""

        def __init__(self, vllm_config: Any, role: KVConnectorRole,
                     kv_cache_config: Any = None) -> None:
            self._connector_metadata: Optional[KVConnectorMetadata] = None
            self._vllm_config = vllm_config
            self._kv_transfer_config = getattr(vllm_config, "kv_transfer_config", None)
            if self._kv_transfer_config is None:
                raise ValueError("kv_transfer_config must be set for KVConnectorBase_V1")
            self._kv_cache_config = kv_cache_config
            self._role = role

        @property
        def role(self) -> KVConnectorRole:
            return self._role

        def bind_connector_metadata(self, connector_metadata: KVConnectorMetadata) -> None:
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self) -> None:
            self._connector_metadata = None

        def has_connector_metadata(self) -> bool:
            return self._connector_metadata is not None

        def _get_connector_metadata(self) -> KVConnectorMetadata:
            assert self._connector_metadata is not None
            return self._connector_metadata

        def register_kv_caches(self, kv_caches: Dict[str, torch.Tensor]) -> None:
            return

        def get_finished(self, finished_req_ids) -> Tuple[Optional[set], Optional[set]]:
            return None, None

        def get_block_ids_with_load_errors(self) -> set:
            return set()

        def request_finished(self, request: Any, block_ids: List[int]):
            return False, None


if TYPE_CHECKING:  # pragma: no cover
    from .compressed_vram_pool import CompressedVRAMPool

logger = logging.getLogger("amf_kv_connector")


# ------------------------------------------------------------------ helpers --


def _token_words(token_ids) -> bytes:
    """The tokens mod 2**32 as consecutive 4-byte little-endian words."""
    try:
        a = np.asarray(token_ids, dtype=np.int64)
    except (OverflowError, TypeError, ValueError):
        return b"".join(int(t & 0xFFFFFFFF).to_bytes(4, "little") for t in token_ids)
    return (a & 0xFFFFFFFF).astype("<u4").tobytes()


def _prefix_hash(token_ids) -> str:
    """First 16 hex digits of SHA-256 over the tokens as 4-byte little-endian
    words (reference: amf_kv_connector.py:64-69, which feeds the words one
    update at a time; the digest of the concatenation is the same)."""
    return hashlib.sha256(_token_words(token_ids)).hexdigest()[:16]


def align_to_block_size(num_tokens: int, block_size: int) -> int:
    """(num_tokens - 1) // block_size * block_size (reference:
    amf_kv_connector.py:72-74; a multiple of block_size loses its last
    block)."""
    return (num_tokens - 1) // block_size * block_size


def _layer_index(layer_name: str) -> Optional[int]:
    """The integer after "layers" in a dotted module name
    ("model.layers.27.self_attn" -> 27), else None."""
    parts = layer_name.split(".")
    for i, p in enumerate(parts):
        if p == "layers" and i + 1 < len(parts):
            try:
                return int(parts[i + 1])
            except ValueError:
                pass
    return None


def _layer_groups(layers: List[Tuple[int, str, torch.Tensor]],
                  split_first: bool) -> List[list]:
    """Split index-sorted (index, name, cache) layers into launch groups: runs
    of consecutive layers of one geometry in one launch each and, with
    split_first (a restore on a side stream), the first layer alone before
    them, so that the forward's first attention waits only for a short
    launch.  A launch costs tens of microseconds of host work, more than the
    device time of a few layers, so the rest are not cut further: by the
    time the forward reaches the second layer the one large launch is well
    under way."""
    groups: List[list] = []
    geom_prev = None
    for item in layers:
        t = item[2]
        geom = (t.shape, t.stride(), t.dtype)
        g = groups[-1] if groups else None
        if (g is not None and (len(groups) > 1 or not split_first) and item[0] == g[-1][0] + 1
                and geom == geom_prev):
            g.append(item)
        else:
            groups.append([item])
        geom_prev = geom
    return groups


# ----------------------------------------------------------------- metadata --


@dataclass
class AMFReqMeta:
    """Per-request metadata passed from scheduler to worker (reference:
    amf_kv_connector.py:80-115)."""

    request_id: str
    prefix_hash: str
    token_ids: torch.Tensor
    slot_mapping: torch.Tensor
    is_store: bool
    num_tokens: int

    @staticmethod
    def make(request_id: str, prefix_hash: str, token_ids: List[int], block_ids: List[int],
             block_size: int, is_store: bool) -> "AMFReqMeta":
        """Slots of the first align_to_block_size(len(token_ids)) tokens:
        block b_i's slots b_i * block_size + [0, block_size) in block order."""
        valid = align_to_block_size(len(token_ids), block_size)
        blocks = torch.from_numpy(np.asarray(block_ids, dtype=np.int64)).reshape(-1, 1)
        slots = (blocks * block_size + torch.arange(block_size, dtype=torch.int64)).flatten()
        return AMFReqMeta(
            request_id=request_id,
            prefix_hash=prefix_hash,
            token_ids=torch.from_numpy(np.asarray(token_ids[:valid], dtype=np.int64)),
            slot_mapping=slots[:valid],
            is_store=is_store,
            num_tokens=valid,
        )


@dataclass
class AMFConnectorMetadata(KVConnectorMetadata):
    requests: List[AMFReqMeta] = field(default_factory=list)


# ---------------------------------------------------------------- connector --


class AMFKVConnector(KVConnectorBase_V1):
    """AMF compressed VRAM pool as a vLLM KV connector."""

    def __init__(self, vllm_config: Any, role: KVConnectorRole,
                 kv_cache_config: Any = None) -> None:
        super().__init__(vllm_config=vllm_config, role=role, kv_cache_config=kv_cache_config)
        self._block_size = vllm_config.cache_config.block_size
        self._requests_need_load: Dict[str, Any] = {}

        extra = getattr(self._kv_transfer_config, "kv_connector_extra_config", None) or {}
        self._num_layers = int(extra.get("num_layers", 28))
        self._num_kv_heads = int(extra.get("num_kv_heads", 2))
        self._head_dim = int(extra.get("head_dim", 64))
        self._bytes_per_layer = int(extra.get("bytes_per_layer", 1 << 23))
        self._default_format = str(extra.get("default_format", "fp8_e4m3"))
        self._min_prefix_tokens = int(extra.get("min_prefix_tokens", 64))
        load_stream = str(extra.get("load_stream", "current")).lower()
        if load_stream not in ("side", "current"):
            raise ValueError(f"load_stream must be 'side' or 'current', got {load_stream!r}")
        self._side_load = load_stream == "side"

        # Created on first use, so that a scheduler without a GPU still starts.
        self._pool: Optional["CompressedVRAMPool"] = None
        self._pool_init_done = False

        # prefix hash -> layer name -> (cache tensor of that layer, request slots)
        self._save_layers: Dict[str, Dict[str, Tuple[torch.Tensor, SlotMap]]] = {}
        self._save_slots: Dict[str, SlotMap] = {}  # request id -> its slots, this step
        self._known_hashes: set = set()
        self._load_error_blocks: set = set()  # blocks of hit requests whose load missed
        self._layer_idx_cache: Dict[str, Optional[int]] = {}
        self._load_stream: Optional[torch.cuda.Stream] = None
        self._layer_events: Dict[str, torch.cuda.Event] = {}
        self._waited: set = set()  # (event, stream) pairs already waited this step
        self._last_load_event: Optional[torch.cuda.Event] = None  # the step's final restore
        self._device_index = 0
        self._groups_memo = None

        logger.info(
            "[AMF_CONNECTOR] init role=%s layers=%d heads=%d head_dim=%d bytes_per_layer=%d "
            "format=%s block_size=%d", getattr(role, "name", role), self._num_layers,
            self._num_kv_heads, self._head_dim, self._bytes_per_layer, self._default_format,
            self._block_size)

    # ------------------------------------------------------------- pool --

    def _ensure_pool(self) -> Optional["CompressedVRAMPool"]:
        """The pool on the current GPU, made on first call; None (logged) when
        it cannot be made, e.g. without a GPU (reference: :174-197)."""
        if self._pool_init_done:
            return self._pool
        self._pool_init_done = True
        try:
            from .compressed_vram_pool import CompressedVRAMPool

            device = "cuda" if torch.cuda.is_available() else "cpu"
            self._pool = CompressedVRAMPool(
                num_layers=self._num_layers,
                bytes_per_layer=self._bytes_per_layer,
                block_bytes=1 << 17,
                default_format=self._default_format,
                device=device,
            )
            logger.info("[AMF_CONNECTOR] Pool created: %d layers x %d bytes on %s",
                        self._num_layers, self._bytes_per_layer, device)
        except Exception as exc:  # the connector then runs without a pool
            logger.warning("[AMF_CONNECTOR] Pool init failed: %s", exc)
            self._pool = None
        return self._pool

    # =========================================================== scheduler ==

    def get_num_new_matched_tokens(self, request: Any,
                                   num_computed_tokens: int) -> Tuple[Optional[int], bool]:
        """Tokens of the request's prompt the pool holds beyond those already
        computed; never asynchronous (reference: :203-241)."""
        token_ids = list(request.prompt_token_ids or [])
        if len(token_ids) < self._min_prefix_tokens:
            return 0, False
        n_check = align_to_block_size(len(token_ids) - 1, self._block_size)
        if n_check <= 0:
            return 0, False
        prefix_hash = _prefix_hash(token_ids[:n_check])
        pool = self._ensure_pool()
        # The pool is the authority when this process has one (an entry may
        # have been evicted or dropped since it was saved); the saved-hash set
        # only stands in for it in a scheduler without a GPU.
        hit = (prefix_hash in pool) if pool is not None else prefix_hash in self._known_hashes
        if not hit:
            return 0, False
        matched = n_check - num_computed_tokens
        if matched <= 0:
            return 0, False
        logger.info("[AMF_CONNECTOR] HIT prefix=%s matched=%d computed=%d total=%d",
                    prefix_hash[:12], matched, num_computed_tokens, n_check)
        return matched, False

    def update_state_after_alloc(self, request: Any, blocks: Any,
                                 num_external_tokens: int) -> None:
        if num_external_tokens > 0:
            self._requests_need_load[request.request_id] = request

    def build_connector_meta(self, scheduler_output: Any) -> AMFConnectorMetadata:
        """Load metadata for the requests update_state_after_alloc accepted,
        store metadata for every other new request (reference: :250-320)."""
        meta = AMFConnectorMetadata()
        bs = self._block_size
        loads = 0
        for new_req in scheduler_output.scheduled_new_reqs:
            token_ids = list(new_req.prompt_token_ids or [])
            n = align_to_block_size(len(token_ids) - 1, bs)
            prefix_hash = _prefix_hash(token_ids[:n]) if n > 0 else ""
            is_load = new_req.req_id in self._requests_need_load
            meta.requests.append(AMFReqMeta.make(
                request_id=new_req.req_id, prefix_hash=prefix_hash, token_ids=token_ids,
                block_ids=new_req.block_ids[0], block_size=bs, is_store=not is_load))
            loads += int(is_load)

        cached = scheduler_output.scheduled_cached_reqs
        for i, req_id in enumerate(cached.req_ids):
            if req_id not in cached.resumed_req_ids or req_id not in self._requests_need_load:
                continue
            request = self._requests_need_load[req_id]
            total = cached.num_computed_tokens[i] + scheduler_output.num_scheduled_tokens[req_id]
            token_ids = list(request.all_token_ids[:total])
            n = align_to_block_size(len(token_ids) - 1, bs)
            prefix_hash = _prefix_hash(token_ids[:n]) if n > 0 else ""
            new_block_ids = cached.new_block_ids[i]
            assert new_block_ids is not None
            meta.requests.append(AMFReqMeta.make(
                request_id=req_id, prefix_hash=prefix_hash, token_ids=token_ids,
                block_ids=new_block_ids[0], block_size=bs, is_store=False))
            loads += 1

        assert loads == len(self._requests_need_load), (
            f"Expected {len(self._requests_need_load)} loads, scheduled {loads}")
        self._requests_need_load.clear()
        return meta

    # ============================================================== worker ==

    def _layer_name_to_idx(self, layer_name: str) -> Optional[int]:
        if layer_name not in self._layer_idx_cache:
            self._layer_idx_cache[layer_name] = _layer_index(layer_name)
        return self._layer_idx_cache[layer_name]

    def _paged_layer(self, kv: torch.Tensor) -> Optional[torch.Tensor]:
        """A layer's KV as [2, num_blocks, block_size, H, D] (a view).  Flat
        [2, slots, H, D] and [2, slots, H * D] caches become pages of one
        token; None for any other shape."""
        if kv.dim() == 5 and kv.shape[0] == 2:
            return kv
        if kv.dim() == 4 and kv.shape[0] == 2:
            return kv.unsqueeze(2)
        if kv.dim() == 3 and kv.shape[0] == 2:
            return kv.view(2, kv.shape[1], 1, self._num_kv_heads, self._head_dim)
        return None

    def _load_groups(self, forward_context: Any) -> List[list]:
        """The step's attention layers as launch groups of (index, name, paged
        cache), rebuilt only when the layers' cache tensors change (vLLM
        passes the same tensors every step; the memo holds weak references)."""
        ve = getattr(forward_context, "virtual_engine", 0) or 0
        items = []
        for name, layer in forward_context.no_compile_layers.items():
            kv = getattr(layer, "kv_cache", None)
            if isinstance(kv, (list, tuple)):
                kv = kv[ve] if len(kv) > ve else None
            items.append((name, kv))
        key = (self._side_load,) + tuple((name, id(kv)) for name, kv in items)
        memo = self._groups_memo
        if memo is not None and memo[0] == key and all(
                r() is kv for r, (_, kv) in zip(memo[1], items)):
            return memo[2]
        layers = []
        for name, kv in items:
            idx = self._layer_name_to_idx(name)
            if kv is None or idx is None or not isinstance(kv, torch.Tensor) or kv.numel() == 0:
                continue
            pk = self._paged_layer(kv)
            if pk is None:
                logger.warning("[AMF_CONNECTOR] Unexpected kv_cache shape %s for %s",
                               tuple(kv.shape), name)
                continue
            layers.append((idx, name, pk))
        layers.sort(key=lambda t: t[0])
        groups = _layer_groups(layers, self._side_load)
        refs = [weakref.ref(kv) if isinstance(kv, torch.Tensor) else (lambda: None)
                for _, kv in items]
        self._groups_memo = (key, refs, groups)
        return groups

    def start_load_kv(self, forward_context: Any, **kwargs: Any) -> None:
        """Restore every hit request of this step into its slots, in layer
        groups, on the load stream (reference: :326-392, which restores
        request by request and layer by layer on the forward's stream before
        returning)."""
        metadata = self._get_connector_metadata()
        assert isinstance(metadata, AMFConnectorMetadata)
        self._layer_events.clear()
        self._waited.clear()
        pool = self._ensure_pool()
        if pool is None or getattr(forward_context, "attn_metadata", None) is None:
            return

        hits = []
        for req in metadata.requests:
            if req.is_store:
                continue
            entry = pool.get(req.prefix_hash)
            if entry is None:
                # Evicted (or dropped as a failed save) after the scheduler
                # counted it as a hit: the request's blocks were not filled,
                # so they are reported for recomputation instead of read.
                logger.warning("[AMF_CONNECTOR] LOAD MISS prefix=%s (pool has %d entries)",
                               req.prefix_hash[:12], pool.num_prefixes())
                self._known_hashes.discard(req.prefix_hash)
                self._load_error_blocks.update(
                    torch.unique(req.slot_mapping // self._block_size).tolist())
                continue
            logger.info("[AMF_CONNECTOR] Loading %d tokens for prefix=%s", req.num_tokens,
                        req.prefix_hash[:12])
            hits.append((req, entry, SlotMap(req.slot_mapping)))
        if not hits:
            return

        groups = self._load_groups(forward_context)
        if not groups:
            return

        device = pool.device
        self._device_index = device.index if device.index is not None else \
            torch.cuda.current_device()
        forward = torch.cuda.current_stream(device)
        stream = forward
        if self._side_load:
            if self._load_stream is None:
                self._load_stream = torch.cuda.Stream(device)  # default priority
            stream = self._load_stream
            stream.wait_stream(forward)
        with torch.cuda.stream(stream):
            for group in groups:
                first = group[0][0]
                caches = [pk for _, _, pk in group]
                for req, entry, slots in hits:
                    if first < entry.num_layers:
                        pool.restore_entry_to_slots(entry, caches, slots, first_layer=first)
                if self._side_load:
                    ev = torch.cuda.Event()
                    ev.record(stream)
                    for _, name, _ in group:
                        self._layer_events[name] = ev
                    self._last_load_event = ev
        for req, _, _ in hits:
            logger.info("[AMF_CONNECTOR] Loaded prefix=%s into paged buffer",
                        req.prefix_hash[:12])

    def wait_for_layer_load(self, layer_name: str) -> None:
        """Order the forward's stream after the restore of `layer_name` (no
        host wait)."""
        ev = self._layer_events.pop(layer_name, None)
        if ev is None:
            return
        key = (id(ev), torch._C._cuda_getCurrentRawStream(self._device_index))
        if key not in self._waited:  # layers of one launch share its event
            self._waited.add(key)
            torch.cuda.current_stream(self._pool.device).wait_event(ev)

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata: Any,
                      **kwargs: Any) -> None:
        """Note the layer's cache for every store request of this step; the
        rows are read by wait_for_save, before the step's forward returns and
        while the request still owns its pages (reference: :394-436)."""
        metadata = self._get_connector_metadata()
        assert isinstance(metadata, AMFConnectorMetadata)
        paged = None
        for req in metadata.requests:
            if not req.is_store:
                continue
            if paged is None:
                paged = self._paged_layer(kv_layer)
                if paged is None:
                    logger.warning("[AMF_CONNECTOR] Unexpected kv_layer shape %s for %s",
                                   tuple(kv_layer.shape), layer_name)
                    return
            slots = self._save_slots.get(req.request_id)
            if slots is None:
                n = min(int(req.slot_mapping.shape[0]), req.num_tokens)
                slots = self._save_slots[req.request_id] = SlotMap(req.slot_mapping[:n])
            self._save_layers.setdefault(req.prefix_hash, {})[layer_name] = (paged, slots)

    def wait_for_save(self) -> None:
        """Store each noted prefix, layers in index order, in the pool's
        default format (reference: :438-483)."""
        pool = self._ensure_pool()
        ev, self._last_load_event = self._last_load_event, None
        if pool is not None and ev is not None:
            # every restore of the step is ordered before the next step's work,
            # also for a layer whose wait_for_layer_load never came (the last
            # layer's wait usually did this already)
            key = (id(ev), torch._C._cuda_getCurrentRawStream(self._device_index))
            if key not in self._waited:
                self._waited.add(key)
                torch.cuda.current_stream(pool.device).wait_event(ev)
        self._save_slots.clear()
        if pool is None or not self._save_layers:
            self._save_layers.clear()
            return
        for prefix_hash, layers in self._save_layers.items():
            if not layers:
                continue
            names = sorted(layers, key=lambda n: self._layer_name_to_idx(n) or 0)
            caches = [layers[n][0] for n in names]
            slots = layers[names[0]][1]
            logger.info("[AMF_CONNECTOR] Saving prefix=%s (%d layers, %d tokens)",
                        prefix_hash[:12], len(caches), slots.n)
            ok = pool.put_from_slots(prefix_hash, caches, slots, format=self._default_format)
            if ok:
                self._known_hashes.add(prefix_hash)
                logger.info("[AMF_CONNECTOR] Saved prefix=%s (%d layers, pool=%d entries)",
                            prefix_hash[:12], len(caches), pool.num_prefixes())
            else:
                logger.warning("[AMF_CONNECTOR] Save FAILED for prefix=%s", prefix_hash[:12])
        self._save_layers.clear()

    def get_block_ids_with_load_errors(self) -> set:
        """Block ids of this step's loads that found no pool entry (vLLM's
        KVConnectorBase_V1 hook: the scheduler recomputes those tokens)."""
        out, self._load_error_blocks = self._load_error_blocks, set()
        return out

    @classmethod
    def requires_piecewise_for_cudagraph(cls, extra_config: Dict[str, Any]) -> bool:
        """save_kv_layer runs Python between layers."""
        return True


__all__ = [
    "AMFConnectorMetadata",
    "AMFKVConnector",
    "AMFReqMeta",
    "KVConnectorBase_V1",
    "KVConnectorMetadata",
    "KVConnectorRole",
    "align_to_block_size",
]
