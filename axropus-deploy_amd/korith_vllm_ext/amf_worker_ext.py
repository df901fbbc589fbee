"""amf_worker_ext.py - vLLM worker extension exposing AMF save / restore.

vLLM mixes the class named by `--worker-extension-cls` into its GPU worker;
the engine then calls `collective_rpc("amf_save_kv", ...)` and
`collective_rpc("amf_restore_kv", ...)` on every worker rank (the serving
command of the reference's README.md:80-90 names
korith_vllm_ext.amf_worker_ext.AmfWorkerExtension).  Each rank works on its
own shard of the KV cache (under tensor parallelism a rank holds
num_kv_heads / tp heads of every layer), so no rank talks to another.

Storage tier, chosen from the environment on first use (README.md:52-75):
  KORITH_VRAM_POOL_GB > 0    CompressedVRAMPool of that many GiB, format from
                             KORITH_VRAM_POOL_QUANT: "fp8" -> fp8_e4m3_ph,
                             "int4" -> int4_sym_block, or any pool format name
  KORITH_VRAM_CACHE_GB > 0   raw page snapshots (no quantization) in a pool of
                             that many GiB
  otherwise                  AMFK files under KORITH_AMF_PATH (needs token ids)
KORITH_VRAM_CACHE_DEVICE names the device (default: the worker's).

Return values are picklable: amf_save_kv -> bool, amf_restore_kv -> int
tokens (0 on a miss), amf_kv_stats -> dict.
"""

from __future__ import annotations

import logging
import os
from typing import Any, List, Optional, Sequence, Union

import torch

from .amf_kv_manager import AmfKvManager, amf_hash_tokens
from .codecs import FMT_FP8_E4M3_PH, FMT_INT4_BLOCK, FMT_RAW
from .compressed_vram_pool import POOL_FORMATS, CompressedVRAMPool

logger = logging.getLogger(__name__)

_QUANT_ALIASES = {"fp8": FMT_FP8_E4M3_PH, "int4": FMT_INT4_BLOCK}


def _env_float(name: str) -> float:
    try:
        return float(os.environ.get(name, "0") or 0)
    except ValueError:
        return 0.0


def prefix_key(prefix_hash_or_tokens: Union[str, int, Sequence[int]]) -> str:
    """Pool key: a string is used as is, an int is formatted as 16 hex digits,
    a token sequence is hashed (FNV-1a prefix hash) and formatted."""
    if isinstance(prefix_hash_or_tokens, str):
        return prefix_hash_or_tokens
    if isinstance(prefix_hash_or_tokens, int):
        return f"{prefix_hash_or_tokens & ((1 << 64) - 1):016x}"
    return f"{amf_hash_tokens(prefix_hash_or_tokens):016x}"


class _CacheEngineView:
    """The `gpu_cache` attribute AmfKvManager reads, over a worker's caches."""

    def __init__(self, worker: "AmfWorkerExtension") -> None:
        self._worker = worker

    @property
    def gpu_cache(self) -> List[torch.Tensor]:
        return self._worker._amf_kv_caches()


class AmfWorkerExtension:
    """Mixin for vLLM's GPU worker (`--worker-extension-cls`)."""

    _amf_pool: Optional[CompressedVRAMPool] = None
    _amf_manager: Optional[AmfKvManager] = None
    _amf_format: Optional[str] = None

    # ---------------------------------------------------------- caches --

    def _amf_kv_caches(self) -> List[torch.Tensor]:
        """Per-layer KV tensors of the worker ([2, num_blocks, block_size, H, D])."""
        runner = getattr(self, "model_runner", None)
        caches = getattr(runner, "kv_caches", None) if runner is not None else None
        if caches is None:
            caches = getattr(self, "kv_cache", None) or getattr(self, "gpu_cache", None)
        if isinstance(caches, dict):
            caches = list(caches.values())
        if caches and isinstance(caches[0], (list, tuple)):
            caches = caches[0]  # one virtual engine
        if not caches:
            raise RuntimeError("AmfWorkerExtension: the worker has no KV cache tensors")
        return list(caches)

    def _amf_device(self, caches: List[torch.Tensor]) -> torch.device:
        name = os.environ.get("KORITH_VRAM_CACHE_DEVICE", "")
        return torch.device(name) if name else caches[0].device

    def _amf_tier(self):
        if self._amf_pool is not None or self._amf_manager is not None:
            return
        caches = self._amf_kv_caches()
        pool_gb = _env_float("KORITH_VRAM_POOL_GB")
        raw_gb = _env_float("KORITH_VRAM_CACHE_GB")
        if pool_gb > 0 or raw_gb > 0:
            if pool_gb > 0:
                q = os.environ.get("KORITH_VRAM_POOL_QUANT", "int4").strip().lower()
                fmt = _QUANT_ALIASES.get(q, q)
                if fmt not in POOL_FORMATS or fmt == FMT_RAW:
                    raise ValueError(f"KORITH_VRAM_POOL_QUANT={q!r} names no pool format")
                gib = pool_gb
            else:
                fmt, gib = FMT_RAW, raw_gb
            per_layer = int(gib * (1 << 30)) // len(caches)
            per_layer -= per_layer % (1 << 17)
            self._amf_pool = CompressedVRAMPool(
                len(caches), per_layer, 1 << 17,
                default_format=fmt if fmt != FMT_RAW else FMT_INT4_BLOCK,
                device=self._amf_device(caches))
            self._amf_format = fmt
            logger.info("AMF worker: %s pool of %.1f GiB over %d layers", fmt, gib, len(caches))
        else:
            path = os.environ.get("KORITH_AMF_PATH", "/tmp/axropus-amf")
            cfg = getattr(getattr(self, "model_runner", None), "model_config", None)
            self._amf_manager = AmfKvManager(
                _CacheEngineView(self), path, cfg,
                tenant_id=os.environ.get("KORITH_TENANT_ID", "__shared__"))
            logger.info("AMF worker: AMFK snapshots under %s", path)

    # ------------------------------------------------------------- rpc --

    def amf_save_kv(self, prefix_hash_or_tokens: Union[str, int, Sequence[int]],
                    block_ids: List[int], num_tokens: int, format: Optional[str] = None) -> bool:
        """Save the pages `block_ids` of every layer under the prefix key."""
        self._amf_tier()
        if self._amf_pool is not None:
            return self._amf_pool.put_from_vllm(prefix_key(prefix_hash_or_tokens),
                                                self._amf_kv_caches(), list(block_ids),
                                                num_tokens, format=format or self._amf_format)
        if isinstance(prefix_hash_or_tokens, (str, int)):
            raise ValueError("AMFK snapshots are keyed by token ids")
        return self._amf_manager.save_kv_state(list(prefix_hash_or_tokens), list(block_ids))

    def amf_restore_kv(self, prefix_hash_or_tokens: Union[str, int, Sequence[int]],
                       block_ids: List[int]) -> int:
        """Restore the prefix into the pages `block_ids`; tokens restored."""
        self._amf_tier()
        if self._amf_pool is not None:
            return self._amf_pool.restore_to_vllm(prefix_key(prefix_hash_or_tokens),
                                                  self._amf_kv_caches(), list(block_ids))
        if isinstance(prefix_hash_or_tokens, (str, int)):
            raise ValueError("AMFK snapshots are keyed by token ids")
        return self._amf_manager.restore_kv_state(list(prefix_hash_or_tokens), list(block_ids))

    def amf_kv_stats(self) -> dict:
        self._amf_tier()
        if self._amf_pool is not None:
            return dict(self._amf_pool.stats(), format=self._amf_format)
        return dict(self._amf_manager.stats(), format="amfk")


__all__ = ["AmfWorkerExtension", "prefix_key"]
