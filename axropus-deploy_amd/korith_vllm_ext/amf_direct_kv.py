"""amf_direct_kv.py - AMFK KV snapshots through pinned host staging.

Python face of libamf_hip.so's amf_direct_kv_* entry points, the native
snapshot path of the reference (core/amf_direct_kv.{h,cu}: a context with a
pinned staging buffer; save = AMFK header + layer table + D2H of every layer;
restore = validate, then H2D of every layer).  Here the KV tensors are
given by the caller instead of read out of a llama.cpp context, and the
paged forms move vLLM cache pages through a two-slot device staging ring so
that the PCIe copies of one slot overlap the gather / scatter of the other.

Blobs returned by save() are views of the context's pinned buffer, valid
until the next call on the same context.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np
import torch

import amf_hip

from . import _paged

HEADER_BYTES = 56
LAYER_BYTES = 32


def _tokens_i32(tokens: Sequence[int]) -> np.ndarray:
    """Tokens as their 32-bit patterns (the header's prefix hash steps on the
    32-bit value of each token, amf_kv_manager.py:75-81)."""
    a = np.asarray(tokens, dtype=np.int64) if len(tokens) else np.zeros(0, np.int64)
    return np.ascontiguousarray((a & 0xFFFFFFFF).astype(np.uint32).view(np.int32))


def _addr_of(buf) -> tuple:
    """(address, size) of a host bytes-like object (kept alive by the caller)."""
    if isinstance(buf, tuple):
        return int(buf[0]), int(buf[1])
    a = np.frombuffer(buf, dtype=np.uint8)
    return int(a.ctypes.data), int(a.size)


def _u64_array(vals: Sequence[int]):
    return (ctypes.c_uint64 * max(1, len(vals)))(*[int(v) for v in vals])


class AmfDirectKv:
    """One direct-KV context (pinned staging buffer + copy stream).

    Not thread-safe: use one context per thread."""

    def __init__(self, max_kv_bytes: int = 0) -> None:
        self._lib = amf_hip.load()
        h = self._lib.amf_direct_kv_init(int(max_kv_bytes))
        if not h:
            msg = self._lib.amf_last_error()
            raise amf_hip.AmfHipError("amf_direct_kv_init", amf_hip.ERR_RUNTIME,
                                      msg.decode() if msg else "")
        self._h = ctypes.c_void_p(h)

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.amf_direct_kv_free(h)

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        if not self._h:
            raise ValueError("AmfDirectKv context is closed")
        return self._h

    # ------------------------------------------------------------ helpers --

    @staticmethod
    def is_direct_format(data) -> bool:
        addr, n = _addr_of(data)
        return bool(amf_hip.load().amf_direct_kv_is_direct_format(addr, n))

    def staging(self, nbytes: int) -> memoryview:
        """Writable view of the pinned staging buffer, grown to nbytes (waits
        for copies still reading it)."""
        out = ctypes.c_void_p()
        amf_hip.call("amf_direct_kv_staging", self.handle, int(nbytes), ctypes.byref(out))
        return memoryview((ctypes.c_ubyte * int(nbytes)).from_address(out.value)).cast("B")

    @staticmethod
    def _blob_view(ptr: ctypes.c_void_p, n: ctypes.c_uint64) -> memoryview:
        return memoryview((ctypes.c_ubyte * int(n.value)).from_address(ptr.value)).cast("B")

    # --------------------------------------------------- contiguous tensors --

    def save(self, k: Sequence[Optional[torch.Tensor]], v: Sequence[Optional[torch.Tensor]], *,
             tokens: Sequence[int], n_kv_heads: int, head_dim: int, dtype_tag: int,
             model_hash: int = 0) -> memoryview:
        """AMFK blob of the contiguous device tensors k[i], v[i] (None for a
        layer without KV), copied on torch's current stream."""
        if len(k) != len(v) or not k:
            raise ValueError("need one K and one V entry per layer")
        dev = next((t.device for t in k if t is not None), None)
        kp, kb, vp, vb = self._layer_arrays(k, v)
        toks = _tokens_i32(tokens)
        ptr, n = ctypes.c_void_p(), ctypes.c_uint64()
        amf_hip.call("amf_direct_kv_save", self.handle, kp, kb, vp, vb, len(k), n_kv_heads, head_dim,
                     dtype_tag, model_hash & ((1 << 64) - 1), toks.ctypes.data, toks.size,
                     ctypes.byref(ptr), ctypes.byref(n),
                     amf_hip.stream_handle(dev) if dev is not None else 0)
        return self._blob_view(ptr, n)

    def restore(self, blob, k: Sequence[Optional[torch.Tensor]],
                v: Sequence[Optional[torch.Tensor]]) -> int:
        """Validate `blob` against k, v and copy every layer in (stream-ordered
        on torch's current stream); the snapshot's token count."""
        if len(k) != len(v):
            raise ValueError("need one K and one V entry per layer")
        dev = next((t.device for t in k if t is not None), None)
        kp, kb, vp, vb = self._layer_arrays(k, v)
        addr, size = _addr_of(blob)
        nt = ctypes.c_uint32()
        amf_hip.call("amf_direct_kv_restore", self.handle, addr, size, kp, kb, vp, vb, len(k),
                     ctypes.byref(nt), amf_hip.stream_handle(dev) if dev is not None else 0)
        return int(nt.value)

    @staticmethod
    def _layer_arrays(k, v):
        for t in list(k) + list(v):
            if t is not None and not t.is_contiguous():
                raise ValueError("direct KV tensors must be contiguous")
        kp = _u64_array([0 if t is None else t.data_ptr() for t in k])
        kb = _u64_array([0 if t is None else t.numel() * t.element_size() for t in k])
        vp = _u64_array([0 if t is None else t.data_ptr() for t in v])
        vb = _u64_array([0 if t is None else t.numel() * t.element_size() for t in v])
        return kp, kb, vp, vb

    # --------------------------------------------------------- paged caches --

    def save_pages(self, view: "_paged.CacheView", block_ids: Optional[torch.Tensor], n_pages: int,
                   staging: torch.Tensor, *, tokens: Sequence[int], n_kv_heads: int,
                   head_dim: int, dtype_tag: int, model_hash: int = 0,
                   err_flag: Optional[torch.Tensor] = None) -> memoryview:
        """AMFK blob of pages block_ids[0..n_pages) of every plane of `view`
        (K0 V0 K1 V1 ... in the payload), through the device `staging` ring."""
        toks = _tokens_i32(tokens)
        planes = _u64_array(view.planes)
        ptr, n = ctypes.c_void_p(), ctypes.c_uint64()
        amf_hip.call("amf_direct_kv_save_pages", self.handle, planes, view.page_stride,
                     _paged._ptr(block_ids), view.pool_pages, n_pages, view.page_bytes,
                     view.n_layers, n_kv_heads, head_dim, dtype_tag,
                     model_hash & ((1 << 64) - 1), toks.ctypes.data, toks.size,
                     staging.data_ptr(), staging.numel() * staging.element_size(),
                     ctypes.byref(ptr), ctypes.byref(n), _paged._ptr(err_flag),
                     amf_hip.stream_handle(view.device))
        return self._blob_view(ptr, n)

    def restore_pages(self, blob, view: "_paged.CacheView", block_ids: Optional[torch.Tensor],
                      n_pages: int, staging: torch.Tensor,
                      err_flag: Optional[torch.Tensor] = None) -> int:
        """Validate `blob` and scatter each layer's pages into block_ids of
        `view` (stream-ordered on torch's current stream); the token count."""
        addr, size = _addr_of(blob)
        planes = _u64_array(view.planes)
        nt = ctypes.c_uint32()
        amf_hip.call("amf_direct_kv_restore_pages", self.handle, addr, size, planes,
                     view.page_stride, _paged._ptr(block_ids), view.pool_pages, n_pages,
                     view.page_bytes, view.n_layers, staging.data_ptr(),
                     staging.numel() * staging.element_size(), ctypes.byref(nt),
                     _paged._ptr(err_flag), amf_hip.stream_handle(view.device))
        return int(nt.value)


def staging_bytes_for(payload_bytes: int, page_bytes: int, slot_cap: int = 16 << 20) -> int:
    """Size of a two-slot staging ring for a payload: each slot a quarter of
    the payload (so copies and kernels overlap over four chunks), at least one
    page and at most slot_cap, in whole pages."""
    slot = min(slot_cap, max(page_bytes, payload_bytes // 4))
    slot = max(page_bytes, slot // page_bytes * page_bytes)
    return 2 * slot


__all__ = ["AmfDirectKv", "HEADER_BYTES", "LAYER_BYTES", "staging_bytes_for"]
