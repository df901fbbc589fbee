"""_paged.py - host-side plumbing between torch tensors and libamf_hip.so.

Describes a vLLM paged KV cache as "planes" (one K or V array of one layer),
lays out a compressed blob (codes + params of every plane of one layer, one
contiguous span), builds the device address tables the kernels take, and
launches the gather/scatter and codec entry points on torch's current stream.

Blob layout for `n` pages of geometry (block_size bs, heads H, head_dim D)
and P planes (P = 2 for a vLLM layer: K then V):

    [plane 0 codes][plane 1 codes]...[pad to 16][params]

params are either one region shared by every plane (fp8_e4m3's FP8ScaleSidecar,
int4_sym's per-channel scales) or one 16-byte-aligned region per plane.  The
byte formats of codes and params are the AMF_FMT_* layouts of
include/amf_hip.h.
"""

from __future__ import annotations

import math
import weakref
from collections import OrderedDict
from dataclasses import dataclass, field
from functools import cached_property
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

import amf_hip

# ---------------------------------------------------------------- formats --

FMT_FP8_E4M3 = "fp8_e4m3"
FMT_FP8_E4M3_PH = "fp8_e4m3_ph"
FMT_INT4_SYM = "int4_sym"
FMT_INT4_BLOCK = "int4_sym_block"
FMT_INT4_ASYM_G32 = "int4_asym_g32"
# Raw page bytes (no codec): already-quantized 1-byte caches, and the
# uncompressed snapshot tier.
FMT_RAW = "raw"

_FMT_IDS = {
    FMT_FP8_E4M3: amf_hip.FMT_FP8_E4M3,
    FMT_FP8_E4M3_PH: amf_hip.FMT_FP8_E4M3_PH,
    FMT_INT4_BLOCK: amf_hip.FMT_INT4_SYM_BLOCK,
    FMT_INT4_SYM: amf_hip.FMT_INT4_SYM,
    FMT_INT4_ASYM_G32: amf_hip.FMT_INT4_ASYM_G32,
}

PAGED_FORMATS = tuple(_FMT_IDS)

# Tokens per page a dense (unpaged) [.., T, H, D] tensor is cut into.  The
# reference's INT4PerBlockCodec blocks 128 tokens (amf_codec.py:353); the
# other formats are indifferent to paging and use vLLM's 16.
DENSE_PAGE_TOKENS = {
    FMT_FP8_E4M3: 16,
    FMT_FP8_E4M3_PH: 16,
    FMT_INT4_BLOCK: 128,
    FMT_INT4_SYM: 16,
    FMT_INT4_ASYM_G32: 16,
}


def _align16(n: int) -> int:
    return (n + 15) // 16 * 16


@dataclass(frozen=True)
class BlobLayout:
    """Byte layout of one compressed blob (n_pages pages of n_planes planes).
    elem_bytes is the cache element size of the raw format (codes are then
    the page bytes themselves)."""

    fmt: str
    n_planes: int
    n_pages: int
    block_size: int
    num_heads: int
    head_dim: int
    elem_bytes: int = 1

    @cached_property
    def fmt_id(self) -> int:
        return _FMT_IDS[self.fmt]

    @cached_property
    def family(self) -> str:
        if self.fmt == FMT_RAW:
            return "raw"
        return "fp8" if self.fmt.startswith("fp8") else "int4"

    @cached_property
    def page_elems(self) -> int:
        return self.block_size * self.num_heads * self.head_dim

    @cached_property
    def code_bytes_per_page(self) -> int:
        if self.family == "raw":
            return self.page_elems * self.elem_bytes
        return self.page_elems if self.family == "fp8" else self.page_elems // 2

    @cached_property
    def plane_code_bytes(self) -> int:
        return self.n_pages * self.code_bytes_per_page

    @cached_property
    def data_bytes(self) -> int:
        return self.n_planes * self.plane_code_bytes

    @cached_property
    def shared_params(self) -> bool:
        return self.fmt in (FMT_FP8_E4M3, FMT_INT4_SYM)

    @cached_property
    def plane_param_bytes(self) -> int:
        """Param bytes of one plane (0 for the shared-param formats)."""
        n, H, D = self.n_pages, self.num_heads, self.head_dim
        if self.fmt == FMT_FP8_E4M3_PH:
            return n * H * 4
        if self.fmt == FMT_INT4_BLOCK:
            return n * 2
        if self.fmt == FMT_INT4_ASYM_G32:
            return n * H * self.block_size * (D // 32) * 4
        return 0

    @cached_property
    def shared_param_bytes(self) -> int:
        if self.fmt == FMT_FP8_E4M3:
            return 16  # [k_scale, v_scale, q_scale, prob_scale] fp32
        if self.fmt == FMT_INT4_SYM:
            return self.head_dim * 2
        return 0

    @cached_property
    def scale_offset(self) -> int:
        return _align16(self.data_bytes)

    @cached_property
    def scale_bytes(self) -> int:
        if self.shared_params:
            return self.shared_param_bytes
        return (self.n_planes - 1) * _align16(self.plane_param_bytes) + self.plane_param_bytes

    @cached_property
    def total_bytes(self) -> int:
        return self.scale_offset + self.scale_bytes

    def code_offset(self, plane: int) -> int:
        return plane * self.plane_code_bytes

    def param_offset(self, plane: int) -> int:
        if self.shared_params:
            return self.scale_offset
        return self.scale_offset + plane * _align16(self.plane_param_bytes)

    def validate(self) -> None:
        if self.fmt == FMT_RAW:
            if self.code_bytes_per_page % 16:
                raise ValueError("raw pages must be a multiple of 16 bytes")
            return
        if self.fmt not in _FMT_IDS:
            raise KeyError(f"format {self.fmt!r} has no paged kernel")
        if self.head_dim % 32:
            raise ValueError(f"head_dim {self.head_dim} must be a multiple of 32")
        if self.fmt == FMT_INT4_ASYM_G32:
            if self.block_size != 16:
                raise ValueError("int4_asym_g32 pages hold 16 tokens")
            if self.n_planes % 2:
                raise ValueError("int4_asym_g32 needs (K, V) plane pairs")


# ------------------------------------------------------------- cache view --


@dataclass
class CacheView:
    """A list of per-layer KV tensors seen as planes (K0, V0, K1, V1, ...).

    Accepted per-layer shapes (compressed_vram_pool.py:483-486):
      [2, num_blocks, block_size, H, D]  stacked K/V (vLLM >= 0.6)
      [num_blocks, block_size, H, D]     one array used for both K and V
    Each page must be contiguous ([block_size][H][D] row-major).
    """

    planes: List[int]
    page_stride: int  # bytes
    pool_pages: int
    block_size: int
    num_heads: int
    head_dim: int
    dtype: torch.dtype
    device: torch.device
    keep: list = field(default_factory=list, repr=False)

    @property
    def n_layers(self) -> int:
        return len(self.planes) // 2

    @property
    def page_bytes(self) -> int:
        return self.block_size * self.num_heads * self.head_dim * _elem_size(self.dtype)


def _elem_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def _kv_planes(layer: torch.Tensor):
    """(K address, V address), plane shape [num_blocks, block_size, H, D] and
    plane strides (elements) of one layer, from its own shape and strides (no
    per-plane tensor is built: this runs once per layer on every save/load)."""
    shape = layer.shape
    st = layer.stride()
    if len(shape) == 5 and shape[0] == 2:
        base = layer.data_ptr()
        return (base, base + st[0] * layer.element_size()), tuple(shape[1:]), st[1:]
    if len(shape) == 4:
        base = layer.data_ptr()
        return (base, base), tuple(shape), st
    raise ValueError(
        f"KV cache layer of shape {tuple(shape)}: expected [2, num_blocks, block_size, H, D]"
        " or [num_blocks, block_size, H, D]"
    )


# Geometry of recently seen cache lists, by the identity of their tensors
# (weak references: a cached entry never keeps a cache alive, and a freed
# tensor whose id is reused fails the identity check).  A hit also requires
# every tensor's address, shape and strides to be the ones the view was built
# from: a live tensor whose storage was swapped in place (set_, resize_,
# .data =) misses and is measured again, so no launch gets stale addresses
# or a stale page count.
_VIEWS: "OrderedDict[tuple, tuple]" = OrderedDict()
_VIEWS_MAX = 64


def _layout_sig(t: torch.Tensor) -> tuple:
    return (t.data_ptr(), t.shape, t.stride())


def cache_view(gpu_cache: Sequence[torch.Tensor]) -> CacheView:
    key = tuple(map(id, gpu_cache))
    hit = _VIEWS.get(key)
    if hit is not None:
        refs, sigs, v = hit
        if all(r() is t and _layout_sig(t) == sg for r, sg, t in zip(refs, sigs, gpu_cache)):
            _VIEWS.move_to_end(key)
            return CacheView(v.planes, v.page_stride, v.pool_pages, v.block_size, v.num_heads,
                             v.head_dim, v.dtype, v.device, keep=list(gpu_cache))
    view = _make_cache_view(gpu_cache)
    geom = CacheView(view.planes, view.page_stride, view.pool_pages, view.block_size,
                     view.num_heads, view.head_dim, view.dtype, view.device, keep=[])
    _VIEWS[key] = ([weakref.ref(t) for t in gpu_cache], [_layout_sig(t) for t in gpu_cache], geom)
    while len(_VIEWS) > _VIEWS_MAX:
        _VIEWS.popitem(last=False)
    return view


def _make_cache_view(gpu_cache: Sequence[torch.Tensor]) -> CacheView:
    if len(gpu_cache) == 0:
        raise ValueError("empty KV cache")
    planes: List[int] = []
    geom = None
    for layer in gpu_cache:
        addrs, (nb, bs, H, D), st = _kv_planes(layer)
        if st[3] != 1 or st[2] != D or st[1] != H * D:
            raise ValueError("KV cache pages must be contiguous [block_size][H][D]")
        g = (nb, bs, H, D, st[0] * layer.element_size(), layer.dtype, layer.device)
        if geom is None:
            geom = g
        elif g != geom:
            raise ValueError(f"KV cache layers differ in geometry: {g} vs {geom}")
        planes.extend(addrs)
    nb, bs, H, D, stride, dtype, device = geom
    return CacheView(planes, stride, nb, bs, H, D, dtype, device, keep=list(gpu_cache))


def planes_view(planes: Sequence[torch.Tensor]) -> CacheView:
    """One plane per [num_blocks, block_size, H, D] tensor (contiguous pages)."""
    addrs = []
    geom = None
    for t in planes:
        nb, bs, H, D = t.shape
        if t.stride(3) != 1 or t.stride(2) != D or t.stride(1) != H * D:
            raise ValueError("plane pages must be contiguous [block_size][H][D]")
        g = (nb, bs, H, D, t.stride(0) * t.element_size(), t.dtype, t.device)
        if geom is None:
            geom = g
        elif g != geom:
            raise ValueError("planes differ in geometry")
        addrs.append(t.data_ptr())
    nb, bs, H, D, stride, dtype, device = geom
    return CacheView(addrs, stride, nb, bs, H, D, dtype, device, keep=list(planes))


def dense_view(x: torch.Tensor, page_tokens: int) -> Tuple[CacheView, int, torch.Tensor]:
    """View a contiguous [..., T, H, D] tensor as planes of pages.

    Leading dims become planes.  T is zero-padded to a multiple of page_tokens
    (a copy; zero rows change no absmax and are dropped on the way back).
    Returns (view, n_pages, padded tensor kept alive by the view).
    """
    if x.dim() < 3:
        raise ValueError(f"expected [..., tokens, heads, head_dim], got {tuple(x.shape)}")
    T, H, D = x.shape[-3:]
    P = int(math.prod(x.shape[:-3])) if x.dim() > 3 else 1
    xp = x.reshape(P, T, H, D)
    n_pages = max(1, -(-T // page_tokens))
    Tp = n_pages * page_tokens
    if Tp != T or not xp.is_contiguous():
        pad = torch.zeros((P, Tp, H, D), dtype=x.dtype, device=x.device)
        pad[:, :T].copy_(xp)
        xp = pad
    es = xp.element_size()
    page_stride = page_tokens * H * D * es
    planes = [xp.data_ptr() + p * Tp * H * D * es for p in range(P)]
    v = CacheView(planes, page_stride, n_pages, page_tokens, H, D, xp.dtype, xp.device, keep=[xp])
    return v, n_pages, xp


# ---------------------------------------------------------------- launches --


def _device_ids(ids, device) -> Optional[torch.Tensor]:
    """Block ids as a device int32 tensor; host ids travel through pinned
    memory, queued on the current stream without a host wait."""
    if ids is None:
        return None
    if isinstance(ids, torch.Tensor) and ids.device.type != "cpu":
        if ids.dtype == torch.int32 and ids.device == torch.device(device) and ids.is_contiguous():
            return ids
        return ids.to(device=device, dtype=torch.int32).contiguous()
    if isinstance(ids, torch.Tensor):
        host = ids.to(torch.int32).contiguous()
    else:
        host = torch.tensor(list(ids), dtype=torch.int32)
    return amf_hip.to_device(host, device)


def check_block_ids(ids: Sequence[int], pool_pages: int, *, unique: bool) -> None:
    """Host-side validation of a block table (ValueError, like the reference's
    shape checks) so that the kernels' in-kernel skip never has to trigger."""
    import numpy as np

    a = np.asarray(list(ids), dtype=np.int64)
    if a.size == 0:
        return
    if a.min() < 0 or a.max() >= pool_pages:
        raise ValueError(f"block id out of range [0, {pool_pages}): min {a.min()} max {a.max()}")
    if unique and np.unique(a).size != a.size:
        raise ValueError("duplicate block ids in a scatter target")


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else int(t.data_ptr())


def gather_pages(view: CacheView, block_ids, out_planes: Sequence[int], out_page_stride: int,
                 n_pages: int, err_flag: Optional[torch.Tensor] = None) -> None:
    dev = view.device
    ids = _device_ids(block_ids, dev)
    src = amf_hip.address_table(view.planes, dev)
    dst = amf_hip.address_table(out_planes, dev)
    amf_hip.call(
        "amf_kv_gather_pages", _ptr(src), view.page_stride, _ptr(ids), view.pool_pages, _ptr(dst),
        out_page_stride, len(view.planes), n_pages, view.page_bytes, _ptr(err_flag),
        amf_hip.stream_handle(dev),
    )


def scatter_pages(in_planes: Sequence[int], in_page_stride: int, view: CacheView, block_ids,
                  n_pages: int, err_flag: Optional[torch.Tensor] = None) -> None:
    dev = view.device
    ids = _device_ids(block_ids, dev)
    src = amf_hip.address_table(in_planes, dev)
    dst = amf_hip.address_table(view.planes, dev)
    amf_hip.call(
        "amf_kv_scatter_pages", _ptr(src), in_page_stride, _ptr(dst), view.page_stride, _ptr(ids),
        view.pool_pages, len(view.planes), n_pages, view.page_bytes, _ptr(err_flag),
        amf_hip.stream_handle(dev),
    )


@dataclass
class PlaneTables:
    """Device address tables of one codec launch (kept alive until enqueued)."""

    codes: torch.Tensor
    params: torch.Tensor


def blob_tables(layout: BlobLayout, blob_bases: Sequence[int], planes_per_blob: int,
                device) -> PlaneTables:
    """Code/param plane tables for blobs at `blob_bases` (one blob per group of
    planes_per_blob planes)."""
    co = [layout.code_offset(p) for p in range(planes_per_blob)]
    po = [layout.param_offset(p) for p in range(planes_per_blob)]
    codes = [base + o for base in blob_bases for o in co]
    params = [base + o for base in blob_bases for o in po]
    return PlaneTables(amf_hip.address_table(codes, device), amf_hip.address_table(params, device))


def quant_gather(layout: BlobLayout, view: CacheView, block_ids, blob_bases: Sequence[int],
                 planes_per_blob: int, workspace: Optional[torch.Tensor] = None,
                 err_flag: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Gather + quantize every plane of `view` into the blobs at blob_bases.

    Returns the workspace (it holds each scale group's absmax bits for the
    shared-scale formats after the launch)."""
    layout.validate()
    dev = view.device
    n_planes = len(view.planes)
    if n_planes != planes_per_blob * len(blob_bases):
        raise ValueError("plane count does not match the blobs")
    tables = blob_tables(layout, blob_bases, planes_per_blob, dev)
    ids = _device_ids(block_ids, dev)
    ws_bytes = amf_hip.quant_workspace_bytes(layout.fmt_id, n_planes, planes_per_blob, view.head_dim)
    if ws_bytes and (workspace is None or workspace.numel() * 4 < ws_bytes):
        workspace = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev)
    fn = "amf_fp8_quant_gather" if layout.family == "fp8" else "amf_int4_quant_gather"
    amf_hip.call(
        fn, layout.fmt_id, _ptr(amf_hip.address_table(view.planes, dev)), view.page_stride,
        amf_hip.dtype_tag(view.dtype), _ptr(ids), view.pool_pages, _ptr(tables.codes),
        _ptr(tables.params), n_planes, planes_per_blob, layout.n_pages, view.block_size,
        view.num_heads, view.head_dim, _ptr(workspace),
        0 if workspace is None else workspace.numel() * 4, _ptr(err_flag),
        amf_hip.stream_handle(dev),
    )
    return workspace


def dequant_scatter(layout: BlobLayout, blob_bases: Sequence[int], planes_per_blob: int,
                    view: CacheView, block_ids, err_flag: Optional[torch.Tensor] = None,
                    n_pages: Optional[int] = None) -> None:
    """Dequantize the first n_pages pages (default: all) of each plane of the
    blobs at blob_bases into the cache pages block_ids."""
    layout.validate()
    n = layout.n_pages if n_pages is None else n_pages
    if not 0 <= n <= layout.n_pages:
        raise ValueError(f"n_pages {n} outside [0, {layout.n_pages}]")
    dev = view.device
    n_planes = len(view.planes)
    if n_planes != planes_per_blob * len(blob_bases):
        raise ValueError("plane count does not match the blobs")
    tables = blob_tables(layout, blob_bases, planes_per_blob, dev)
    ids = _device_ids(block_ids, dev)
    fn = "amf_fp8_dequant_scatter" if layout.family == "fp8" else "amf_int4_dequant_scatter"
    amf_hip.call(
        fn, layout.fmt_id, _ptr(tables.codes), _ptr(tables.params),
        _ptr(amf_hip.address_table(view.planes, dev)), view.page_stride,
        amf_hip.dtype_tag(view.dtype), _ptr(ids), view.pool_pages, n_planes, n,
        view.block_size, view.num_heads, view.head_dim, _ptr(err_flag), amf_hip.stream_handle(dev),
    )


class PreparedCodecLaunch:
    """A dequant-scatter or quant-gather with its device tables built once.

    Repeated launches (a pool entry restored into the same cache, a timed
    loop) then cost one ctypes call each.  The object keeps every tensor the
    kernel reads alive."""

    def __init__(self, direction: str, layout: BlobLayout, blob_bases: Sequence[int],
                 planes_per_blob: int, view: CacheView, block_ids,
                 err_flag: Optional[torch.Tensor] = None) -> None:
        if direction not in ("save", "restore"):
            raise ValueError(direction)
        layout.validate()
        dev = view.device
        n_planes = len(view.planes)
        if n_planes != planes_per_blob * len(blob_bases):
            raise ValueError("plane count does not match the blobs")
        self.direction = direction
        self.layout = layout
        self.view = view
        self.tables = blob_tables(layout, blob_bases, planes_per_blob, dev)
        self.cache_tab = amf_hip.address_table(view.planes, dev)
        self.ids = _device_ids(block_ids, dev)
        self.err_flag = err_flag
        self.planes_per_blob = planes_per_blob
        self.workspace = None
        ws_bytes = amf_hip.quant_workspace_bytes(layout.fmt_id, n_planes, planes_per_blob,
                                                 view.head_dim)
        if direction == "save" and ws_bytes:
            self.workspace = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev)
        fam = layout.family
        self.fn = f"amf_{fam}_quant_gather" if direction == "save" else f"amf_{fam}_dequant_scatter"
        self._cfn = getattr(amf_hip.load(), self.fn)

    def launch(self, stream: Optional[int] = None) -> None:
        v, lay = self.view, self.layout
        s = amf_hip.stream_handle(v.device) if stream is None else stream
        if self.direction == "save":
            ws = self.workspace
            rc = self._cfn(lay.fmt_id, _ptr(self.cache_tab), v.page_stride,
                           amf_hip.dtype_tag(v.dtype), _ptr(self.ids), v.pool_pages,
                           _ptr(self.tables.codes), _ptr(self.tables.params), len(v.planes),
                           self.planes_per_blob, lay.n_pages, v.block_size, v.num_heads,
                           v.head_dim, _ptr(ws), 0 if ws is None else ws.numel() * 4,
                           _ptr(self.err_flag), s)
        else:
            rc = self._cfn(lay.fmt_id, _ptr(self.tables.codes), _ptr(self.tables.params),
                           _ptr(self.cache_tab), v.page_stride, amf_hip.dtype_tag(v.dtype),
                           _ptr(self.ids), v.pool_pages, len(v.planes), lay.n_pages,
                           v.block_size, v.num_heads, v.head_dim, _ptr(self.err_flag), s)
        amf_hip.check(self.fn, rc)


# ------------------------------------------------------------- token slots --


class SlotMap:
    """A vLLM slot mapping (one slot id per token, slot = block * block_size +
    offset; reference: AMFReqMeta.make, amf_kv_connector.py:90-115).

    Kept on the host, where the page-structure test runs, and copied once per
    device for the slot kernels.  A device tensor given here costs one
    device-to-host copy."""

    def __init__(self, slots) -> None:
        if isinstance(slots, torch.Tensor):
            host = slots.detach().reshape(-1).to("cpu", torch.int64)
        else:
            host = torch.tensor(list(slots), dtype=torch.int64)
        self.host = host.contiguous()
        self._np = self.host.numpy()  # shares the tensor's memory
        self.n = int(self.host.numel())
        self._dev = {}
        self._checked = set()
        self._pages = {}

    @classmethod
    def of(cls, slots) -> "SlotMap":
        return slots if isinstance(slots, SlotMap) else cls(slots)

    def on(self, device) -> torch.Tensor:
        """The slots on `device`, made once; recorded on every other stream
        that uses them so their memory outlives the kernels queued there."""
        dev = torch.device(device)
        key = (dev.type, dev.index)
        return self._cached_on(key, dev, lambda: amf_hip.to_device(self.host, dev))

    def _cached_on(self, key, dev, make) -> torch.Tensor:
        sid = amf_hip.stream_handle(dev)
        got = self._dev.get(key)
        if got is None:
            got = (make(), {sid})
            self._dev[key] = got
        t, streams = got
        if sid not in streams:
            t.record_stream(torch.cuda.current_stream(dev))
            streams.add(sid)
        return t

    def check(self, pool_slots: int, n: Optional[int] = None) -> None:
        """ValueError unless the first n slots lie in [0, pool_slots)."""
        n = self.n if n is None else n
        if (pool_slots, n) in self._checked:
            return
        a = self._np[:n]
        if a.size and (int(a.min()) < 0 or int(a.max()) >= pool_slots):
            raise ValueError(f"slot id out of range [0, {pool_slots}): min {int(a.min())} "
                             f"max {int(a.max())}")
        self._checked.add((pool_slots, n))

    def page_ids(self, n_tokens: int, block_size: int) -> Optional[List[int]]:
        """Block ids when the first n_tokens slots are whole pages in order
        (token p*block_size + i at slot b_p*block_size + i); None otherwise."""
        ids = self._page_array(n_tokens, block_size)
        return None if ids is None else ids.tolist()

    def _page_array(self, n_tokens: int, block_size: int) -> Optional[np.ndarray]:
        key = (n_tokens, block_size)
        if key not in self._pages:
            self._pages[key] = self._page_ids(n_tokens, block_size)
        return self._pages[key]

    def _page_ids(self, n_tokens: int, block_size: int) -> Optional[np.ndarray]:
        if n_tokens <= 0 or n_tokens > self.n or n_tokens % block_size:
            return None
        a = self._np[:n_tokens].reshape(-1, block_size)
        first = a[:, 0]
        if (first % block_size).any():
            return None
        if not np.array_equal(a, first[:, None] + np.arange(block_size, dtype=np.int64)):
            return None
        ids = first // block_size
        if ids.size and int(ids.max()) > np.iinfo(np.int32).max:
            return None
        return ids.astype(np.int32)

    def page_ids_on(self, n_tokens: int, block_size: int, device) -> Optional[torch.Tensor]:
        """page_ids as a device int32 tensor, made once per device."""
        ids = self._page_array(n_tokens, block_size)
        if ids is None:
            return None
        dev = torch.device(device)
        return self._cached_on((dev.type, dev.index, n_tokens, block_size), dev,
                               lambda: amf_hip.to_device(torch.from_numpy(ids), dev))


def _row_bytes(view: CacheView) -> int:
    return view.num_heads * view.head_dim * _elem_size(view.dtype)


def token_pages(view: CacheView, page_tokens: int) -> Optional[CacheView]:
    """The same planes cut in pages of page_tokens rows: the view itself when
    its pages already hold page_tokens rows, else a re-cut when the token
    rows are evenly spaced (pages unpadded), page p then starting at token
    row p * page_tokens.  None otherwise."""
    if page_tokens == view.block_size:
        return view
    row = _row_bytes(view)
    if view.page_stride != view.block_size * row:
        return None
    n = view.pool_pages * view.block_size // page_tokens
    if n == 0:
        return None
    return CacheView(view.planes, page_tokens * row, n, page_tokens, view.num_heads,
                     view.head_dim, view.dtype, view.device, keep=view.keep)


def gather_slots(view: CacheView, slots: SlotMap, n: int, out_planes: Sequence[int],
                 out_row_stride: int, err_flag: Optional[torch.Tensor] = None) -> None:
    """out_planes[i] row j <- the cache row slots[j] of plane i, j < n."""
    dev = view.device
    amf_hip.call(
        "amf_kv_gather_slots", _ptr(amf_hip.address_table(view.planes, dev)), view.page_stride,
        view.block_size, _ptr(slots.on(dev)), view.pool_pages * view.block_size,
        _ptr(amf_hip.address_table(out_planes, dev)), out_row_stride, len(view.planes), n,
        _row_bytes(view), _ptr(err_flag), amf_hip.stream_handle(dev),
    )


def scatter_slots(in_planes: Sequence[int], in_row_stride: int, view: CacheView, slots: SlotMap,
                  n: int, err_flag: Optional[torch.Tensor] = None) -> None:
    """The cache row slots[j] of plane i <- in_planes[i] row j, j < n."""
    dev = view.device
    amf_hip.call(
        "amf_kv_scatter_slots", _ptr(amf_hip.address_table(in_planes, dev)), in_row_stride,
        _ptr(amf_hip.address_table(view.planes, dev)), view.page_stride, view.block_size,
        _ptr(slots.on(dev)), view.pool_pages * view.block_size, len(view.planes), n,
        _row_bytes(view), _ptr(err_flag), amf_hip.stream_handle(dev),
    )
