"""GPU parity of libamf_hip.so against the oracle, through the C ABI.

Bar: raw gather/scatter and quantized codes/params bit-exact; dequantized
cache values bit-exact (the spec and the oracle share every rounding step);
untouched cache pages keep their sentinel.  Decode attention: max |err| <=
2e-2 and sum|err| / sum|ref| <= 1e-2 against float64 attention over the
fp32-dequantized INT4 KV.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import amf_hip
from korith_vllm_ext import _paged
from oracle import attention as oatt
from oracle import codecs as oc
from oracle import gen
from oracle import paging as opg

from helpers import bits, bytes_of, check_attention, sentinel_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _cache_from(values: torch.Tensor) -> list:
    """values [L, 2, pool, bs, H, D] (CPU) -> list of per-layer device tensors."""
    return [values[l].to(DEV).contiguous() for l in range(values.shape[0])]


def _pages(values: torch.Tensor, l: int, ids: torch.Tensor) -> torch.Tensor:
    return values[l][:, ids.long()]


# ------------------------------------------------------------ raw copies --


def test_raw_gather_scatter_qwen05b_full():
    """Raw bf16 snapshot + restore at the Qwen2-0.5B shape: 24 layers, 2 KV heads,
    head_dim 64, pool 4096, a 2048-token (128-page) prefix."""
    s = gen.WORKLOADS["raw_qwen05b"]
    g = torch.Generator(device="cuda").manual_seed(s.seed)
    cache = [torch.randn(2, s.pool_blocks, s.block_size, s.kv_heads, s.head_dim, generator=g,
                         device=DEV).to(torch.bfloat16) for _ in range(s.layers)]
    src_ids = gen.block_table(s.pool_blocks, s.prefix_blocks, seed=101)
    dst_ids = gen.block_table(s.pool_blocks, s.prefix_blocks, seed=202)
    view = _paged.cache_view(cache)
    snap = torch.empty(s.layers, 2, s.prefix_blocks, s.block_size, s.kv_heads, s.head_dim,
                       dtype=torch.bfloat16, device=DEV)
    page_bytes = view.page_bytes
    out_planes = [snap[l, kv].data_ptr() for l in range(s.layers) for kv in range(2)]
    _paged.gather_pages(view, src_ids, out_planes, page_bytes, s.prefix_blocks)
    target = sentinel_cache(s.layers, s.pool_blocks, s.block_size, s.kv_heads, s.head_dim,
                            torch.bfloat16, DEV)
    tview = _paged.cache_view(target)
    _paged.scatter_pages(out_planes, page_bytes, tview, dst_ids, s.prefix_blocks)
    torch.cuda.synchronize()

    src = np.stack([bits(c) for c in cache])                     # [L, 2, pool, ...]
    want_snap = opg.gather(src.reshape(s.layers * 2, s.pool_blocks, -1), src_ids.numpy())
    got_snap = bits(snap).reshape(s.layers * 2, s.prefix_blocks, -1)
    assert np.array_equal(got_snap, want_snap)
    tgt0 = np.stack([bits(c) for c in sentinel_cache(s.layers, s.pool_blocks, s.block_size,
                                                     s.kv_heads, s.head_dim, torch.bfloat16,
                                                     "cpu")])
    want_tgt = opg.scatter(tgt0.reshape(s.layers * 2, s.pool_blocks, -1), dst_ids.numpy(),
                           want_snap)
    got_tgt = np.stack([bits(c) for c in target]).reshape(s.layers * 2, s.pool_blocks, -1)
    assert np.array_equal(got_tgt, want_tgt)


def test_raw_out_of_range_id_is_skipped_and_flagged():
    cache = [torch.randn(2, 8, 16, 2, 64, device=DEV).to(torch.bfloat16)]
    view = _paged.cache_view(cache)
    snap = torch.zeros(2, 3, 16, 2, 64, dtype=torch.bfloat16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    ids = torch.tensor([1, 99, 2], dtype=torch.int32)
    _paged.gather_pages(view, ids, [snap[0].data_ptr(), snap[1].data_ptr()], view.page_bytes, 3,
                        err_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) & amf_hip.ERRFLAG_BLOCK_RANGE
    assert torch.equal(snap[:, 1], torch.zeros_like(snap[:, 1]))           # skipped page
    assert torch.equal(snap[:, 0], cache[0][:, 1]) and torch.equal(snap[:, 2], cache[0][:, 2])


# ------------------------------------------------------------------ codecs --

CODEC_GEOM = dict(L=2, pool=64, n=24, bs=16, H=8, D=128)
# 48 heads: pages too large for the register-resident save kernels (and, for
# int4_asym_g32, for the LDS page stage), so the two-read kernels run.
WIDE_GEOM = dict(L=1, pool=16, n=6, bs=16, H=48, D=128)
CODEC_CASES = [
    pytest.param(torch.bfloat16, CODEC_GEOM, id="bf16"),
    pytest.param(torch.float16, CODEC_GEOM, id="fp16"),
    pytest.param(torch.float32, CODEC_GEOM, id="fp32"),
    pytest.param(torch.bfloat16, WIDE_GEOM, id="bf16-48heads"),
    pytest.param(torch.float32, WIDE_GEOM, id="fp32-48heads"),
]


def _codec_case(dtype, seed, geom=CODEC_GEOM, outliers=True):
    L, pool, n, bs, H, D = (geom[k] for k in ("L", "pool", "n", "bs", "H", "D"))
    g = torch.Generator().manual_seed(seed)
    values = gen.kv_values((L, 2, pool, bs, H, D), D, g, outliers, dtype)
    src_ids = gen.block_table(pool, n, seed + 1)
    dst_ids = gen.block_table(pool, n, seed + 2)
    return values, src_ids, dst_ids


def _save(fmt, values, src_ids, dtype, geom=CODEC_GEOM):
    L, n, bs, H, D = geom["L"], geom["n"], geom["bs"], geom["H"], geom["D"]
    cache = _cache_from(values)
    view = _paged.cache_view(cache)
    layout = _paged.BlobLayout(fmt, 2, n, bs, H, D)
    blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    ws = _paged.quant_gather(layout, view, src_ids, [b.data_ptr() for b in blobs], 2)
    torch.cuda.synchronize()
    return layout, blobs, ws


def _restore(layout, blobs, dst_ids, dtype, geom=CODEC_GEOM):
    L, pool, bs, H, D = geom["L"], geom["pool"], geom["bs"], geom["H"], geom["D"]
    target = sentinel_cache(L, pool, bs, H, D, dtype, DEV)
    view = _paged.cache_view(target)
    _paged.dequant_scatter(layout, [b.data_ptr() for b in blobs], 2, view, dst_ids)
    torch.cuda.synchronize()
    return target


def _check_restored(target, dst_ids, want_pages_per_layer, dtype, geom=CODEC_GEOM):
    L, pool, bs, H, D = geom["L"], geom["pool"], geom["bs"], geom["H"], geom["D"]
    base = sentinel_cache(1, pool, bs, H, D, dtype, "cpu")[0]
    for l in range(L):
        want = base.clone()
        want[:, dst_ids.long()] = want_pages_per_layer[l]
        assert np.array_equal(bits(target[l]), bits(want)), f"layer {l}"


def _seg(blob, off, nbytes):
    return blob[off:off + nbytes]


@pytest.mark.parametrize("dtype,geom", CODEC_CASES)
def test_fp8_tensor_format_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 10, geom)
    layout, blobs, ws = _save("fp8_e4m3", values, src_ids, dtype, geom)
    want = []
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, src_ids)
        codes, scale = oc.fp8_tensor_compress(pages)
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(codes))
        side = _seg(blob, layout.scale_offset, 16).view(torch.float32).cpu()
        assert torch.equal(side, oc.fp8_sidecar(scale))
        want.append(oc.fp8_tensor_decompress(codes, scale, dtype))
    target = _restore(layout, blobs, dst_ids, dtype, geom)
    _check_restored(target, dst_ids, want, dtype, geom)


# Scale groups of at least 4 MiB whose pages are whole multiples of 256
# 16-byte chunks take the single-read cooperative kernel: an odd group count
# (the last group has no partner buffer), one page per workgroup (CPT 8),
# several pages per workgroup (CPT 1), and two pages per workgroup of CPT 8
# (1200-page groups: more than the 768 workgroups that 256 CUs keep resident).
COOP_CASES = [
    pytest.param(torch.bfloat16, dict(L=3, pool=512, n=160, bs=16, H=8, D=128), id="bf16-3groups"),
    pytest.param(torch.float16, dict(L=2, pool=2048, n=1200, bs=16, H=2, D=64), id="fp16-cpt1"),
    pytest.param(torch.bfloat16, dict(L=2, pool=700, n=600, bs=16, H=8, D=128), id="bf16-2ppw"),
]


@pytest.mark.parametrize("dtype,geom", COOP_CASES)
def test_fp8_tensor_single_read_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 12, geom)
    # an out-of-range block id: that page is skipped (its codes stay as they
    # were, zero here) and flagged; the others' scale ignores it
    src_ids = src_ids.clone()
    bad = 7
    src_ids[bad] = geom["pool"] + 3
    L, n, bs, H, D = geom["L"], geom["n"], geom["bs"], geom["H"], geom["D"]
    cache = _cache_from(values)
    view = _paged.cache_view(cache)
    layout = _paged.BlobLayout("fp8_e4m3", 2, n, bs, H, D)
    blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    _paged.quant_gather(layout, view, src_ids, [b.data_ptr() for b in blobs], 2, err_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == amf_hip.ERRFLAG_BLOCK_RANGE
    ok_ids = src_ids.clone()
    ok_ids[bad] = 0
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, ok_ids).clone()
        pages[:, bad] = 0
        codes, scale = oc.fp8_tensor_compress(pages)
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(codes)), l
        side = _seg(blob, layout.scale_offset, 16).view(torch.float32).cpu()
        assert torch.equal(side, oc.fp8_sidecar(scale)), l


def _tensor_save_digest(dtype, geom):
    import hashlib
    values, src_ids, _ = _codec_case(dtype, 12, geom)
    L, n, bs, H, D = geom["L"], geom["n"], geom["bs"], geom["H"], geom["D"]
    view = _paged.cache_view(_cache_from(values))
    layout = _paged.BlobLayout("fp8_e4m3", 2, n, bs, H, D)
    blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    _paged.quant_gather(layout, view, src_ids, [b.data_ptr() for b in blobs], 2)
    torch.cuda.synchronize()
    return hashlib.sha256(b"".join(bytes_of(b).tobytes() for b in blobs)).hexdigest()


def test_fp8_tensor_no_coop_environment_same_bytes():
    """AMF_NO_COOP=1 (read once per process, so checked in a child process)
    sends a per-tensor save that the single-read kernel would take to the
    two-pass kernels: same bytes."""
    import os
    import subprocess
    import sys
    geom = dict(L=3, pool=512, n=160, bs=16, H=8, D=128)
    want = _tensor_save_digest(torch.bfloat16, geom)
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [here, root, os.path.join(root, "axropus-deploy_amd")]
    code = ("import sys, torch; sys.path[:0] = %r; import test_gpu_kernels as T; "
            "print(T._tensor_save_digest(torch.bfloat16, %r))" % (paths, geom))
    env = dict(os.environ, AMF_NO_COOP="1")
    print("child process: per-tensor save with AMF_NO_COOP=1", flush=True)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=240, cwd=root)
    assert out.returncode == 0, out.stderr[-2000:]
    assert out.stdout.strip().splitlines()[-1] == want


def test_fp8_tensor_single_read_beside_another_stream():
    """The cooperative per-tensor save issued while restores run on a second
    stream (default priority): it completes without a sync give-up and its
    codes still equal the oracle's."""
    dtype, geom = torch.bfloat16, dict(L=3, pool=512, n=160, bs=16, H=8, D=128)
    values, src_ids, dst_ids = _codec_case(dtype, 14, geom)
    L, n, bs, H, D = geom["L"], geom["n"], geom["bs"], geom["H"], geom["D"]
    cache = _cache_from(values)
    view = _paged.cache_view(cache)
    layout = _paged.BlobLayout("fp8_e4m3", 2, n, bs, H, D)
    blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    # busy work for the side stream: restores of a PH blob into a scratch cache
    ph = _paged.BlobLayout("fp8_e4m3_ph", 2, n, bs, H, D)
    ph_blobs = [torch.zeros(ph.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    _paged.quant_gather(ph, view, src_ids, [b.data_ptr() for b in ph_blobs], 2)
    scratch = [torch.empty_like(c) for c in cache]
    sview = _paged.cache_view(scratch)
    torch.cuda.synchronize()
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(200):
            _paged.dequant_scatter(ph, [b.data_ptr() for b in ph_blobs], 2, sview, dst_ids)
    for _ in range(3):
        _paged.quant_gather(layout, view, src_ids, [b.data_ptr() for b in blobs], 2,
                            err_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    for l, blob in enumerate(blobs):
        codes, scale = oc.fp8_tensor_compress(_pages(values, l, src_ids))
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(codes)), l
        side_scale = _seg(blob, layout.scale_offset, 16).view(torch.float32).cpu()
        assert torch.equal(side_scale, oc.fp8_sidecar(scale)), l


_GIVE_UP_SCRIPT = r"""
import sys, torch
sys.path[:0] = sys.argv[2:4]
from korith_vllm_ext import _paged
cache = torch.load(sys.argv[1] + "/cache.pt", weights_only=True)
ids = torch.load(sys.argv[1] + "/ids.pt", weights_only=True)
L, n = len(cache), ids.numel()
layout = _paged.BlobLayout("fp8_e4m3", 2, n, 16, 8, 128)
blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device="cuda") for _ in range(L)]
flag = torch.zeros(1, dtype=torch.int32, device="cuda")
view = _paged.cache_view([c.cuda() for c in cache])
_paged.quant_gather(layout, view, ids, [b.data_ptr() for b in blobs], 2, err_flag=flag)
torch.cuda.synchronize()
torch.save({"flag": flag.cpu(), "blobs": [b.cpu() for b in blobs]}, sys.argv[1] + "/out.pt")
"""


def test_fp8_tensor_single_read_give_up_path(tmp_path):
    """With the wait bound forced to zero polls (AMF_COOP_SPIN_LIMIT=0, read
    once per process, hence a child process) a workgroup that finds its
    group not yet complete takes the give-up path at once.  Whether any does
    depends on timing (a workgroup's loads of the next group usually outlast
    the exchange), so the check is the invariant: the launch finishes, and
    each layer holds either the oracle's codes or an infinite scale (never
    plausible wrong values), with AMF_ERRFLAG_SYNC raised exactly when some
    layer is poisoned."""
    import os
    import subprocess
    import sys

    geom = dict(L=3, pool=512, n=160, bs=16, H=8, D=128)
    values, src_ids, _ = _codec_case(torch.bfloat16, 16, geom)
    torch.save([values[l].contiguous() for l in range(geom["L"])], tmp_path / "cache.pt")
    torch.save(src_ids, tmp_path / "ids.pt")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, AMF_COOP_SPIN_LIMIT="0")
    subprocess.run([sys.executable, "-c", _GIVE_UP_SCRIPT, str(tmp_path), root,
                    os.path.join(root, "axropus-deploy_amd")], env=env, check=True, timeout=90)
    out = torch.load(tmp_path / "out.pt", weights_only=True)
    gave_up = bool(int(out["flag"].item()) & amf_hip.ERRFLAG_SYNC)
    layout = _paged.BlobLayout("fp8_e4m3", 2, geom["n"], 16, 8, 128)
    poisoned = 0
    for l, blob in enumerate(out["blobs"]):
        side = blob[layout.scale_offset:layout.scale_offset + 16].view(torch.float32)
        if torch.isinf(side[0]):
            poisoned += 1
            continue
        codes, scale = oc.fp8_tensor_compress(_pages(values, l, src_ids))
        assert np.array_equal(bytes_of(blob[:layout.data_bytes]), bytes_of(codes)), l
        assert torch.equal(side, oc.fp8_sidecar(scale)), l
    assert gave_up == (poisoned > 0), (gave_up, poisoned)


@pytest.mark.parametrize("dtype,geom", CODEC_CASES)
def test_fp8_page_head_format_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 20, geom)
    # one page of layer 0, head 3 all zeros: absmax 0 -> the 1e-8 floor
    values[0, :, int(src_ids[5]), :, 3, :] = 0
    layout, blobs, _ = _save("fp8_e4m3_ph", values, src_ids, dtype, geom)
    want = []
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, src_ids)
        codes, scales = oc.fp8_ph_compress(pages)
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(codes))
        for p in range(2):
            got = _seg(blob, layout.param_offset(p), layout.plane_param_bytes).view(torch.float32)
            assert torch.equal(got.cpu().view(scales[p].shape), scales[p])
        want.append(oc.fp8_ph_decompress(codes, scales, dtype))
    target = _restore(layout, blobs, dst_ids, dtype, geom)
    _check_restored(target, dst_ids, want, dtype, geom)


def test_fp8_encode_every_bf16_in_range():
    """With a (page, head) absmax of exactly 448 the scale is 1.0 and every bf16
    input is encoded directly: all 2 x 32640 finite bf16 values in [-448, 448]."""
    u = np.arange(0, 0x43E1, dtype=np.uint32)            # +0 .. 448 as bf16 bits
    u = np.concatenate([u, u | 0x8000])
    vals = torch.from_numpy((u << 16).view(np.float32)).to(torch.bfloat16)
    n_rows = -(-vals.numel() // 128)
    n_pages = -(-n_rows // 16)
    x = torch.zeros(n_pages * 16 * 128, dtype=torch.bfloat16)
    x[:vals.numel()] = vals
    x = x.view(1, 1, n_pages, 16, 1, 128).clone()
    x[..., 0, 0, 0] = 448.0                              # absmax 448 in every page
    geom = dict(L=1, pool=n_pages, n=n_pages, bs=16, H=1, D=128)
    ids = torch.arange(n_pages, dtype=torch.int32)
    values = torch.cat([x, x], dim=1)                    # K and V identical
    layout, blobs, _ = _save("fp8_e4m3_ph", values, ids, torch.bfloat16, geom)
    codes, scales = oc.fp8_ph_compress(values[0])
    assert torch.all(scales == 1.0)
    assert np.array_equal(bytes_of(_seg(blobs[0], 0, layout.data_bytes)), bytes_of(codes))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_decode_every_code(dtype):
    """Dequant of all 256 codes with scale 1: the restored cache bits equal the
    cast of each code's value, signed zero included (NaN codes excluded)."""
    n = 2
    codes = torch.arange(256, dtype=torch.uint8).repeat(n * 16 * 128 // 256).view(1, n, 16, 1, 128)
    codes = torch.cat([codes, codes], dim=0)              # [2, n, 16, 1, 128]
    layout = _paged.BlobLayout("fp8_e4m3_ph", 2, n, 16, 1, 128)
    blob = torch.zeros(layout.total_bytes, dtype=torch.uint8)
    blob[:layout.data_bytes] = codes.flatten()
    for p in range(2):
        o = layout.param_offset(p)
        blob[o:o + layout.plane_param_bytes] = torch.ones(n, dtype=torch.float32).view(torch.uint8)
    blob = blob.to(DEV)
    target = sentinel_cache(1, n, 16, 1, 128, dtype, DEV)
    _paged.dequant_scatter(layout, [blob.data_ptr()], 2, _paged.cache_view(target),
                           torch.arange(n, dtype=torch.int32))
    torch.cuda.synchronize()
    want = codes.view(torch.float8_e4m3fn).float().to(dtype)
    finite = ~torch.isnan(want)
    assert np.array_equal(bits(target[0].cpu()[finite]), bits(want[finite]))


@pytest.mark.parametrize("dtype,geom", CODEC_CASES)
def test_int4_sym_block_format_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 30, geom)
    values[geom["L"] - 1, :, int(src_ids[3])] = 0          # an all-zero page
    layout, blobs, _ = _save("int4_sym_block", values, src_ids, dtype, geom)
    want = []
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, src_ids)                 # [2, n, bs, H, D]
        packed, scales, meta = oc.int4_block_compress(pages)
        assert meta["n_blocks"] == 1
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(packed))
        for p in range(2):
            got = _seg(blob, layout.param_offset(p), layout.plane_param_bytes).view(torch.float16)
            assert torch.equal(got.cpu(), scales[p].flatten())
        want.append(oc.int4_block_decompress(packed, scales, tuple(pages.shape), meta, dtype))
    target = _restore(layout, blobs, dst_ids, dtype, geom)
    _check_restored(target, dst_ids, want, dtype, geom)


@pytest.mark.parametrize("dtype,geom", CODEC_CASES)
def test_int4_sym_channel_format_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 40, geom)
    layout, blobs, _ = _save("int4_sym", values, src_ids, dtype, geom)
    want = []
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, src_ids)
        packed, scales = oc.int4_channel_compress(pages)
        assert np.array_equal(bytes_of(_seg(blob, 0, layout.data_bytes)), bytes_of(packed))
        got = _seg(blob, layout.scale_offset, layout.shared_param_bytes).view(torch.float16)
        assert torch.equal(got.cpu(), scales)
        want.append(oc.int4_channel_decompress(packed, scales, tuple(pages.shape), dtype))
    target = _restore(layout, blobs, dst_ids, dtype, geom)
    _check_restored(target, dst_ids, want, dtype, geom)


# Per-channel INT4 on larger scale groups (the reduction spans several
# absmax workgroups per plane), head_dim 64 to 1024, with an out-of-range
# block id.
CHAN_LARGE_CASES = [
    pytest.param(torch.bfloat16, dict(L=3, pool=512, n=160, bs=16, H=8, D=128), id="bf16-d128"),
    pytest.param(torch.float16, dict(L=2, pool=2048, n=1200, bs=16, H=2, D=64), id="fp16-d64"),
    pytest.param(torch.bfloat16, dict(L=2, pool=256, n=160, bs=16, H=4, D=256), id="bf16-d256"),
    # rows of 64 and 128 lanes: no two lanes of a wave share channels
    pytest.param(torch.float32, dict(L=2, pool=128, n=70, bs=16, H=2, D=512), id="fp32-d512"),
    pytest.param(torch.float16, dict(L=2, pool=128, n=70, bs=16, H=1, D=1024), id="fp16-d1024"),
]


@pytest.mark.parametrize("dtype,geom", CHAN_LARGE_CASES)
def test_int4_sym_channel_large_groups_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 42, geom)
    src_ids = src_ids.clone()
    bad = 5
    src_ids[bad] = geom["pool"] + 1                 # skipped and flagged
    L, n, bs, H, D = geom["L"], geom["n"], geom["bs"], geom["H"], geom["D"]
    cache = _cache_from(values)
    view = _paged.cache_view(cache)
    layout = _paged.BlobLayout("int4_sym", 2, n, bs, H, D)
    blobs = [torch.zeros(layout.total_bytes, dtype=torch.uint8, device=DEV) for _ in range(L)]
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    _paged.quant_gather(layout, view, src_ids, [b.data_ptr() for b in blobs], 2, err_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == amf_hip.ERRFLAG_BLOCK_RANGE
    ok_ids = src_ids.clone()
    ok_ids[bad] = 0
    page_bytes = bs * H * D // 2
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, ok_ids).clone()
        pages[:, bad] = 0                           # a skipped page adds nothing to the max
        packed, scales = oc.int4_channel_compress(pages)
        got = bytes_of(_seg(blob, 0, layout.data_bytes)).reshape(2, n, page_bytes)
        want = bytes_of(packed).reshape(2, n, page_bytes)
        keep = np.arange(n) != bad                  # the skipped page's codes stay zero
        assert np.array_equal(got[:, keep], want[:, keep]), l
        assert not got[:, bad].any(), l
        sc = _seg(blob, layout.scale_offset, layout.shared_param_bytes).view(torch.float16)
        assert torch.equal(sc.cpu(), scales), l


# Odd head counts (the V restore pairs head blocks) and head_dim 64 / 256.
ASYM_CASES = CODEC_CASES + [
    pytest.param(torch.bfloat16, dict(L=2, pool=32, n=12, bs=16, H=3, D=64), id="bf16-3heads-d64"),
    pytest.param(torch.float16, dict(L=1, pool=32, n=10, bs=16, H=1, D=256), id="fp16-1head-d256"),
]


@pytest.mark.parametrize("dtype,geom", ASYM_CASES)
def test_int4_asym_g32_format_bitexact(dtype, geom):
    values, src_ids, dst_ids = _codec_case(dtype, 50, geom)
    values[0, 1, int(src_ids[2]), 4, geom["H"] - 1, 32:64] = 1.5   # a constant group
    layout, blobs, _ = _save("int4_asym_g32", values, src_ids, dtype, geom)
    want = []
    for l, blob in enumerate(blobs):
        pages = _pages(values, l, src_ids)
        codes, params = oc.int4_asym_compress(pages)
        for p in range(2):
            got_c = _seg(blob, layout.code_offset(p), layout.plane_code_bytes)
            assert np.array_equal(bytes_of(got_c), codes[p].to(torch.uint8).flatten().numpy()), p
            got_p = _seg(blob, layout.param_offset(p), layout.plane_param_bytes).view(torch.int32)
            want_p = params[p].flatten().to(torch.int64) & 0xFFFFFFFF
            assert np.array_equal(got_p.cpu().numpy().view(np.uint32).astype(np.int64),
                                  want_p.numpy()), p
        want.append(oc.int4_asym_decompress(codes, params, 16, geom["H"], geom["D"], dtype))
    target = _restore(layout, blobs, dst_ids, dtype, geom)
    _check_restored(target, dst_ids, want, dtype, geom)


# ------------------------------------------------------ decode attention --


def _decode_case(R, Hkv, ctxs, seed):
    B, D, bs = len(ctxs), 128, 16
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, R * Hkv, D, generator=g).to(torch.bfloat16)
    pages = [max(1, -(-c // bs)) for c in ctxs]
    pool = sum(pages) + 3
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    M = max(pages)
    bt = torch.full((B, M), -1, dtype=torch.int32)         # unused slots: never read
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kv = gen.kv_values((2, pool, bs, Hkv, D), D, g, True, torch.bfloat16)
    codes, params = oc.int4_asym_compress(kv)              # planes K, V
    u, s16, z16 = oc.int4_asym_quantize(kv)
    kv32 = oc.int4_asym_dequant_f32(u, s16, z16)           # [2, pool, bs, Hkv, D]
    return q, bt, torch.tensor(ctxs, dtype=torch.int32), pool, codes, params, kv32


def _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo, max_ctx=None,
                out_dtype=torch.float32):
    B, Hq, D = q.shape
    max_ctx = int(ctx.max()) if max_ctx is None else max_ctx
    dq = q.to(DEV)
    out = torch.full(dq.shape, 3.0, dtype=out_dtype, device=DEV)
    kc = codes[0].to(torch.uint8).to(DEV)
    vc = codes[1].to(torch.uint8).to(DEV)
    kp = (params[0] & 0xFFFFFFFF).to(torch.int64).numpy().astype(np.uint32).view(np.int32)
    vp = (params[1] & 0xFFFFFFFF).to(torch.int64).numpy().astype(np.uint32).view(np.int32)
    kp = torch.from_numpy(kp).to(DEV)
    vp = torch.from_numpy(vp).to(DEV)
    dbt = bt.to(DEV)
    dctx = ctx.to(DEV)
    ws_bytes = amf_hip.decode_workspace_bytes(B, Hq, Hkv, D, max_ctx)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    amf_hip.call(
        "amf_int4_paged_decode_attn", dq.data_ptr(), amf_hip.DTYPE_BF16, out.data_ptr(),
        amf_hip.dtype_tag(out_dtype),
        kc.data_ptr(), kp.data_ptr(), vc.data_ptr(), vp.data_ptr(), pool, dbt.data_ptr(),
        bt.shape[1], dctx.data_ptr(), B, Hq, Hkv, D, 16, max_ctx, 0.0, ws.data_ptr(),
        ws.numel() * 4, algo, flag.data_ptr(), amf_hip.stream_handle(DEV))
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), int(flag.item())


DECODE_ALGOS = [amf_hip.DECODE_MFMA, amf_hip.DECODE_MFMA_PRECISE, amf_hip.DECODE_VALU]


@pytest.mark.parametrize("algo", DECODE_ALGOS)
@pytest.mark.parametrize("R", [1, 2, 4, 8])
def test_int4_paged_decode_matches_f64(algo, R):
    if algo == amf_hip.DECODE_VALU and R > 4:
        pytest.skip("the VALU path handles GQA groups up to 4")
    ctxs = [1, 16, 37, 300, 1500, 0]
    Hkv = 2
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, ctxs, seed=60 + R)
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
    assert flag == 0
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    check_attention(got, ref)
    if algo == amf_hip.DECODE_MFMA_PRECISE:
        # bf16 hi + lo PV weights keep about 16 bits per weight (fp16
        # weights: about 11 bits): mean error about 10x below the fp16 path's
        check_attention(got, ref, max_abs=5e-3, mean_rel=2e-4)
    assert np.all(got[-1] == 0.0)                          # empty context -> zeros
    # bf16 output = round-to-nearest-even of the same fp32 result
    got16, _ = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo, out_dtype=torch.bfloat16)
    assert np.array_equal(got16, torch.from_numpy(got).to(torch.bfloat16).float().numpy())


def test_int4_paged_decode_shares_span_many_pairs():
    """Many short sequences (more chunks than the device has resident waves):
    a wave's share then covers several (sequence, KV head) pairs, the middle
    ones whole (finished in place) and the ends shared with neighbours
    (merged from partial slots); empty sequences in between give zeros."""
    g = torch.Generator().manual_seed(91)
    ctxs = torch.randint(1, 160, (700,), generator=g).tolist()
    for i in range(0, 700, 97):
        ctxs[i] = 0
    R, Hkv = 4, 8
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, ctxs, seed=92)
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    # every algorithm within the stated tolerance on fp32 output; the default
    # MFMA kernel keeps these short, peaked rows on precise PV weights (its
    # fp16 weights only where their rounding error budget allows)
    for algo in DECODE_ALGOS:
        got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
        assert flag == 0
        check_attention(got, ref, label=f"algo {algo}")
        assert np.all(got[np.asarray(ctxs) == 0] == 0.0)
        if algo == amf_hip.DECODE_MFMA_PRECISE:
            # bf16 hi/lo PV weights throughout: the work map's indexing to a tight bound
            check_attention(got, ref, max_abs=5e-3, mean_rel=2e-4, label="precise, tight")


@pytest.mark.parametrize("algo", DECODE_ALGOS)
def test_int4_paged_decode_peaked_scores(algo):
    """Extreme score range across tiles (after tests/test_kernels.py:115-133 of
    the reference): early tokens aligned with q dominate."""
    R, Hkv = 4, 1
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, [700], seed=77)
    # rebuild K so that the first 40 tokens are 3 x q of head 0
    kv = oc.int4_asym_dequant_f32(*oc.int4_asym_quantize(
        gen.kv_values((2, pool, 16, Hkv, 128), 128, torch.Generator().manual_seed(5), True)))
    order = bt[0][: -(-700 // 16)].long()
    flat_k = kv[0][order].reshape(-1, Hkv, 128)
    flat_k[:40, 0] = 3.0 * q[0, 0].float()
    kv[0][order] = flat_k.reshape(-1, 16, Hkv, 128)
    kv_bf = kv.to(torch.bfloat16)
    codes, params = oc.int4_asym_compress(kv_bf)
    kv32 = oc.int4_asym_dequant_f32(*oc.int4_asym_quantize(kv_bf))
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    check_attention(got, ref)


@pytest.mark.parametrize("algo", [amf_hip.DECODE_MFMA, amf_hip.DECODE_MFMA_PRECISE])
@pytest.mark.parametrize("case", ["large", "small", "mixed"])
def test_int4_paged_decode_scale_range_paths(case, algo):
    """The MFMA kernel's PV product takes fp16 weights for a 32-token chunk
    whose V scales all lie in [2^-10, 255] and bf16 hi + lo weights otherwise.
    V scaled x300 (scales above 255), x1e-5 (below 2^-10), and x300 on every
    other page of each sequence (both paths inside one split) must all decode
    to the float64 result, compared after dividing out the factor."""
    R, Hkv, D, bs = 4, 2, 128, 16
    ctxs = [37, 700, 1500, 300]
    g = torch.Generator().manual_seed(141)
    q = torch.randn(len(ctxs), R * Hkv, D, generator=g).to(torch.bfloat16)
    pages = [-(-c // bs) for c in ctxs]
    pool = sum(pages) + 3
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    bt = torch.full((len(ctxs), max(pages)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kv = gen.kv_values((2, pool, bs, Hkv, D), D, g, True, torch.float32)
    factor = {"large": 300.0, "small": 1e-5, "mixed": 300.0}[case]
    if case == "mixed":
        for b, n in enumerate(pages):
            for i in range(0, n, 2):
                kv[1, int(bt[b, i])] *= factor
    else:
        kv[1] *= factor
    kv = kv.to(torch.bfloat16)
    codes, params = oc.int4_asym_compress(kv)
    kv32 = oc.int4_asym_dequant_f32(*oc.int4_asym_quantize(kv))
    s_v = oc.int4_asym_quantize(kv)[1][1].float()
    if case == "small":
        assert float(s_v.max()) < 2.0 ** -10
    else:
        assert float(s_v.max()) > 255.0
    ctx = torch.tensor(ctxs, dtype=torch.int32)
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
    assert flag == 0
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    check_attention(got / factor, ref / factor)


@pytest.mark.parametrize("algo", [amf_hip.DECODE_MFMA, amf_hip.DECODE_MFMA_PRECISE])
@pytest.mark.parametrize("factor", [3e5, 1e-6])
def test_int4_paged_decode_query_range(factor, algo):
    """The QK^T tiles take the query as fp16 scaled per wave by a power of two:
    a bf16 query beyond the fp16 range (x3e5) and one far below its normal
    range (x1e-6) must score as the float64 reference does."""
    R, Hkv = 4, 2
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, [40, 333, 1100], seed=151)
    q = (q.float() * factor).to(torch.bfloat16)
    assert (float(q.float().abs().max()) > 65504.0) == (factor > 1.0)
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
    assert flag == 0
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    check_attention(got, ref)


@pytest.mark.parametrize("algo", DECODE_ALGOS)
def test_int4_paged_decode_ignores_slots_past_the_context(algo):
    """Slots past a sequence's context (the tail of its last page) may hold
    any bytes: NaN and infinite scales and zero points there must not reach
    the output."""
    R, Hkv, bs = 4, 2, 16
    ctxs = [37, 300, 1500, 7, 33]
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, ctxs, seed=93)
    u, s16, z16 = oc.int4_asym_unlayout(codes, params, bs, Hkv, 128)
    s_bits, z_bits = s16.view(torch.int16), z16.view(torch.int16)
    poison = [(0x7C00, 0x7E00), (0x7E00, 0xFC00 - 0x10000)]     # (+inf, NaN), (NaN, -inf)
    n_poisoned = 0
    for b, c in enumerate(ctxs):
        tail = c % bs
        if tail:
            page = int(bt[b, c // bs])
            for p in range(2):
                s_bits[p, page, tail:] = poison[p][0]
                z_bits[p, page, tail:] = poison[p][1]
            n_poisoned += bs - tail
    assert n_poisoned > 0
    codes, params = oc.int4_asym_layout(u, s16, z16)
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, algo)
    assert flag == 0
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    assert np.all(np.isfinite(got))
    check_attention(got, ref)


def test_int4_paged_decode_split_major_grid():
    """More than 65535 splits (max_context_len 64M + 1 tokens at 1024-token
    splits) selects the (max_splits, num_kv_heads, num_seqs) grid; the short
    real contexts must decode as on the head-major grid."""
    R, Hkv = 4, 2
    ctxs = [1500, 37]
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, ctxs, seed=91)
    max_ctx = 65536 * 1024 + 1
    wide = torch.full((len(ctxs), -(-max_ctx // 16)), -1, dtype=torch.int32)
    wide[:, :bt.shape[1]] = bt
    ref = oatt.paged_decode_f64(q.float().numpy(), kv32[0].numpy(), kv32[1].numpy(), bt.numpy(),
                                ctx.numpy())
    for algo in (amf_hip.DECODE_MFMA, amf_hip.DECODE_VALU):
        got, flag = _run_decode(q, wide, ctx, pool, codes, params, Hkv, algo, max_ctx=max_ctx)
        assert flag == 0
        check_attention(got, ref)


def test_int4_paged_decode_bad_page_flagged_not_faulting():
    R, Hkv = 2, 2
    q, bt, ctx, pool, codes, params, kv32 = _decode_case(R, Hkv, [64, 64], seed=90)
    bt[1, 2] = pool + 1000                                 # out of range
    got, flag = _run_decode(q, bt, ctx, pool, codes, params, Hkv, amf_hip.DECODE_MFMA)
    assert flag & amf_hip.ERRFLAG_BLOCK_RANGE
    ref = oatt.paged_decode_f64(q.float().numpy()[:1], kv32[0].numpy(), kv32[1].numpy(),
                                bt.numpy()[:1], ctx.numpy()[:1])
    check_attention(got[:1], ref)                          # the clean sequence is unaffected
    assert np.all(np.isfinite(got))
