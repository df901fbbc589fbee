"""Host logic on the CPU: blob layouts and their byte counts, cache views,
block-table validation, the codec registry and selection policy, the FP8
sidecar, and the kernel dispatch registry.  Nothing here launches a kernel;
the entry points that need a device are checked to refuse CPU tensors."""

from __future__ import annotations

import pytest
import torch

from korith_vllm_ext import _paged
from korith_vllm_ext.codecs import (
    FMT_FP8_E4M3,
    FMT_INT4_BLOCK,
    FMT_NVFP4,
    FMT_TURBOQUANT,
    FP8ScaleSidecar,
    apply_fp8_scales,
    get_codec,
    list_codecs,
    select_codec,
)


def test_restore_algorithmic_bytes():
    """Per-launch bytes of the benchmark restores: codes + params read, bf16
    pages written, for 32 layers."""
    fp8 = _paged.BlobLayout("fp8_e4m3_ph", 2, 512, 16, 8, 128)
    assert fp8.data_bytes == 2 * 512 * 16 * 8 * 128
    assert fp8.scale_bytes == 2 * 512 * 8 * 4
    assert 32 * (fp8.data_bytes + fp8.scale_bytes + 2 * 512 * fp8.page_elems * 2) == 1_611_661_312
    i4 = _paged.BlobLayout("int4_asym_g32", 2, 2048, 16, 8, 128)
    assert i4.data_bytes == 2048 * 16 * 8 * 128
    assert i4.scale_bytes == 2 * 2048 * 16 * 8 * 4 * 4
    assert 32 * (i4.data_bytes + i4.scale_bytes + 2 * 2048 * i4.page_elems * 2) == 5_637_144_576
    # decode reads 1280 B per context token over 8 KV heads (16 tokens per page)
    per_page = 2 * (i4.code_bytes_per_page + i4.plane_param_bytes // i4.n_pages)
    assert per_page // 16 == 1280


@pytest.mark.parametrize("fmt", _paged.PAGED_FORMATS)
def test_blob_layout_offsets(fmt):
    lay = _paged.BlobLayout(fmt, 2, 37, 16, 4, 64)
    lay.validate()
    assert lay.code_offset(1) == lay.plane_code_bytes
    assert lay.scale_offset % 16 == 0 and lay.scale_offset >= lay.data_bytes
    for p in range(2):
        assert lay.param_offset(p) % 16 == 0
        assert lay.param_offset(p) + max(lay.plane_param_bytes, lay.shared_param_bytes) \
            <= lay.total_bytes
    if lay.shared_params:
        assert lay.param_offset(0) == lay.param_offset(1)
    else:
        assert lay.param_offset(1) - lay.param_offset(0) >= lay.plane_param_bytes


def test_blob_layout_validation():
    with pytest.raises(ValueError):
        _paged.BlobLayout("int4_asym_g32", 3, 4, 16, 2, 64).validate()
    with pytest.raises(ValueError):
        _paged.BlobLayout("int4_asym_g32", 2, 4, 32, 2, 64).validate()
    with pytest.raises(ValueError):
        _paged.BlobLayout("fp8_e4m3_ph", 2, 4, 16, 2, 48).validate()
    with pytest.raises(KeyError):
        _paged.BlobLayout("nvfp4", 2, 4, 16, 2, 64).validate()


def test_cache_view_shapes():
    layers = [torch.zeros(2, 10, 16, 2, 64, dtype=torch.bfloat16) for _ in range(3)]
    v = _paged.cache_view(layers)
    assert v.n_layers == 3 and len(v.planes) == 6 and v.pool_pages == 10
    assert v.page_stride == v.page_bytes == 16 * 2 * 64 * 2
    assert v.planes[1] - v.planes[0] == 10 * v.page_bytes
    single = _paged.cache_view([torch.zeros(10, 16, 2, 64, dtype=torch.float16)])
    assert single.planes[0] == single.planes[1]
    with pytest.raises(ValueError):
        _paged.cache_view([torch.zeros(2, 10, 16, 2, 64)[:, :, :, :, :32]])
    with pytest.raises(ValueError):
        _paged.cache_view([layers[0], torch.zeros(2, 11, 16, 2, 64, dtype=torch.bfloat16)])
    with pytest.raises(ValueError):
        _paged.cache_view([])


def test_cache_view_memo_sees_storage_swapped_in_place():
    """A memoized view is reused only while every tensor keeps the address,
    shape and strides it was built from: set_ / resize_ / .data = on a live
    tensor give a fresh view (addresses and page count)."""
    layers = [torch.zeros(2, 10, 16, 2, 64, dtype=torch.bfloat16) for _ in range(2)]
    v1 = _paged.cache_view(layers)
    assert _paged.cache_view(layers).planes == v1.planes          # memo hit
    layers[1].set_(torch.zeros(2, 10, 16, 2, 64, dtype=torch.bfloat16))
    v2 = _paged.cache_view(layers)
    assert v2.planes[:2] == v1.planes[:2] and v2.planes[2] == layers[1].data_ptr()
    assert v2.planes[2] != v1.planes[2]
    layers[0].data = torch.zeros(2, 6, 16, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):                               # 6 vs 10 pages now
        _paged.cache_view(layers)
    layers[1].data = torch.zeros(2, 6, 16, 2, 64, dtype=torch.bfloat16)
    v3 = _paged.cache_view(layers)
    assert v3.pool_pages == 6 and v3.planes[0] == layers[0].data_ptr()


def test_dense_view_pads_tokens():
    x = torch.randn(3, 20, 2, 64).to(torch.bfloat16)
    v, n, xp = _paged.dense_view(x, 16)
    assert n == 2 and len(v.planes) == 3 and xp.shape == (3, 32, 2, 64)
    assert torch.equal(xp[:, :20], x) and not xp[:, 20:].any()
    v2, n2, xp2 = _paged.dense_view(torch.randn(32, 2, 64), 16)
    assert n2 == 2 and len(v2.planes) == 1


def test_block_id_checks():
    _paged.check_block_ids([0, 5, 9], 10, unique=True)
    _paged.check_block_ids([], 10, unique=True)
    with pytest.raises(ValueError):
        _paged.check_block_ids([0, 10], 10, unique=False)
    with pytest.raises(ValueError):
        _paged.check_block_ids([-1], 10, unique=False)
    with pytest.raises(ValueError):
        _paged.check_block_ids([3, 3], 10, unique=True)
    _paged.check_block_ids([3, 3], 10, unique=False)


# ------------------------------------------------------------- codecs ----


def test_codec_registry():
    names = list_codecs()
    for f in ("fp8_e4m3", "fp8_e4m3_ph", "int4_sym", "int4_sym_block", "int4_asym_g32"):
        assert f in names
        assert get_codec(f).FORMAT == f
    with pytest.raises(KeyError):
        get_codec("nvfp4")
    assert get_codec("fp8_e4m3").memory_ratio() == 0.5
    assert get_codec("int4_sym_block").memory_ratio() == 0.25


def test_select_codec_policy():
    """tests/test_codecs.py:140-150 plus the gfx950 row (device version 95)."""
    assert select_codec(100) in {FMT_NVFP4, FMT_TURBOQUANT}
    assert select_codec(80) == FMT_INT4_BLOCK
    assert select_codec(90, density_budget=0.50) == FMT_FP8_E4M3
    assert select_codec(90, density_budget=0.20) == FMT_TURBOQUANT
    assert select_codec(95) == FMT_INT4_BLOCK
    assert select_codec(95, density_budget=0.5) == FMT_FP8_E4M3
    assert select_codec(70) == "fp16"


def test_fp8_sidecar_roundtrip_and_apply():
    """tests/test_codecs.py:92-137."""
    s = FP8ScaleSidecar(k_scale=0.123, v_scale=0.456, q_scale=1.0, prob_scale=2.0)
    s2 = FP8ScaleSidecar.from_tensor(s.to_tensor())
    assert abs(s2.k_scale - 0.123) < 1e-6 and abs(s2.prob_scale - 2.0) < 1e-6
    Attention = type("Attention", (), {})
    attn = Attention()
    attn._k_scale = attn._v_scale = attn._q_scale = attn._prob_scale = 1.0
    attn.calculate_kv_scales = True
    buf = torch.ones(1)
    attn.k_scale = buf

    class MockModel:
        def modules(self):
            yield attn

    apply_fp8_scales(MockModel(), FP8ScaleSidecar(k_scale=0.05, v_scale=0.07))
    assert attn._k_scale == 0.05 and attn._v_scale == 0.07
    assert attn.calculate_kv_scales is False
    assert attn.k_scale is buf and buf.item() == pytest.approx(0.05)


def test_codecs_refuse_host_tensors():
    for f in ("fp8_e4m3", "int4_sym_block", "int4_asym_g32"):
        with pytest.raises(RuntimeError, match="GPU"):
            get_codec(f).compress(torch.randn(2, 16, 2, 64))


# ----------------------------------------------------------- dispatch ----


def test_dispatch_registry_on_cpu():
    from korith_vllm_ext.kernels import dispatch

    # without a device the version is 0; the storage-format rule still picks
    # the HIP kernel, and unknown formats get the dense-attention entry point
    assert dispatch.dispatch_kernel("int4_sym", "fp8_e4m3") is dispatch.hip_decode_attention
    assert dispatch.dispatch_kernel("nvfp4", "nvfp4") is dispatch.fallback_fp16_kernel
    assert (dispatch.GFX950_VERSION, "int4_sym", "fp8_e4m3") in dispatch.KERNEL_DISPATCH


def test_decode_entry_refuses_host_tensors():
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention

    q = torch.randn(1, 2, 1, 64)
    k = torch.randn(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        int4_decode_attention(q, k, k)


# ---- positional attention: which CompressedKV the in-place INT4 kernel takes --


def _int4_sym_kv(shape, device="cpu"):
    """A CompressedKV shaped as the int4_sym codec leaves one: codes uint8
    [*shape[:-1], D / 2] and fp16 scales [D] (values irrelevant here)."""
    from korith_vllm_ext.codecs import CompressedKV

    D = shape[-1]
    return CompressedKV(format="int4_sym",
                        data=torch.zeros(*shape[:-1], D // 2, dtype=torch.uint8, device=device),
                        scales=torch.ones(D, dtype=torch.float16, device=device), shape=shape,
                        dtype_original=torch.bfloat16)


def test_int4_sym_operands_accepts_the_codec_layout_only():
    """_int4_sym_operands (kernels/dispatch.py) hands the in-place kernel the
    codes and scales only when they are laid out as the codec writes them,
    on q's device, with q's lead dims; anything else is None (the caller
    then restores and runs the dense kernel)."""
    from korith_vllm_ext.codecs import CompressedKV
    from korith_vllm_ext.kernels.dispatch import _int4_sym_operands

    q = torch.zeros(2, 8, 1, 128, dtype=torch.bfloat16)
    good = _int4_sym_kv((2, 4, 300, 128))
    ops = _int4_sym_operands(good, q)
    assert ops is not None and ops[0] is good.data and ops[1] is good.scales
    # other formats, plain tensors
    fp8 = CompressedKV(format="fp8_e4m3", data=good.data, scales=good.scales, shape=good.shape)
    assert _int4_sym_operands(fp8, q) is None
    assert _int4_sym_operands(torch.zeros(2, 4, 300, 128), q) is None
    # lead dims or head_dim not q's
    assert _int4_sym_operands(_int4_sym_kv((3, 4, 300, 128)), q) is None
    assert _int4_sym_operands(_int4_sym_kv((2, 4, 300, 64)), q) is None
    assert _int4_sym_operands(_int4_sym_kv((4, 300, 128)), q) is None
    # codes: wrong dtype, shape or a non-contiguous view
    bad = _int4_sym_kv((2, 4, 300, 128))
    bad.data = bad.data.to(torch.int8)
    assert _int4_sym_operands(bad, q) is None
    bad = _int4_sym_kv((2, 4, 300, 128))
    bad.data = torch.zeros(2, 4, 300, 128, dtype=torch.uint8)
    assert _int4_sym_operands(bad, q) is None
    bad = _int4_sym_kv((2, 4, 300, 128))
    bad.data = torch.zeros(2, 4, 64, 300, dtype=torch.uint8).transpose(-1, -2)
    assert _int4_sym_operands(bad, q) is None
    # scales: wrong dtype or count
    bad = _int4_sym_kv((2, 4, 300, 128))
    bad.scales = bad.scales.float()
    assert _int4_sym_operands(bad, q) is None
    bad = _int4_sym_kv((2, 4, 300, 128))
    bad.scales = torch.ones(64, dtype=torch.float16)
    assert _int4_sym_operands(bad, q) is None


def test_int4_sym_attention_declines_without_launching():
    """int4_sym_attention returns None before any device work for head dims
    the split kernel does not take and for K/V it cannot read in place."""
    from korith_vllm_ext.kernels.dispatch import int4_sym_attention

    q80 = torch.zeros(1, 4, 1, 80, dtype=torch.bfloat16)
    assert int4_sym_attention(q80, _int4_sym_kv((1, 4, 16, 80)), _int4_sym_kv((1, 4, 16, 80)),
                              None, None) is None
    q = torch.zeros(1, 4, 1, 128, dtype=torch.int32)
    assert int4_sym_attention(q, _int4_sym_kv((1, 4, 16, 128)), _int4_sym_kv((1, 4, 16, 128)),
                              None, None) is None
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    k = _int4_sym_kv((1, 4, 16, 128))
    assert int4_sym_attention(q, k, _int4_sym_kv((1, 4, 17, 128)), None, None) is None
    assert int4_sym_attention(q, k, torch.zeros(1, 4, 16, 128), None, None) is None
    # GQA needs the query heads to be a multiple of the KV heads
    q3 = torch.zeros(1, 6, 1, 128, dtype=torch.bfloat16)
    assert int4_sym_attention(q3, k, k, None, None) is None
