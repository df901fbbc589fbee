"""The codec API (korith_vllm_ext.codecs) on the GPU, mirroring the
reference's codec tests (tests/test_codecs.py, tests/test_fp8_restore.py) and
checking the reference formats bit for bit against the oracle on dense
tensors of any [..., tokens, heads, head_dim] shape and dtype."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codecs as oc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

# tests/test_codecs.py:33-41 (reference formats) and the new formats.
TOLERANCES = {"fp8_e4m3": 0.05, "int4_sym": 0.20, "int4_sym_block": 0.22,
              "fp8_e4m3_ph": 0.05, "int4_asym_g32": 0.10}


@pytest.fixture
def sample_kv():
    torch.manual_seed(0)
    return torch.randn(2, 256, 8, 128).to(DEV)


@pytest.mark.parametrize("fmt", list(TOLERANCES))
def test_roundtrip_shape_dtype_error_ratio(fmt, sample_kv):
    from korith_vllm_ext.codecs import get_codec

    codec = get_codec(fmt)
    blob = codec.compress(sample_kv)
    out16 = codec.decompress_to(blob, target_dtype=torch.float16)
    assert out16.shape == sample_kv.shape and out16.dtype == torch.float16
    out = codec.decompress_to(blob, target_dtype=torch.float32)
    rel = (out - sample_kv).norm().item() / sample_kv.norm().item()
    assert rel < TOLERANCES[fmt], (fmt, rel)
    ratio = blob.nbytes() / blob.original_bytes()
    assert ratio < codec.memory_ratio() * 1.5 + 0.05, (fmt, ratio)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 256, 8, 128), (300, 4, 64), (3, 2, 40, 2, 64),
                                   (2, 8, 1024, 128), (3, 5, 7, 64)])
def test_reference_formats_bitexact(dtype, shape):
    """Codes, scales and restored values of the reference formats against the
    oracle.  Shapes whose row count has a power-of-two factor of at least
    2048 / head_dim are compressed as pages of rows ((2, 256, 8, 128),
    (3, 2, 40, 2, 64) and the [batch, kv_heads, tokens, head_dim] tensor
    (2, 8, 1024, 128)); the others as pages of dim -3."""
    from korith_vllm_ext.codecs import get_codec

    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=g) * 3).to(dtype)
    dx = x.to(DEV)
    rows = x.numel() // shape[-1]
    flat = any(rows % b == 0 and b * shape[-1] >= 2048 for b in (16, 32, 64, 128, 256))
    # fp8_e4m3: codes, the Python-double tensor_scale and the decompression
    c = get_codec("fp8_e4m3").compress(dx)
    assert (c.meta["_layout"].num_heads == 1 and c.meta["_layout"].n_planes == 1) == flat
    codes, scale = oc.fp8_tensor_compress(x)
    assert c.data.dtype == torch.float8_e4m3fn and c.data.shape == x.shape
    assert torch.equal(c.data.view(torch.uint8).cpu(), codes)
    assert c.tensor_scale == scale and c.meta["sidecar"].k_scale == scale
    assert torch.equal(c.scales.cpu(), oc.fp8_sidecar(scale))
    for tdt in (torch.float32, dtype):
        got = get_codec("fp8_e4m3").decompress_to(c, tdt).cpu()
        assert torch.equal(got, oc.fp8_tensor_decompress(codes, scale, tdt))
    # int4_sym: packed codes, fp16 channel scales, decompression
    c = get_codec("int4_sym").compress(dx)
    assert (c.meta["_layout"].num_heads == 1 and c.meta["_layout"].n_planes == 1) == flat
    packed, sc = oc.int4_channel_compress(x)
    assert torch.equal(c.data.cpu(), packed) and torch.equal(c.scales.cpu(), sc)
    got = get_codec("int4_sym").decompress_to(c, torch.float32).cpu()
    assert torch.equal(got, oc.int4_channel_decompress(packed, sc, x.shape, torch.float32))
    # int4_sym_block: 128-token blocks along dim -3
    c = get_codec("int4_sym_block").compress(dx)
    packed, sc, meta = oc.int4_block_compress(x)
    assert torch.equal(c.data.cpu(), packed) and torch.equal(c.scales.cpu(), sc)
    got = get_codec("int4_sym_block").decompress_to(c, torch.float32).cpu()
    assert torch.equal(got, oc.int4_block_decompress(packed, sc, x.shape, meta, torch.float32))


def test_fp8_sidecar_and_drift():
    """tests/test_fp8_restore.py:55-63, 101-146."""
    from korith_vllm_ext.codecs import get_codec

    codec = get_codec("fp8_e4m3")
    torch.manual_seed(1)
    raw = (torch.randn(4, 128, 8, 128) * 0.3).to(DEV)
    blob = codec.compress(raw)
    sidecar = blob.meta["sidecar"]
    assert sidecar.k_scale > 0 and sidecar.v_scale > 0
    assert abs(blob.tensor_scale - sidecar.k_scale) < 1e-9
    restored = codec.decompress_to(blob, target_dtype=torch.float32)
    correct_err = (restored - raw).norm().item() / raw.norm().item()
    assert correct_err < 0.05
    restored_fp32 = blob.data.to(torch.float32)
    new_scale = float(restored_fp32.abs().amax().clamp_min(1e-8)) / 448.0
    drifted = restored_fp32 * new_scale
    drifted_err = (drifted.view_as(raw) - raw).norm().item() / raw.norm().item()
    assert correct_err <= drifted_err + 1e-6


def test_page_tensor_is_paged_per_page():
    """A layer page tensor [2, nb, bs, H, D] is compressed page by page (the
    reference's codecs on put_from_vllm's stacked gather): int4_sym_block
    gives one scale per (K/V, page)."""
    from korith_vllm_ext.codecs import get_codec

    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 7, 16, 8, 128, generator=g).to(torch.bfloat16)
    c = get_codec("int4_sym_block").compress(x.to(DEV))
    packed, sc, meta = oc.int4_block_compress(x)
    assert tuple(c.scales.shape) == (2, 7, 1)
    assert torch.equal(c.data.cpu(), packed)
    assert torch.equal(c.scales.cpu().reshape(sc.shape), sc)
