"""int4_decode_attention on the GPU: the positional (dense) contract through
amf_dense_attn, and the paged INT4 contract through the dispatch entry point,
against float64 attention."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import codecs as oc
from oracle import gen

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype,B,Hq,Hkv,Tq,T,D", [
    (torch.bfloat16, 2, 8, 8, 1, 200, 64),
    (torch.float16, 3, 8, 2, 1, 1000, 128),
    (torch.float32, 1, 4, 4, 3, 63, 80),
    (torch.bfloat16, 2, 4, 1, 2, 130, 100),  # head_dim not a multiple of 8: scalar loads
    (torch.bfloat16, 1, 2, 2, 1, 1, 256),
])
def test_dense_attention_f32_and_rounded(dtype, B, Hq, Hkv, Tq, T, D):
    from korith_vllm_ext.kernels import dense_attention

    g = torch.Generator().manual_seed(B * 1000 + T)
    q = torch.randn(B, Hq, Tq, D, generator=g).to(dtype)
    k = (torch.randn(B, Hkv, T, D, generator=g) * 2).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    ref = oatt.dense_attention_f64(_f64(q), _f64(k), _f64(v))
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    out32 = dense_attention(dq, dk, dv, None, None, torch.float32)
    torch.cuda.synchronize()
    err = float(np.abs(out32.cpu().numpy() - ref).max())
    assert err <= 1e-4, err
    out = dense_attention(dq, dk, dv, None, None)
    assert out.dtype == dtype and out.shape == q.shape
    assert torch.equal(out.cpu(), out32.cpu().to(dtype))


def test_dense_attention_mask_scale_and_edges():
    from korith_vllm_ext.kernels import dense_attention

    g = torch.Generator().manual_seed(7)
    B, H, Tq, T, D = 2, 4, 3, 90, 64
    q = torch.randn(B, H, Tq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    # causal-style mask broadcast over batch and heads, plus a row of all -inf
    mask = torch.zeros(Tq, T)
    for i in range(Tq):
        mask[i, T - Tq + i + 1:] = float("-inf")
    mask[1, 5] = -3.0
    mask4 = mask.clone()
    mask4[2, :] = float("-inf")
    ref = oatt.dense_attention_f64(_f64(q), _f64(k), _f64(v), 0.3, mask4.numpy())
    out = dense_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0.3, mask4.to(DEV), torch.float32)
    got = out.cpu().numpy()
    assert np.isnan(got[:, :, 2]).all() and np.isnan(ref[:, :, 2]).all()
    assert float(np.abs(got[:, :, :2] - ref[:, :, :2]).max()) <= 1e-4
    # empty context -> zeros (an empty sum, as matmul over a zero-length axis)
    z = dense_attention(q.to(DEV), k[:, :, :0].to(DEV), v[:, :, :0].to(DEV), None, None)
    assert torch.count_nonzero(z).item() == 0


def test_positional_contract_with_compressed_kv():
    """int4_decode_attention(q, CompressedKV, CompressedKV): K/V decompressed by
    the HIP codec, attention by the HIP kernel (dispatch.py:117-152 flow)."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention

    g = torch.Generator().manual_seed(11)
    B, H, T, D = 2, 8, 300, 128
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    for fmt in ("int4_sym", "int4_sym_block", "fp8_e4m3"):
        codec = get_codec(fmt)
        ck, cv = codec.compress(k), codec.compress(v)
        kd = codec.decompress_to(ck, torch.bfloat16)
        vd = codec.decompress_to(cv, torch.bfloat16)
        out = int4_decode_attention(q, ck, cv)
        torch.cuda.synchronize()
        assert out.shape == q.shape and out.dtype == q.dtype
        ref = oatt.dense_attention_f64(_f64(q), _f64(kd), _f64(vd))
        d = np.abs(out.float().cpu().numpy() - ref)
        assert float((d - (2e-2 + np.abs(ref) * 2.0 ** -8)).max()) <= 0.0, (fmt, float(d.max()))


@pytest.mark.parametrize("R", [1, 4, 8])
def test_paged_contract_int4_pool(R):
    """int4_decode_attention(q, kv_pool, block_tables=..., context_lens=...)."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention

    g = torch.Generator().manual_seed(100 + R)
    Hkv, D, pool = 2, 128, 96
    pages = gen.kv_values((2, pool, 16, Hkv, D), D, g, True)
    ckv = get_codec("int4_asym_g32").compress(pages.to(DEV))
    ctx = torch.tensor([1, 16, 17, 700, 1200], dtype=torch.int32)
    n_max = (int(ctx.max()) + 15) // 16
    bt = torch.stack([torch.randperm(pool, generator=g)[:n_max] for _ in ctx]).to(torch.int32)
    q = torch.randn(len(ctx), Hkv * R, 1, D, generator=g).to(torch.bfloat16)
    out = int4_decode_attention(q.to(DEV), ckv, block_tables=bt.to(DEV),
                                context_lens=ctx.to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert out.shape == q.shape
    kv32 = oc.int4_asym_dequant_f32(*oc.int4_asym_quantize(pages)).numpy()
    ref = oatt.paged_decode_f64(q[:, :, 0].float().numpy(), kv32[0], kv32[1], bt.numpy(),
                                ctx.numpy())
    err = float(np.abs(out[:, :, 0].cpu().numpy() - ref).max())
    assert err <= 2e-2, err


def test_paged_contract_caller_buffers():
    """The keyword path with caller-owned `out` and `workspace`: correct
    buffers are used as given (same result as without them); a buffer on the
    CPU, non-contiguous, of the wrong shape or dtype is refused with
    ValueError before any launch (the output stays untouched)."""
    import amf_hip
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention

    g = torch.Generator().manual_seed(123)
    Hkv, R, D, pool = 2, 4, 128, 40
    pages = gen.kv_values((2, pool, 16, Hkv, D), D, g, True)
    ckv = get_codec("int4_asym_g32").compress(pages.to(DEV))
    ctx = torch.tensor([100, 333, 5], dtype=torch.int32, device=DEV)
    bt = torch.stack([torch.randperm(pool, generator=g)[:21] for _ in range(3)]).to(torch.int32)
    bt = bt.to(DEV)
    q = torch.randn(3, Hkv * R, D, generator=g).to(torch.bfloat16).to(DEV)
    want = int4_decode_attention(q, ckv, block_tables=bt, context_lens=ctx,
                                 out_dtype=torch.float32)
    wsb = amf_hip.decode_workspace_bytes(3, Hkv * R, Hkv, D, 21 * 16)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    out = torch.full((3, Hkv * R, D), 9.0, dtype=torch.float32, device=DEV)
    got = int4_decode_attention(q, ckv, block_tables=bt, context_lens=ctx, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr() and torch.equal(got, want)
    sentinel = torch.full_like(out, 9.0)
    bad = [
        dict(out=torch.empty(3, Hkv * R, D)),                                      # on the CPU
        dict(out=torch.empty(3, D, Hkv * R, device=DEV).transpose(1, 2)),          # strided
        dict(out=torch.empty(3, Hkv * R, D + 8, device=DEV)),                      # shape
        dict(out=sentinel.clone(), out_dtype=torch.float16),                       # dtype
        dict(out=sentinel.clone(), workspace=torch.empty(wsb, dtype=torch.uint8)),  # ws on CPU
        dict(out=sentinel.clone(),
             workspace=torch.empty(2 * wsb, dtype=torch.uint8, device=DEV)[::2]),  # strided ws
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            int4_decode_attention(q, ckv, block_tables=bt, context_lens=ctx, **kw)
        o = kw["out"]
        if o.is_cuda and o.is_contiguous() and o.shape == sentinel.shape:
            torch.cuda.synchronize()
            assert torch.equal(o, sentinel)


def test_dispatch_resolves_to_hip_kernel():
    from korith_vllm_ext.kernels import dispatch

    assert dispatch.get_current_sm_version() == dispatch.GFX950_VERSION
    assert dispatch.dispatch_kernel("int4_sym", "fp8_e4m3") is dispatch.hip_decode_attention
    assert dispatch.try_load_cuda_extension() is not None
