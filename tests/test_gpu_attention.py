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


def _dense_abi(q, k, v, mask, scale, workspace):
    """amf_dense_attn through the C ABI with an explicit workspace (None:
    the single-pass kernel), fp32 output."""
    import amf_hip

    B, Hq, Tq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    out = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    mptr, ms = (0, (0, 0, 0, 0)) if mask is None else (mask.data_ptr(), mask.stride())
    wptr = workspace.data_ptr() if workspace is not None else None
    wsb = workspace.numel() if workspace is not None else 0
    amf_hip.call("amf_dense_attn", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 amf_hip.dtype_tag(q.dtype), mptr, *ms, out.data_ptr(), amf_hip.DTYPE_F32,
                 B, Hq, Hkv, Tq, T, D, scale, wptr, wsb, amf_hip.stream_handle(DEV))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("dtype,B,Hq,Hkv,Tq,T,D,masked", [
    (torch.bfloat16, 1, 32, 8, 1, 20000, 128, False),  # few rows: many splits
    (torch.float16, 2, 8, 1, 1, 4097, 64, True),        # GQA 8, ragged last chunk
    (torch.float32, 1, 4, 2, 2, 3000, 256, True),
    (torch.bfloat16, 3, 6, 3, 1, 65, 128, False),       # units not a multiple of 8
    (torch.bfloat16, 2, 6, 1, 1, 700, 64, False),       # GQA 6: 3 waves of 2 heads
    (torch.float16, 1, 12, 4, 2, 333, 128, True),       # GQA 3: one head per wave
])
def test_dense_split_path_matches_f64_and_single_pass(dtype, B, Hq, Hkv, Tq, T, D, masked):
    """The split (flash-decoding) path against float64 attention and the
    single-pass kernel, with masks that empty whole splits and whole rows."""
    import amf_hip

    print(f"dense split case {dtype} B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} T={T} D={D}", flush=True)
    g = torch.Generator().manual_seed(T + D)
    q = torch.randn(B, Hq, Tq, D, generator=g).to(dtype)
    k = (torch.randn(B, Hkv, T, D, generator=g) * 2).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    mask = None
    if masked:
        mask = torch.zeros(B, Hq, Tq, T)
        mask[:, :, :, : T // 2] = float("-inf")   # the first half of the splits see nothing
        mask[0, 1, 0, :] = float("-inf")          # one row sees nothing: NaN
        mask[:, :, :, T - 7] = -2.5
    ref = oatt.dense_attention_f64(_f64(q), _f64(k), _f64(v), 0.2,
                                   None if mask is None else mask.numpy())
    wsb = int(amf_hip.load().amf_dense_attn_workspace_bytes(B, Hq, Hkv, Tq, T, D))
    assert wsb > 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    dm = None if mask is None else mask.to(DEV)
    split = _dense_abi(dq, dk, dv, dm, 0.2, ws)
    single = _dense_abi(dq, dk, dv, dm, 0.2, None)
    nan_ref = np.isnan(ref)
    assert (np.isnan(split) == nan_ref).all() and (np.isnan(single) == nan_ref).all()
    ok = ~nan_ref
    assert float(np.abs(split[ok] - ref[ok]).max()) <= 1e-4
    assert float(np.abs(split[ok] - single[ok]).max()) <= 1e-4
    # a second call on the same workspace at a shorter context reuses it
    T2 = T // 3 + 1
    ref2 = oatt.dense_attention_f64(_f64(q), _f64(k[:, :, :T2]), _f64(v[:, :, :T2]), 0.2)
    split2 = _dense_abi(dq, dk[:, :, :T2].contiguous(), dv[:, :, :T2].contiguous(), None, 0.2, ws)
    assert float(np.abs(split2 - ref2).max()) <= 1e-4


@pytest.mark.parametrize("dtype,lead,Hq,Hkv,Tq,T,D,masked", [
    (torch.bfloat16, (4,), 32, 8, 1, 8192, 128, False),   # the positional decode workload
    (torch.float16, (2,), 8, 1, 1, 1000, 64, True),
    (torch.float32, (), 4, 2, 2, 300, 256, True),          # no lead dims: [H, T, D]
    (torch.bfloat16, (2, 3), 4, 4, 1, 77, 128, False),     # two lead dims
    (torch.float16, (3,), 8, 4, 3, 200, 128, False),       # GQA 2, three query rows
])
def test_int4_sym_fused_matches_restore_path(dtype, lead, Hq, Hkv, Tq, T, D, masked):
    """int4_sym CompressedKV K/V read in place (amf_int4_sym_dense_attn)
    against the restore-then-attend path (decompress_to + amf_dense_attn) and
    float64 attention.  head_dim 128 with bf16 / fp16 queries and no mask runs
    the MFMA kernel, which attends over the exactly dequantized (c - 8) s (the
    restore rounds them to q's dtype): it is held to float64 attention over
    the exact values and to the restore path within the attention tolerance.
    The other cases dequantize as the restore does and match it exactly."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.kernels import dense_attention, int4_sym_attention

    print(f"int4_sym fused case {dtype} lead={lead} Hq={Hq} Hkv={Hkv} Tq={Tq} T={T} D={D}",
          flush=True)
    g = torch.Generator().manual_seed(T * 7 + D)
    q = torch.randn(*lead, Hq, Tq, D, generator=g).to(dtype).to(DEV)
    k = (torch.randn(*lead, Hkv, T, D, generator=g) * 2).to(dtype).to(DEV)
    v = torch.randn(*lead, Hkv, T, D, generator=g).to(dtype).to(DEV)
    codec = get_codec("int4_sym")
    ck, cv = codec.compress(k), codec.compress(v)
    mask = None
    if masked:
        mask = torch.zeros(Tq, T)
        mask[:, : T // 3] = float("-inf")
        mask[-1, T - 1] = -1.5
        mask = mask.to(DEV)
    fused = int4_sym_attention(q, ck, cv, 0.25, mask, torch.float32)
    assert fused is not None
    kd = codec.decompress_to(ck, dtype)
    vd = codec.decompress_to(cv, dtype)
    two = dense_attention(q, kd, vd, 0.25, mask, torch.float32)
    torch.cuda.synchronize()
    diff = float((fused - two).abs().max())
    print(f"fused vs restore path: max |diff| {diff:.3e}", flush=True)
    mfma = D == 128 and mask is None and dtype != torch.float32
    if mfma:
        kd = codec.decompress_to(ck, torch.float32)  # (c - 8) s, exact in fp32
        vd = codec.decompress_to(cv, torch.float32)
    else:
        assert diff <= 1e-6
    # the float64 oracle takes [batch, heads, tokens, head_dim]
    ref = oatt.dense_attention_f64(_f64(q.reshape(-1, Hq, Tq, D)), _f64(kd.reshape(-1, Hkv, T, D)),
                                   _f64(vd.reshape(-1, Hkv, T, D)), 0.25,
                                   None if mask is None else mask.cpu().numpy())
    err = float(np.abs(fused.reshape(-1, Hq, Tq, D).cpu().numpy() - ref).max())
    print(f"fused vs float64: max |diff| {err:.3e}", flush=True)
    # the MFMA kernel's error is its fp32 accumulation of sum q s c over the
    # raw codes, a few times the score (measured up to 9.6e-5 here)
    assert err <= (3e-4 if mfma else 1e-4)
    if mfma:
        # the restore path's own distance from the exact values (the rounding
        # of the restored K/V) accounts for its distance from this one
        err_two = float(np.abs(two.reshape(-1, Hq, Tq, D).cpu().numpy() - ref).max())
        print(f"restore path vs float64: max |diff| {err_two:.3e}", flush=True)
        assert diff <= err_two + 1e-4
    # q's dtype out: the fp32 result rounded once
    out = int4_sym_attention(q, ck, cv, 0.25, mask)
    assert out.dtype == dtype and torch.equal(out, fused.to(dtype))


@pytest.mark.parametrize("case", ["gqa8_ragged", "gqa16", "gqa12", "gqa6", "rising", "flat",
                                  "large_q", "one_token"])
def test_int4_sym_mfma_edge_cases(case):
    """The MFMA INT4-sym kernel (head_dim 128, no mask) against float64
    attention over the exactly dequantized K/V on inputs that drive its
    corners: GQA 8 and 16 (one wave for the group) over ragged splits, GQA 12
    and 6 (three waves of 4 and of 2 heads per group); scores rising
    along the context (the running max moves inside splits, by more than
    the rescale slack); near-uniform softmax over 6000 tokens (the centred V
    sums); large fp16 queries (the per-wave power-of-two scaling of q s);
    a one-token context."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.kernels import int4_sym_attention

    dtype, B, Hq, Hkv, T = torch.bfloat16, 2, 8, 2, 3000
    q_mul, scale = 1.0, 0.25
    if case == "gqa8_ragged":
        B, Hq, Hkv, T = 3, 16, 2, 5000 + 17
    elif case == "gqa16":
        B, Hq, Hkv, T = 2, 32, 2, 3000 + 5
    elif case == "gqa12":
        B, Hq, Hkv, T = 2, 24, 2, 2000
    elif case == "gqa6":
        B, Hq, Hkv, T = 2, 12, 2, 2000
    elif case == "flat":
        q_mul, T = 1e-3, 6000
    elif case == "large_q":
        dtype, q_mul = torch.float16, 30.0
    elif case == "one_token":
        T = 1
    print(f"int4_sym mfma edge case {case}: B={B} Hq={Hq} Hkv={Hkv} T={T}", flush=True)
    g = torch.Generator().manual_seed(len(case) * 131 + T)
    q = (torch.randn(B, Hq, 1, 128, generator=g) * q_mul).to(dtype).to(DEV)
    k = torch.randn(B, Hkv, T, 128, generator=g) * 2
    if case == "rising":
        k = k * (1.0 + torch.arange(T, dtype=torch.float32) / 64.0)[:, None]
    v = torch.randn(B, Hkv, T, 128, generator=g)
    v[..., 5] += 40.0  # an outlier channel: a large V scale
    codec = get_codec("int4_sym")
    ck, cv = codec.compress(k.to(dtype).to(DEV)), codec.compress(v.to(dtype).to(DEV))
    out = int4_sym_attention(q, ck, cv, scale, None, torch.float32)
    torch.cuda.synchronize()
    kd = codec.decompress_to(ck, torch.float32)  # (c - 8) s, exact in fp32
    vd = codec.decompress_to(cv, torch.float32)
    ref = oatt.dense_attention_f64(_f64(q), _f64(kd), _f64(vd), scale)
    err = np.abs(out.cpu().numpy() - ref)
    vmax = float(np.abs(_f64(vd)).max())
    kx = np.repeat(_f64(kd), Hq // Hkv, axis=1)
    smax = float(np.abs(np.einsum("bhqd,bhtd->bhqt", _f64(q), kx)).max()) * scale / math.log(2)
    print(f"max |diff| {err.max():.3e} (max |v| {vmax:.2f}, max |score| {smax:.1f} in log2 units)",
          flush=True)
    assert np.isfinite(out.cpu().numpy()).all()
    # fp32 accumulation of the exact products, relative to the V range, plus
    # the fp32 rounding of scores this large (an error of 2^-22 |score| in a
    # score moves the weights by that much relative)
    assert err.max() <= 3e-4 * max(1.0, vmax / 4.0) + 2.0 ** -22 * smax * vmax


def test_int4_sym_fused_empty_context_and_declines():
    """kv_len 0 gives zeros, all -inf scores NaN; head dims outside
    64/128/256 (32 here) and other formats decline (None), so the caller restores and
    runs dense attention."""
    import amf_hip
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.kernels import int4_sym_attention

    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 1, 128, generator=g).to(torch.bfloat16).to(DEV)
    out = torch.full((2, 4, 1, 128), 7.0, device=DEV)
    amf_hip.call("amf_int4_sym_dense_attn", q.data_ptr(), amf_hip.DTYPE_BF16, None, None, None,
                 None, None, 0, 0, 0, 0, out.data_ptr(), amf_hip.DTYPE_F32, 2, 4, 4, 1, 0, 128,
                 0.1, None, 0, amf_hip.stream_handle(DEV))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
    codec = get_codec("int4_sym")
    k0 = codec.compress(torch.randn(2, 4, 16, 128, generator=g).to(torch.bfloat16).to(DEV))
    z = int4_sym_attention(q, k0, k0, None, torch.full((1, 16), float("-inf"), device=DEV))
    assert z is not None and torch.isnan(z.float()).all()
    q32 = torch.randn(2, 4, 1, 32, generator=g).to(torch.bfloat16).to(DEV)
    k32 = codec.compress(torch.randn(2, 4, 16, 32, generator=g).to(torch.bfloat16).to(DEV))
    assert int4_sym_attention(q32, k32, k32, None, None) is None
    kf = get_codec("int4_sym_block").compress(
        torch.randn(2, 4, 16, 128, generator=g).to(torch.bfloat16).to(DEV))
    assert int4_sym_attention(q, kf, kf, None, None) is None


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


def test_int4_sym_attention_in_a_hip_graph():
    """The positional INT4-sym call captured in a HIP graph (the split and
    merge launches, the split scratch taken for the capture): every replay,
    with eager calls of the same shape on the default stream in between,
    gives the eager result bit for bit."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.kernels import int4_sym_attention

    g = torch.Generator().manual_seed(77)
    q = torch.randn(2, 8, 1, 128, generator=g).to(torch.bfloat16).to(DEV)
    codec = get_codec("int4_sym")
    ck = codec.compress(torch.randn(2, 2, 1500, 128, generator=g).to(torch.bfloat16).to(DEV))
    cv = codec.compress(torch.randn(2, 2, 1500, 128, generator=g).to(torch.bfloat16).to(DEV))
    want = int4_sym_attention(q, ck, cv, None, None, torch.float32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        int4_sym_attention(q, ck, cv, None, None, torch.float32)  # warm-up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = int4_sym_attention(q, ck, cv, None, None, torch.float32)
    for _ in range(3):
        got.zero_()
        graph.replay()
        eager = int4_sym_attention(q, ck, cv, None, None, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(eager, want)


def test_paged_decode_in_a_hip_graph():
    """The paged INT4 decode (the decode launch and its merge) captured in a
    HIP graph over caller-owned output and workspace: every replay, with an
    eager call on other buffers in between, gives the eager result bit for
    bit, and replays follow context lengths changed in place."""
    import amf_hip
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention

    g = torch.Generator().manual_seed(321)
    Hkv, R, D, pool = 2, 4, 128, 64
    pages = gen.kv_values((2, pool, 16, Hkv, D), D, g, True)
    ckv = get_codec("int4_asym_g32").compress(pages.to(DEV))
    ctx = torch.tensor([700, 37, 1000, 16], dtype=torch.int32, device=DEV)
    bt = torch.stack([torch.randperm(pool, generator=g)[:63] for _ in range(4)]).to(torch.int32)
    bt = bt.to(DEV)
    q = torch.randn(4, Hkv * R, D, generator=g).to(torch.bfloat16).to(DEV)
    wsb = amf_hip.decode_workspace_bytes(4, Hkv * R, Hkv, D, 63 * 16)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    out = torch.empty(4, Hkv * R, D, dtype=torch.float32, device=DEV)
    kw = dict(block_tables=bt, context_lens=ctx, out=out, workspace=ws)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        int4_decode_attention(q, ckv, **kw)  # warm-up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        int4_decode_attention(q, ckv, **kw)
    for lens in ([700, 37, 1000, 16], [5, 999, 1, 512], [700, 37, 1000, 16]):
        ctx.copy_(torch.tensor(lens, dtype=torch.int32))
        out.zero_()
        graph.replay()
        eager = int4_decode_attention(q, ckv, block_tables=bt, context_lens=ctx,
                                      out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), lens


@pytest.mark.parametrize("D,int4", [(128, False), (128, True), (64, False), (256, True)])
def test_split_attention_many_splits(D, int4):
    """One query row over a long context: hundreds of splits, so the merge
    reads weights and accumulators past its first register batch and its
    first 64 (m, l) pairs; dense bf16 K/V and int4_sym K/V (the MFMA kernel at
    head_dim 128, the VALU one at 256) against float64 attention."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.kernels import dense_attention, int4_sym_attention

    T = 60000 if D == 256 else 100000
    g = torch.Generator().manual_seed(D * 7 + int4)
    q = torch.randn(1, 1, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    k = (torch.randn(1, 1, T, D, generator=g) * 2).to(torch.bfloat16).to(DEV)
    v = torch.randn(1, 1, T, D, generator=g).to(torch.bfloat16).to(DEV)
    if int4:
        codec = get_codec("int4_sym")
        ck, cv = codec.compress(k), codec.compress(v)
        out = int4_sym_attention(q, ck, cv, None, None, torch.float32)
        # the MFMA kernel attends over the exact (c - 8) s, the VALU one over
        # the values the restore writes in q's dtype
        kv_dtype = torch.float32 if D == 128 else q.dtype
        k = codec.decompress_to(ck, kv_dtype)
        v = codec.decompress_to(cv, kv_dtype)
    else:
        out = dense_attention(q, k, v, None, None, torch.float32)
    torch.cuda.synchronize()
    ref = oatt.dense_attention_f64(_f64(q), _f64(k), _f64(v))
    err = float(np.abs(out.cpu().numpy() - ref).max())
    print(f"D={D} int4={int4} T={T}: max |diff| {err:.3e}", flush=True)
    # fp32 accumulation over 1e5 tokens (the MFMA kernel: of the raw-code
    # products, measured 9.1e-6); the other cases measured below 1e-7
    assert err <= (1e-4 if (int4 and D == 128) else 1e-5)


def test_split_scratch_per_stream():
    """The attention wrappers' split-K scratch is one buffer per (device,
    stream): calls on two streams at once each use their own and both give
    the single-stream result."""
    from korith_vllm_ext.kernels import dense_attention
    from korith_vllm_ext.kernels import dispatch

    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 8, 1, 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(2, 2, 3000, 128, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(2, 2, 3000, 128, generator=g).to(torch.bfloat16).to(DEV)
    want = dense_attention(q, k, v, None, None, torch.float32)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            outs.append([dense_attention(q, k, v, None, None, torch.float32) for _ in range(4)])
    torch.cuda.synchronize()
    for o in outs:
        for x in o:
            assert torch.equal(x, want)
    idx = DEV.index if DEV.index is not None else torch.cuda.current_device()
    bufs = {key: t.data_ptr() for key, t in dispatch._SCRATCH.items() if key[0] == idx}
    assert (idx, s1.cuda_stream) in bufs and (idx, s2.cuda_stream) in bufs
    assert bufs[(idx, s1.cuda_stream)] != bufs[(idx, s2.cuda_stream)]
