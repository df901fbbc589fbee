"""The reference's kernel tests (tests/test_kernels.py:29-133), run through
the HIP positional path: fallback_fp16_kernel and int4_decode_attention on
the GPU (split-K dense attention, and the INT4-sym kernel that reads the
codes in place), with the reference's inputs, seeds and tolerances.  The
reference compares against torch's scaled_dot_product_attention in fp16;
here the reference attention is float32 on the CPU (the same formula, more
exact), and the GPU's fp16 output is held to the same relative-L2 bounds."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _sdpa_cpu(q, k, v, mask=None):
    """softmax(q k^T / sqrt(D) + mask) v in float32 on the CPU."""
    q, k, v = q.float().cpu(), k.float().cpu(), v.float().cpu()
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / q.shape[-1] ** 0.5
    if mask is not None:
        s = s + mask.float().cpu()
    return torch.matmul(torch.softmax(s, dim=-1), v)


def _rel(out, ref):
    return ((out.float().cpu() - ref).norm() / ref.norm()).item()


def _make_qkv(B=2, H=4, T=128, D=128):
    # tests/test_kernels.py:29-33
    q = torch.randn(B, H, 1, D).half()
    k = torch.randn(B, H, T, D).half()
    v = torch.randn(B, H, T, D).half()
    return q, k, v


def test_fallback_matches_sdpa():
    """tests/test_kernels.py:36-41."""
    from korith_vllm_ext.kernels import fallback_fp16_kernel

    torch.manual_seed(0)
    q, k, v = _make_qkv()
    out = fallback_fp16_kernel(q.to(DEV), k.to(DEV), v.to(DEV))
    assert out.dtype == torch.float16 and out.device.type == "cuda"
    assert _rel(out, _sdpa_cpu(q, k, v)) < 1e-2


@pytest.mark.parametrize("fmt,bound", [("int4_sym_block", 0.35), ("int4_sym", 0.35),
                                       ("fp8_e4m3", 0.35)])
def test_compressed_kernel_path_tolerance(fmt, bound):
    """tests/test_kernels.py:54-75: K/V stored as [B, T, H, D], compressed,
    restored and attended; the INT4-sym case also through
    int4_decode_attention with the CompressedKV in the [B, H, T, D] layout
    (the kernel that reads the codes in place)."""
    from korith_vllm_ext.codecs import get_codec
    from korith_vllm_ext.int4_decode_attention import int4_decode_attention
    from korith_vllm_ext.kernels import fallback_fp16_kernel

    torch.manual_seed(0)
    q, k, v = _make_qkv()
    codec = get_codec(fmt)
    k_store = k.permute(0, 2, 1, 3).contiguous().to(DEV)
    v_store = v.permute(0, 2, 1, 3).contiguous().to(DEV)
    k_dec = codec.decompress_to(codec.compress(k_store), torch.float16).permute(0, 2, 1, 3)
    v_dec = codec.decompress_to(codec.compress(v_store), torch.float16).permute(0, 2, 1, 3)
    out = fallback_fp16_kernel(q.to(DEV), k_dec.contiguous(), v_dec.contiguous())
    ref = _sdpa_cpu(q, k, v)
    assert _rel(out, ref) < bound
    if fmt == "int4_sym":
        ck, cv = codec.compress(k.to(DEV)), codec.compress(v.to(DEV))
        out2 = int4_decode_attention(q.to(DEV), ck, cv)
        assert _rel(out2, ref) < bound
        # attention over the exactly dequantized K/V, and within their fp16
        # rounding of attention over the restored tensors
        kx, vx = codec.decompress_to(ck, torch.float32), codec.decompress_to(cv, torch.float32)
        assert _rel(out2, _sdpa_cpu(q, kx, vx)) < 1e-3
        kd, vd = codec.decompress_to(ck, torch.float16), codec.decompress_to(cv, torch.float16)
        out3 = fallback_fp16_kernel(q.to(DEV), kd, vd)
        assert _rel(out2, out3.float().cpu()) < 1e-2


def test_fallback_handles_mask():
    """tests/test_kernels.py:85-92, with the masked tokens checked to carry
    no weight."""
    from korith_vllm_ext.kernels import fallback_fp16_kernel

    torch.manual_seed(0)
    q, k, v = _make_qkv(T=16)
    B, H, T, D = 2, 4, 16, 128
    mask = torch.zeros(B, H, 1, T, dtype=torch.float16)
    mask[..., 8:] = float("-inf")
    out = fallback_fp16_kernel(q.to(DEV), k.to(DEV), v.to(DEV), mask=mask.to(DEV))
    assert out.shape == (B, H, 1, D)
    assert torch.isfinite(out).all()
    ref = _sdpa_cpu(q, k[:, :, :8], v[:, :, :8])
    assert _rel(out, ref) < 1e-2


def test_fallback_multi_tile_correctness():
    """tests/test_kernels.py:95-112: T in {256, 512, 1024}, seed 42."""
    from korith_vllm_ext.kernels import fallback_fp16_kernel

    torch.manual_seed(42)
    B, H, D = 2, 4, 128
    for T in [256, 512, 1024]:
        q = torch.randn(B, H, 1, D).half()
        k = torch.randn(B, H, T, D).half()
        v = torch.randn(B, H, T, D).half()
        out = fallback_fp16_kernel(q.to(DEV), k.to(DEV), v.to(DEV))
        err = _rel(out, _sdpa_cpu(q, k, v))
        assert err < 1e-2, f"T={T}: rel_err={err:.6f}"


def test_online_softmax_rescale_is_numerically_stable():
    """tests/test_kernels.py:115-133, seed 7: the first 128 tokens nearly
    equal to q, so the early splits hold every large score; also with 64
    query heads on 8 KV heads, so that the GQA waves see it too."""
    from korith_vllm_ext.kernels import fallback_fp16_kernel

    torch.manual_seed(7)
    B, H, D = 1, 1, 128
    T = 512
    q = torch.randn(B, H, 1, D).half()
    k = torch.randn(B, H, T, D).half()
    v = torch.randn(B, H, T, D).half()
    k[:, :, :128, :] = q.expand_as(k[:, :, :128, :]) + 0.01 * torch.randn_like(k[:, :, :128, :])
    out = fallback_fp16_kernel(q.to(DEV), k.to(DEV), v.to(DEV))
    err = _rel(out, _sdpa_cpu(q, k, v))
    assert err < 1e-2, f"rel_err={err:.6f}"
    qg = q.repeat(1, 64, 1, 1)
    kg, vg = k.repeat(1, 8, 1, 1), v.repeat(1, 8, 1, 1)
    outg = fallback_fp16_kernel(qg.to(DEV), kg.to(DEV), vg.to(DEV))
    ref = _sdpa_cpu(q, k, v)
    for h in range(64):
        assert _rel(outg[:, h:h + 1], ref) < 1e-2
