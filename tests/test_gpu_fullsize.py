"""Parity at the benchmark's full sizes, every layer and every sequence.

The inputs are exactly the ones bench.py times (its case builders are
reused): the Llama-3-8B FP8 restore (32 layers, 512 pages into 8192) and INT4
restore (2048 pages into 16384), the Llama-3-70B FP8 restore (80 layers x
8192 pages), and the INT4 paged decodes (batch 32, contexts U[1024, 32768],
GQA 4; batch 8 x 131072, GQA 8).  Inputs carry the benchmark's x20 outlier
channels.

  restore  every layer's restored pages equal the oracle's decompression of
           that layer's blob bit for bit, and every untouched page keeps its
           sentinel;
  save     every layer's blob equals the oracle's compression of the gathered
           pages byte for byte;
  decode   every sequence is within 2e-2 max-abs (plus half a bf16 ulp of the
           output) and 1e-2 mean-rel of float64 attention over the
           dequantized KV; the batch-32 output is also compared with the
           reference's own bf16 path (decompress, then matmul -> softmax ->
           matmul in bf16, kernels/dispatch.py:117-143).  That path rounds
           scores and probabilities to bf16, which with x20 outlier channels
           puts it far from float64 itself, so it is reported, and the test
           checks that the kernel is the closer of the two to float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import attention as oatt
from oracle import codecs as oc

from helpers import attn_errors, check_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _oracle_restore(case: "bench.RestoreCase", l: int) -> torch.Tensor:
    lay = case.layout
    blob = case.blobs[l].cpu()
    if case.fmt == "fp8_e4m3_ph":
        codes = blob[:lay.data_bytes].view(2, case.pages, 16, case.heads, case.head_dim)
        sc = torch.stack([blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                          .view(torch.float32).view(case.pages, case.heads) for p in range(2)])
        return oc.fp8_ph_decompress(codes, sc, torch.bfloat16)
    cpl = lay.plane_code_bytes
    c = torch.stack([blob[lay.code_offset(p):lay.code_offset(p) + cpl].view(case.pages, -1)
                     for p in range(2)])
    pr = torch.stack([blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                      .view(torch.int32).view(case.pages, -1).to(torch.int64) & 0xFFFFFFFF
                      for p in range(2)])
    return oc.int4_asym_decompress(c, pr, 16, case.heads, case.head_dim, torch.bfloat16)


def _restore_and_check(case, layers, sentinel=-3.5, check_untouched=True):
    for c in case.cache:
        c.fill_(sentinel)
    case.launch.launch()
    torch.cuda.synchronize()
    ids = case.ids.long().to(DEV)
    mask = torch.ones(case.pool, dtype=torch.bool, device=DEV)
    mask[ids] = False
    for l in layers:
        if check_untouched:
            assert bool((case.cache[l][:, mask] == sentinel).all()), f"layer {l} untouched"
        want = _oracle_restore(case, l)
        got = case.cache[l][:, ids].cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"layer {l}"


@pytest.mark.parametrize("fmt", ["fp8_e4m3_ph", "int4_asym_g32"])
def test_restore_fullsize_every_layer(fmt):
    if fmt == "fp8_e4m3_ph":
        case = bench.RestoreCase(fmt, 32, 8, 128, 8192, 512, seed=2)
    else:
        case = bench.RestoreCase(fmt, 32, 8, 128, 16384, 2048, seed=3)
    print(f"restore {fmt}: {case.layers} layers x {case.pages} pages", flush=True)
    _restore_and_check(case, range(case.layers))
    case.free()


@pytest.mark.parametrize("fmt", ["fp8_e4m3_ph", "fp8_e4m3", "int4_asym_g32"])
def test_save_fullsize_every_layer(fmt):
    """The save kernels at the benchmark's shapes on the benchmark's data
    (N(0,1) with x20 outlier channels; the per-tensor format at this shape
    takes the single-read cooperative kernel)."""
    if fmt in ("fp8_e4m3_ph", "fp8_e4m3"):
        case = bench.RestoreCase(fmt, 32, 8, 128, 8192, 512, seed=2)
    else:
        case = bench.RestoreCase(fmt, 32, 8, 128, 16384, 2048, seed=3)
    for l, c in enumerate(case.cache):
        c.copy_(bench.device_kv(c.shape, 128, 900 + l, outliers=True))
    print(f"save {fmt}: {case.layers} layers x {case.pages} pages", flush=True)
    case.save_launch().launch()
    torch.cuda.synchronize()
    lay = case.layout
    ids = case.ids.long()
    for l in range(case.layers):
        pages = case.cache[l][:, ids.to(DEV)].cpu()
        blob = case.blobs[l].cpu()
        if fmt == "fp8_e4m3_ph":
            codes, sc = oc.fp8_ph_compress(pages)
            assert torch.equal(blob[:lay.data_bytes].view(codes.shape), codes), l
            for p in range(2):
                got = blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                assert torch.equal(got.view(torch.float32).view(case.pages, case.heads), sc[p]), l
        elif fmt == "fp8_e4m3":
            codes, scale = oc.fp8_tensor_compress(pages)
            assert torch.equal(blob[:lay.data_bytes].view(codes.shape), codes), l
            side = blob[lay.scale_offset:lay.scale_offset + 16].view(torch.float32)
            assert torch.equal(side, oc.fp8_sidecar(scale)), l
        else:
            codes, params = oc.int4_asym_compress(pages)
            for p in range(2):
                cb = blob[lay.code_offset(p):lay.code_offset(p) + lay.plane_code_bytes]
                pb = blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                assert torch.equal(cb.view(codes[p].shape), codes[p]), (l, p)
                assert torch.equal(pb.view(torch.int32).to(torch.int64).view(params[p].shape) &
                                   0xFFFFFFFF, params[p]), (l, p)
    case.free()


def _seq_kv(dc, b):
    """(ctx, fp32 dequantized K and V [n_pages, 16, Hkv, D]) of sequence b."""
    lay = dc.layout
    cpp = lay.code_bytes_per_page
    ppp = lay.plane_param_bytes // dc.pool
    ctx = int(dc.ctx[b])
    n = (ctx + 15) // 16
    pages = dc.bt_cpu[b, :n].long()
    codes, params = [], []
    for p in range(2):
        cb = dc.blob[lay.code_offset(p): lay.code_offset(p) + lay.plane_code_bytes]
        pb = dc.blob[lay.param_offset(p): lay.param_offset(p) + lay.plane_param_bytes]
        codes.append(cb.view(dc.pool, cpp)[pages.to(cb.device)].cpu())
        params.append(pb.view(dc.pool, ppp)[pages.to(pb.device)].cpu().view(torch.int32)
                      .to(torch.int64) & 0xFFFFFFFF)
    u, s16, z16 = oc.int4_asym_unlayout(torch.stack(codes), torch.stack(params), 16,
                                        dc.kv_heads, dc.D)
    return ctx, n, oc.int4_asym_dequant_f32(u, s16, z16)


def _check_f64(out_b, ref, tag):
    # bf16 output: its own rounding (half an ulp, <= |ref| 2^-8) on top of 2e-2
    half_ulp = np.abs(ref) * 2.0 ** -8
    d = np.abs(out_b - ref)
    assert float((d - (2e-2 + half_ulp)).max()) <= 0.0, (tag, float(d.max()))
    _, mean_rel = attn_errors(out_b, ref)
    assert mean_rel <= 1e-2, (tag, mean_rel)


def test_decode_fullsize_every_sequence():
    """Batch 32, GQA 4: both kernels against float64 on all 32 sequences, and
    the MFMA kernel against the reference's bf16 path."""
    import amf_hip

    dc = bench.DecodeCase()
    outs = {}
    for name, algo in (("mfma", amf_hip.DECODE_MFMA), ("valu", amf_hip.DECODE_VALU)):
        dc.launch(algo)
        torch.cuda.synchronize()
        outs[name] = dc.out.float().cpu().numpy()
    # the default kernel with fp32 output: held to 2e-2 / 1e-2 without the
    # bf16 output's own rounding
    o32 = torch.empty(dc.out.shape, dtype=torch.float32, device=DEV)
    dc.launch(amf_hip.DECODE_MFMA, out=o32)
    torch.cuda.synchronize()
    out32 = o32.cpu().numpy()
    refs = []
    R = dc.q_heads // dc.kv_heads
    acc = {k: [0.0, 0.0, 0.0] for k in ("hip_vs_fallback", "fallback_vs_f64", "hip_vs_f64")}

    def add(key, got, ref):
        d = np.abs(got - ref)
        a = acc[key]
        a[0] = max(a[0], float(d.max()))
        a[1] += float(d.sum())
        a[2] += float(np.abs(ref).sum())

    for b in range(dc.batch):
        ctx, n, kv32 = _seq_kv(dc, b)
        q = dc.q[b:b + 1].float().cpu().numpy()
        ref = oatt.paged_decode_f64(q, kv32[0].numpy(), kv32[1].numpy(), np.arange(n)[None],
                                    dc.ctx[b:b + 1].numpy())
        for name, out in outs.items():
            _check_f64(out[b:b + 1], ref, (name, b))
        refs.append(ref[0])
        # the reference's own path: bf16 decompress, matmul -> softmax -> matmul in bf16
        kvb = kv32.to(torch.bfloat16)
        k = kvb[0].reshape(n * 16, dc.kv_heads, dc.D)[:ctx].permute(1, 0, 2)
        v = kvb[1].reshape(n * 16, dc.kv_heads, dc.D)[:ctx].permute(1, 0, 2)
        k = k.repeat_interleave(R, dim=0)[None]
        v = v.repeat_interleave(R, dim=0)[None].contiguous()
        fb = oatt.fallback_attention(dc.q[b].cpu()[None, :, None, :], k, v)[0, :, 0]
        fb = fb.float().numpy()
        add("hip_vs_fallback", outs["mfma"][b], fb)
        add("fallback_vs_f64", fb, ref[0])
        add("hip_vs_f64", outs["mfma"][b], ref[0])
    check_attention(out32, np.stack(refs), label="mfma fp32 output, 32 sequences")
    res = {k: (a[0], a[1] / a[2]) for k, a in acc.items()}
    for k, (ma, mr) in res.items():
        print(f"decode over 32 sequences, {k}: max-abs {ma:.3e}, mean-rel {mr:.3e}", flush=True)
    assert res["hip_vs_f64"][0] <= res["fallback_vs_f64"][0]
    assert res["hip_vs_f64"][1] <= res["fallback_vs_f64"][1]


def _free_gib():
    return torch.cuda.mem_get_info()[0] / 2 ** 30


@pytest.fixture(scope="module")
def restore_70b():
    if _free_gib() < 75:
        pytest.skip("needs ~70 GiB of device memory")
    case = bench.RestoreCase("fp8_e4m3_ph", 80, 8, 128, 8192, 8192, seed=5)
    sentinel = -3.5
    for c in case.cache:
        c.fill_(sentinel)
    case.launch.launch()
    torch.cuda.synchronize()
    yield case
    case.free()


@pytest.mark.parametrize("half", [0, 1])
def test_restore_70b_every_layer(restore_70b, half):
    """Llama-3-70B share: FP8-PH restore of a 131072-token prefix (80 layers x
    8192 pages) into an 8192-page bf16 pool through a random permutation (so
    every page of the pool is compared); layers 0-39, then 40-79."""
    case = restore_70b
    ids = case.ids.long().to(DEV)
    print(f"70b restore layers {40 * half}..{40 * half + 39}", flush=True)
    for l in range(40 * half, 40 * half + 40):
        # ids is a permutation of the whole pool: every page is compared
        want = _oracle_restore(case, l)
        got = case.cache[l][:, ids].cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"layer {l}"


def test_decode_70b_every_sequence():
    """Batch 8 x 131072 tokens, 64 query heads over 8 KV heads (GQA 8)."""
    import amf_hip

    if _free_gib() < 8:
        pytest.skip("needs device memory")
    dc = bench.DecodeCase(8, 64, 8, 131072, 131072, 6)
    dc.launch(amf_hip.DECODE_MFMA)
    o32 = torch.empty(dc.out.shape, dtype=torch.float32, device=DEV)
    dc.launch(amf_hip.DECODE_MFMA, out=o32)
    torch.cuda.synchronize()
    out = dc.out.float().cpu().numpy()
    out32 = o32.cpu().numpy()
    refs = []
    for b in range(dc.batch):
        ctx, n, kv32 = _seq_kv(dc, b)
        ref = oatt.paged_decode_f64(dc.q[b:b + 1].float().cpu().numpy(), kv32[0].numpy(),
                                    kv32[1].numpy(), np.arange(n)[None], dc.ctx[b:b + 1].numpy())
        _check_f64(out[b:b + 1], ref, ("mfma70b", b))
        refs.append(ref[0])
    # fp32 output: 2e-2 / 1e-2 without the bf16 output's own rounding
    check_attention(out32, np.stack(refs), label="mfma fp32 output, 70B shape")
    del dc
    torch.cuda.empty_cache()
