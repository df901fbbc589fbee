"""Parity at the benchmark's full sizes, checked on samples.

The inputs are exactly the ones bench.py times (its case builders are
reused): the Llama-3-8B FP8 restore (32 layers, 512 pages into 8192) and INT4
restore (2048 pages into 16384), and the batch-32 INT4 paged decode with
contexts U[1024, 32768].  Restored layers are compared bit-for-bit with the
oracle on sampled layers plus size-independent properties over all layers
(untouched pool pages keep their sentinel; the restored pages of every layer
round-trip through the oracle decompress of that layer's blob is sampled).
Decode is compared with float64 attention on sampled sequences.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import attention as oatt
from oracle import codecs as oc

from helpers import attn_errors

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


@pytest.mark.parametrize("fmt", ["fp8_e4m3_ph", "int4_asym_g32"])
def test_restore_fullsize(fmt):
    if fmt == "fp8_e4m3_ph":
        case = bench.RestoreCase(fmt, 32, 8, 128, 8192, 512, seed=2)
    else:
        case = bench.RestoreCase(fmt, 32, 8, 128, 16384, 2048, seed=3)
    sentinel = torch.tensor(-3.5, dtype=torch.bfloat16)
    for c in case.cache:
        c.fill_(sentinel.item())
    case.launch.launch()
    torch.cuda.synchronize()
    ids = case.ids.long().to(DEV)
    mask = torch.ones(case.pool, dtype=torch.bool, device=DEV)
    mask[ids] = False
    for l in range(case.layers):
        # every layer: untouched pages still hold the sentinel
        assert bool((case.cache[l][:, mask] == sentinel.item()).all()), f"layer {l}"
    for l in (0, 13, case.layers - 1):
        want = _oracle_restore(case, l)
        got = case.cache[l][:, ids].cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"layer {l}"
    case.free()


@pytest.mark.parametrize("fmt", ["fp8_e4m3_ph", "fp8_e4m3", "int4_asym_g32"])
def test_save_fullsize(fmt):
    """The save kernels at the benchmark's shapes (bench.py --profile fp8_save /
    int4_save; the per-tensor format at the same shape takes the single-read
    cooperative kernel): blobs of sampled layers equal the oracle's
    compression of the gathered pages, byte for byte."""
    if fmt in ("fp8_e4m3_ph", "fp8_e4m3"):
        case = bench.RestoreCase(fmt, 32, 8, 128, 8192, 512, seed=2)
    else:
        case = bench.RestoreCase(fmt, 32, 8, 128, 16384, 2048, seed=3)
    g = torch.Generator(device="cuda").manual_seed(21)
    for c in case.cache:
        c.copy_(torch.randn(c.shape, generator=g, device=DEV).to(torch.bfloat16))
    case.save_launch().launch()
    torch.cuda.synchronize()
    lay = case.layout
    ids = case.ids.long()
    for l in (0, 17, case.layers - 1):
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


def _check_decode(dc, algo, seqs):
    out = dc.out.float().cpu().numpy()
    lay = dc.layout
    cpp = lay.code_bytes_per_page
    ppp = lay.plane_param_bytes // dc.pool
    for b in seqs:
        n = (int(dc.ctx[b]) + 15) // 16
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
        kv32 = oc.int4_asym_dequant_f32(u, s16, z16).numpy()
        ref = oatt.paged_decode_f64(dc.q[b:b + 1].float().cpu().numpy(), kv32[0], kv32[1],
                                    np.arange(n)[None], dc.ctx[b:b + 1].numpy())
        # bf16 output: its own rounding (half an ulp, <= |ref| 2^-8) on top of 2e-2
        half_ulp = np.abs(ref) * 2.0 ** -8
        d = np.abs(out[b:b + 1] - ref)
        assert float((d - (2e-2 + half_ulp)).max()) <= 0.0, (algo, b, float(d.max()))
        _, mean_rel = attn_errors(out[b:b + 1], ref)
        assert mean_rel <= 1e-2, (algo, b, mean_rel)


def test_decode_fullsize_sampled():
    import amf_hip

    dc = bench.DecodeCase()
    for algo in (amf_hip.DECODE_MFMA, amf_hip.DECODE_VALU):
        dc.launch(algo)
        torch.cuda.synchronize()
        _check_decode(dc, algo, (0, 7, dc.batch - 1))


def _free_gib():
    return torch.cuda.mem_get_info()[0] / 2 ** 30


def test_restore_70b_fullsize_sampled():
    """Llama-3-70B share: FP8-PH restore of a 131072-token prefix (80 layers x
    8192 pages) into an 8192-page bf16 pool through a random permutation."""
    if _free_gib() < 75:
        pytest.skip("needs ~70 GiB of device memory")
    case = bench.RestoreCase("fp8_e4m3_ph", 80, 8, 128, 8192, 8192, seed=5)
    sentinel = -3.5
    for c in case.cache:
        c.fill_(sentinel)
    case.launch.launch()
    torch.cuda.synchronize()
    for l in range(case.layers):
        # a permutation of the whole pool: no page keeps the sentinel
        assert not bool((case.cache[l][:, :, 0, 0, 0] == sentinel).all()), l
    ids = case.ids.long().to(DEV)
    for l in (0, 41, 79):
        want = _oracle_restore(case, l)
        got = case.cache[l][:, ids].cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"layer {l}"
    case.free()


def test_decode_70b_fullsize_sampled():
    """Batch 8 x 131072 tokens, 64 query heads over 8 KV heads (GQA 8)."""
    import amf_hip

    if _free_gib() < 8:
        pytest.skip("needs device memory")
    dc = bench.DecodeCase(8, 64, 8, 131072, 131072, 6)
    dc.launch(amf_hip.DECODE_MFMA)
    torch.cuda.synchronize()
    _check_decode(dc, amf_hip.DECODE_MFMA, (0, 7))
    del dc
    torch.cuda.empty_cache()
