"""amf_int4_paged_decode_attn_noalloc against amf_int4_paged_decode_attn.

The no-allocation entry point runs the same kernels with the split partials
in the library's scratch array instead of a caller workspace, so its output
must equal the workspace entry point's bit for bit.  Checked through the C
ABI on two calls in a row, the second with a smaller input (fewer
sequences, shorter contexts: the scratch keeps the first call's partials),
for GQA 4 and 8 and bf16 / fp32 outputs, and a request larger than the
scratch is refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import amf_hip
from oracle import attention as oatt
from oracle import codecs as oc
from oracle import gen

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
D = 128


def _case(seed, S, Hkv, R, ctx_hi, pool):
    g = torch.Generator().manual_seed(seed)
    kv = gen.kv_values((2, pool, 16, Hkv, D), D, g, True)
    codes, params = oc.int4_asym_compress(kv)
    ctx = torch.randint(1, ctx_hi + 1, (S,), generator=g, dtype=torch.int32)
    width = (ctx_hi + 15) // 16
    bt = torch.stack([torch.randperm(pool, generator=g)[:width] for _ in range(S)]).to(torch.int32)
    q = torch.randn(S, Hkv * R, D, generator=g).to(torch.bfloat16)

    def words(w):
        return torch.from_numpy((w & 0xFFFFFFFF).numpy().astype(np.uint32).view(np.int32)).to(DEV)

    dev = dict(q=q.to(DEV), kc=codes[0].to(DEV), vc=codes[1].to(DEV), kp=words(params[0]),
               vp=words(params[1]), bt=bt.to(DEV), ctx=ctx.to(DEV))
    kv32 = oc.int4_asym_dequant_f32(*oc.int4_asym_quantize(kv))
    return dev, dict(q=q, ctx=ctx, bt=bt, kv32=kv32, S=S, Hkv=Hkv, R=R, width=width, pool=pool)


def _call(lib, d, h, out, out_dtype, workspace):
    args = (d["q"].data_ptr(), amf_hip.DTYPE_BF16, out.data_ptr(), out_dtype, d["kc"].data_ptr(),
            d["kp"].data_ptr(), d["vc"].data_ptr(), d["vp"].data_ptr(), h["pool"],
            d["bt"].data_ptr(), h["width"], d["ctx"].data_ptr(), h["S"], h["Hkv"] * h["R"],
            h["Hkv"], D, 16, h["width"] * 16, 0.0)
    s = amf_hip.stream_handle(DEV)
    if workspace is None:
        return lib.amf_int4_paged_decode_attn_noalloc(*args, amf_hip.DECODE_AUTO, None, s)
    return lib.amf_int4_paged_decode_attn(*args, workspace.data_ptr(),
                                          workspace.numel(), amf_hip.DECODE_AUTO, None, s)


@pytest.mark.parametrize("R,out_dtype", [(4, amf_hip.DTYPE_BF16), (8, amf_hip.DTYPE_F32)])
def test_noalloc_matches_workspace_entry_point(R, out_dtype):
    lib = amf_hip.load()
    tdt = torch.bfloat16 if out_dtype == amf_hip.DTYPE_BF16 else torch.float32
    # first a larger call, then a smaller one: the second must not see the
    # first call's partials
    for seed, S, ctx_hi, pool in ((1, 12, 3000, 400), (2, 3, 700, 120)):
        dev, host = _case(seed * 10 + R, S, 2, R, ctx_hi, pool)
        print(f"noalloc R={R} S={S} ctx<={ctx_hi}", flush=True)
        wsb = amf_hip.decode_workspace_bytes(S, 2 * R, 2, D, host["width"] * 16)
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        want = torch.full((S, 2 * R, D), 5.0, dtype=tdt, device=DEV)
        got = torch.full((S, 2 * R, D), 7.0, dtype=tdt, device=DEV)
        assert _call(lib, dev, host, want, out_dtype, ws) == amf_hip.OK
        assert _call(lib, dev, host, got, out_dtype, None) == amf_hip.OK, lib.amf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16) if tdt == torch.bfloat16 else got,
                           want.view(torch.int16) if tdt == torch.bfloat16 else want)
        ref = oatt.paged_decode_f64(host["q"].float().numpy(), host["kv32"][0].numpy(),
                                    host["kv32"][1].numpy(), host["bt"].numpy(),
                                    host["ctx"].numpy())
        err = float(np.abs(got.float().cpu().numpy() - ref).max())
        assert err <= 2e-2 + 2.0 ** -8 * float(np.abs(ref).max()), err


def test_noalloc_refuses_more_than_its_scratch():
    lib = amf_hip.load()
    dev, host = _case(3, 2, 2, 4, 100, 20)
    # 1024 sequences x 8 heads x 131072 tokens of partials.  Every buffer is
    # allocated at that shape (the block table, 32 MiB of zeros, names page 0
    # of the 20-page pool; contexts are 50 tokens), so that a broken size
    # check would launch kernels that stay inside their buffers and the
    # asserts below, not a memory fault, report it.
    S, width = 1024, 8192
    assert amf_hip.decode_workspace_bytes(S, 8, 2, D, width * 16) > 64 << 20
    big_dev = dict(dev, q=torch.zeros(S, 8, D, dtype=torch.bfloat16, device=DEV),
                   bt=torch.zeros(S, width, dtype=torch.int32, device=DEV),
                   ctx=torch.full((S,), 50, dtype=torch.int32, device=DEV))
    big = dict(host, S=S, width=width)
    out = torch.full((S, 8, D), 3.0, dtype=torch.float32, device=DEV)
    torch.cuda.synchronize()
    rc = _call(lib, big_dev, big, out, amf_hip.DTYPE_F32, None)
    assert rc == amf_hip.ERR_WORKSPACE and b"scratch" in lib.amf_last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
