"""Pins of the oracle: each oracle function is checked against the reference's
golden vectors, against closed forms or brute force computed here without the
oracle's own arithmetic, and against mathematical special cases.  Each check
is also run on a copy of the oracle with a plausible mistake planted in it (on
the CPU) to show the check would catch that mistake.

Pin map (oracle function -> checks):
  e4m3.encode / code_values     OCP table values; torch float8_e4m3fn cast,
                                exhaustive over bf16 and over every tie
  codecs.fp8_tensor_*           numpy restatement with the table encoder; floor
                                cases of amf_codec.py:183, 191; +-absmax -> +-448;
                                reference tolerance (tests/test_codecs.py:33-88)
  codecs.fp8_ph_*               per-(page, head) brute force; +-448 per head
  codecs.pack_int4 / unpack     all 256 nibble pairs; odd-length padding
  codecs.int4_channel_*         numpy per-channel brute force; ties to even;
                                zero tensor; +-absmax -> +-7
  codecs.int4_block_*           numpy per-block brute force with padding; page
                                tensors (one block per page)
  codecs.int4_asym_*            group brute force; constant groups; error bound;
                                V tile byte formula of include/amf_hip.h
  paging.gather / scatter       loop restatement; scatter(gather) identity
  paging.*slot*, align, hash    (page, offset) brute force; page-form identity;
                                hand-worked align values; SHA-256 empty-message
                                vector
  attention.*                   two independent formulations agree; closed forms
  amfk.*                        FNV goldens (platform/tests/test_vllm_amf.py:
                                63-122, 350-384); AMFK header
                                (tests/test_direct_kv.py:129-189)
"""

from __future__ import annotations

import math
import struct

import numpy as np
import pytest
import torch

from oracle import amfk, attention, codecs, e4m3, gen, paging

# ---------------------------------------------------------------- e4m3 ----


def test_e4m3_table_known_values():
    v = e4m3.code_values()
    assert v[0x00] == 0.0 and v[0x38] == 1.0 and v[0x7E] == 448.0
    assert v[0x08] == 2.0 ** -6 and v[0x01] == 2.0 ** -9 and v[0x07] == 7 * 2.0 ** -9
    assert v[0xB8] == -1.0 and v[0xFE] == -448.0 and v[0x80] == 0.0
    assert math.isnan(v[0x7F]) and math.isnan(v[0xFF])
    finite = v[~np.isnan(v)]
    assert len(finite) == 254 and np.all(np.diff(v[:0x7F]) > 0)


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _check_encoder(enc) -> None:
    # every bf16 value inside the saturating range, and every tie point
    allb = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    fin = allb[np.isfinite(allb) & (np.abs(allb) <= 448.0)]
    assert np.array_equal(enc(fin), _torch_e4m3(fin))
    pos = e4m3.code_values()[:0x7F]
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    ties = np.concatenate([mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1000)])
    assert np.array_equal(enc(ties), _torch_e4m3(ties))


def test_e4m3_encoder_matches_torch_cast():
    _check_encoder(e4m3.encode)


def test_e4m3_pin_catches_ties_away_from_zero():
    pos = e4m3.code_values()[:0x7F]

    def bad(x):
        x = np.asarray(x, dtype=np.float32)
        a = np.abs(x.astype(np.float64))
        idx = np.argmin(np.abs(pos[None, :] - a[:, None]) - 1e-12 * np.arange(127)[None, :], axis=1)
        return (idx.astype(np.uint8)) | (np.signbit(x).astype(np.uint8) << 7)

    with pytest.raises(AssertionError):
        _check_encoder(bad)


# ------------------------------------------------------ FP8 per tensor ----


def _fp8_tensor_numpy(x: torch.Tensor):
    """amf_codec.py:182-194 from the formula: scale = max(absmax, floor)/448
    where the floor is 1e-8 in x's dtype, divide in fp32, clamp, table encode."""
    floor = float(torch.tensor(1e-8, dtype=x.dtype))
    absmax = float(np.abs(x.float().numpy()).max()) if x.numel() else 0.0
    scale = max(absmax, floor) / 448.0
    div = np.float32(max(scale, 1e-12))
    y = np.clip(x.float().numpy() / div, -448.0, 448.0).astype(np.float32)
    return e4m3.encode(y), scale


def _check_fp8_tensor(compress) -> None:
    g = torch.Generator().manual_seed(3)
    cases = [
        torch.randn(2, 64, 4, 64, generator=g).to(torch.bfloat16),
        (torch.randn(3, 50, 2, 32, generator=g) * 1e-3).to(torch.float16),
        torch.randn(4, 16, 2, 64, generator=g) * 300.0,
        gen.kv_values((2, 4, 16, 2, 128), 128, g, True),
        torch.zeros(2, 16, 2, 64, dtype=torch.bfloat16),
        torch.zeros(2, 16, 2, 64, dtype=torch.float16),
    ]
    for x in cases:
        codes, scale = compress(x)
        want, wscale = _fp8_tensor_numpy(x)
        assert scale == wscale, (x.dtype, scale, wscale)
        assert np.array_equal(codes.numpy().ravel(), want.ravel()), x.dtype
        if float(x.float().abs().max()) > 0:
            flat = x.float().numpy().ravel()
            i = int(np.argmax(np.abs(flat)))
            assert codes.numpy().ravel()[i] in (0x7E, 0xFE)


def test_fp8_tensor_compress_closed_form():
    _check_fp8_tensor(codecs.fp8_tensor_compress)


def test_fp8_tensor_floor_cases():
    _, s = codecs.fp8_tensor_compress(torch.zeros(4, 2, 32, dtype=torch.bfloat16))
    assert s == float(torch.tensor(1e-8, dtype=torch.bfloat16)) / 448.0
    codes, s = codecs.fp8_tensor_compress(torch.zeros(4, 2, 32, dtype=torch.float16))
    assert s == 0.0 and int(codes.sum()) == 0  # fp16(1e-8) == 0; divide by 1e-12


def test_fp8_tensor_pin_catches_wrong_max():
    def bad(x):
        peak = x.detach().abs().amax().clamp_min_(1e-8)
        scale = float(peak) / 447.0
        y = (x.float() / scale).clamp_(-448, 448)
        return y.to(torch.float8_e4m3fn).view(torch.uint8), scale

    with pytest.raises(AssertionError):
        _check_fp8_tensor(bad)


def test_fp8_tensor_decompress_every_code():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = e4m3.code_values()
    ok = ~np.isnan(vals)
    for scale in (1.0, 0.0123, 3.5e-3):
        out = codecs.fp8_tensor_decompress(codes, scale, torch.float32).numpy()
        want = (vals[ok].astype(np.float32) * np.float32(scale)).astype(np.float32)
        assert np.array_equal(out[ok], want)
        outb = codecs.fp8_tensor_decompress(codes, scale, torch.bfloat16)
        assert torch.equal(outb[torch.from_numpy(ok)], torch.from_numpy(want).to(torch.bfloat16))


def test_fp8_reference_tolerance():
    """tests/test_codecs.py:33-41, 68-75: rel error < 0.05 on randn [2,256,8,128]."""
    torch.manual_seed(0)
    x = torch.randn(2, 256, 8, 128)
    codes, scale = codecs.fp8_tensor_compress(x)
    out = codecs.fp8_tensor_decompress(codes, scale, torch.float32)
    assert (out - x).norm().item() / x.norm().item() < 0.05
    assert torch.equal(codecs.fp8_sidecar(scale), torch.tensor([scale, scale, 1, 1],
                                                               dtype=torch.float32))


# -------------------------------------------------- FP8 per (page, head) ----


def _check_fp8_ph(compress) -> None:
    g = torch.Generator().manual_seed(5)
    x = gen.kv_values((2, 3, 16, 4, 64), 64, g, True)
    x[1, 2, :, 3, :] = 0  # an all-zero (page, head)
    codes, scales = compress(x)
    xf = x.float().numpy()
    for p in range(2):
        for n in range(3):
            for h in range(4):
                blk = xf[p, n, :, h, :]
                s = np.float32(max(np.float32(np.abs(blk).max()), np.float32(1e-8))) / np.float32(448)
                assert scales[p, n, h].item() == float(np.float32(s))
                want = e4m3.encode(np.clip(blk / np.float32(s), -448, 448).astype(np.float32))
                got = codes[p, n, :, h, :].numpy()
                assert np.array_equal(got, want)
                if np.abs(blk).max() > 0:
                    assert np.isin(got.ravel(), [0x7E, 0xFE]).any()


def test_fp8_ph_brute_force():
    _check_fp8_ph(codecs.fp8_ph_compress)


def test_fp8_ph_pin_catches_per_page_scale():
    def bad(pages):
        x = pages.float()
        scale = torch.clamp_min(x.abs().amax(dim=(2, 3, 4)), 1e-8) / 448.0
        s = scale[:, :, None].expand(-1, -1, x.shape[3])
        y = (x / s[:, :, None, :, None]).clamp(-448, 448)
        return y.to(torch.float8_e4m3fn).view(torch.uint8), s

    with pytest.raises(AssertionError):
        _check_fp8_ph(bad)


# ---------------------------------------------------------- INT4 nibbles ----


def _check_pack(pack, unpack) -> None:
    a, b = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    q = torch.from_numpy(np.stack([a.ravel(), b.ravel()], -1).astype(np.int8))
    packed = pack(q).numpy()[:, 0]
    want = (((b.ravel() + 8) << 4) | (a.ravel() + 8)).astype(np.uint8)
    assert np.array_equal(packed, want)
    assert torch.equal(unpack(pack(q), 2), q)
    odd = torch.tensor([[3, -8, 7]], dtype=torch.int8)
    assert pack(odd).tolist() == [[(0 << 4) | 11, (0 << 4) | 15]]  # u = 11, 0 | 15, pad 0
    assert torch.equal(unpack(pack(odd), 3), odd)


def test_pack_unpack_all_pairs():
    _check_pack(codecs.pack_int4, codecs.unpack_int4)


def test_pack_pin_catches_swapped_nibbles():
    def bad(q):
        u = (q.to(torch.int16) + 8).to(torch.uint8)
        if u.shape[-1] % 2:
            u = torch.cat([u, torch.zeros_like(u[..., :1])], -1)
        return (u[..., 0::2] << 4) | u[..., 1::2]

    with pytest.raises(AssertionError):
        _check_pack(bad, codecs.unpack_int4)


# ----------------------------------------------------- INT4 per channel ----


def _check_channel(compress) -> None:
    g = torch.Generator().manual_seed(9)
    x = gen.kv_values((2, 40, 3, 64), 64, g, True)
    packed, s16 = compress(x)
    xf = x.float().numpy().reshape(-1, 64)
    for c in range(64):
        s = np.float32(max(np.float32(np.abs(xf[:, c]).max()), np.float32(1e-8))) / np.float32(7)
        q = np.clip(np.rint(xf[:, c] / s), -8, 7).astype(np.int64)
        got = codecs.unpack_int4(packed, 64).numpy().reshape(-1, 64)[:, c]
        assert np.array_equal(got, q), c
        assert s16[c].item() == float(np.float16(s))
    # ties to even: absmax 7 gives scale exactly 1.0
    t = torch.tensor([[[7.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -7.0]]]).permute(2, 0, 1)
    pk, sc = compress(t.contiguous())
    assert codecs.unpack_int4(pk, 1).ravel().tolist() == [7, 2, -2, 4, 0, 0, 2, -7]


def test_int4_channel_brute_force():
    _check_channel(codecs.int4_channel_compress)


def test_int4_channel_zero_tensor():
    pk, sc = codecs.int4_channel_compress(torch.zeros(4, 2, 32))
    assert torch.all(pk == 0x88) and torch.all(sc == float(np.float16(np.float32(1e-8) / 7)))


def test_int4_channel_pin_catches_half_up_rounding():
    def bad(x):
        xf = x.float()
        scale = xf.abs().amax(dim=tuple(range(xf.dim() - 1))).clamp_min(1e-8) / 7.0
        q = torch.floor(xf / scale + 0.5).clamp(-8, 7).to(torch.int8)
        return codecs.pack_int4(q), scale.to(torch.float16)

    with pytest.raises(AssertionError):
        _check_channel(bad)


def test_int4_reference_tolerances():
    """tests/test_codecs.py:33-41, 68-75: int4_sym < 0.20, int4_sym_block < 0.22."""
    torch.manual_seed(0)
    x = torch.randn(2, 256, 8, 128)
    pk, sc = codecs.int4_channel_compress(x)
    out = codecs.int4_channel_decompress(pk, sc, x.shape, torch.float32)
    assert (out - x).norm().item() / x.norm().item() < 0.20
    pk, sc, meta = codecs.int4_block_compress(x)
    out = codecs.int4_block_decompress(pk, sc, x.shape, meta, torch.float32)
    assert (out - x).norm().item() / x.norm().item() < 0.22


# ------------------------------------------------------- INT4 per block ----


def _check_block(compress) -> None:
    g = torch.Generator().manual_seed(10)
    for shape in ((2, 300, 2, 32), (2, 5, 16, 2, 64)):
        x = gen.kv_values(shape, shape[-1], g, True)
        packed, scales, meta = compress(x)
        T, H, D = shape[-3:]
        nb = -(-T // 128)
        assert meta == {"block_size": 128, "n_tokens": T, "n_blocks": nb}
        assert tuple(scales.shape) == tuple(shape[:-3]) + (nb,)
        xf = x.float().numpy().reshape(-1, T, H, D)
        q_all = codecs.unpack_int4(packed, D).numpy().reshape(-1, T, H, D)
        sc = scales.numpy().reshape(-1, nb)
        for i in range(xf.shape[0]):
            for b in range(nb):
                blk = xf[i, b * 128:(b + 1) * 128]
                s = np.float32(max(np.float32(np.abs(blk).max()), np.float32(1e-8))) / np.float32(7)
                assert sc[i, b] == np.float16(s)
                q = np.clip(np.rint(blk / s), -8, 7)
                assert np.array_equal(q_all[i, b * 128:(b + 1) * 128], q)


def test_int4_block_brute_force():
    _check_block(codecs.int4_block_compress)


def test_int4_block_pin_catches_unpadded_scale_per_token():
    def bad(x, block=128):
        xf = x.float()
        scale = xf.abs().amax(dim=(-2, -1), keepdim=True).clamp_min(1e-8) / 7.0
        q = torch.round(xf / scale).clamp(-8, 7).to(torch.int8)
        T = x.shape[-3]
        nb = -(-T // block)
        return codecs.pack_int4(q), scale.reshape(*x.shape[:-3], T)[..., :nb].to(torch.float16), \
            {"block_size": block, "n_tokens": T, "n_blocks": nb}

    with pytest.raises(AssertionError):
        _check_block(bad)


# ----------------------------------------------------- INT4 asym g32 ----


def _check_asym(quantize) -> None:
    g = torch.Generator().manual_seed(12)
    x = gen.kv_values((2, 2, 16, 2, 64), 64, g, True)
    x[0, 1, 3, 1, 32:] = 0.375  # a constant group
    u, s16, z16 = quantize(x)
    xf = x.float().numpy().reshape(2, 2, 16, 2, 2, 32)
    for idx in np.ndindex(2, 2, 16, 2, 2):
        grp = xf[idx]
        mn, mx = np.float32(grp.min()), np.float32(grp.max())
        s = np.float32(max(np.float32(mx - mn), np.float32(1e-8))) / np.float32(15)
        q = np.clip(np.rint((grp - mn) / s), 0, 15)
        p, n, t, h, gg = idx
        assert np.array_equal(u[p, n, t, h, gg * 32:(gg + 1) * 32].numpy(), q), idx
        assert s16[idx].item() == float(np.float16(s)) and z16[idx].item() == float(np.float16(mn))
    deq = codecs.int4_asym_dequant_f32(u, s16, z16)
    assert torch.all(deq[0, 1, 3, 1, 32:] == 0.375)
    # |x - deq| <= s/2 + 15 |s - s16| + |mn - z16| (+ fp32 slack)
    xs = x.float().reshape(2, 2, 16, 2, 2, 32)
    s32 = (xs.amax(-1) - xs.amin(-1)).clamp_min(1e-8) / 15
    bound = s32 / 2 + 15 * (s32 - s16.float()).abs() + (xs.amin(-1) - z16.float()).abs()
    err = (deq.reshape(2, 2, 16, 2, 2, 32) - xs).abs().amax(-1)
    assert torch.all(err <= bound * (1 + 1e-5) + 1e-6)


def test_int4_asym_quantize_brute_force():
    _check_asym(codecs.int4_asym_quantize)


def test_int4_asym_pin_catches_levels_16():
    def bad(pages):
        x = pages.float()
        P, n, bs, H, D = x.shape
        xg = x.reshape(P, n, bs, H, D // 32, 32)
        mn, mx = xg.amin(-1), xg.amax(-1)
        scale = torch.clamp_min(mx - mn, 1e-8) / 16.0
        uu = torch.round((xg - mn[..., None]) / scale[..., None]).clamp(0, 15).to(torch.int64)
        return uu.reshape(P, n, bs, H, D), scale.to(torch.float16), mn.to(torch.float16)

    with pytest.raises(AssertionError):
        _check_asym(bad)


def test_int4_asym_layout_byte_formula():
    """include/amf_hip.h: K codes [head][token][D/2] (low nibble = even dim);
    V codes at byte 64*(d/8) + 32*(t/8) + 4*(d%8) + (t%8)/2 of the (page, head)
    block, low nibble for even t; K params [head][token][G], V params
    [head][G][token], word = fp16 scale | fp16 zero << 16."""
    g = torch.Generator().manual_seed(13)
    P, n, bs, H, D = 2, 2, 16, 3, 64
    G = D // 32
    u = torch.randint(0, 16, (P, n, bs, H, D), generator=g)
    s16 = torch.rand(P, n, bs, H, G, generator=g).to(torch.float16)
    z16 = torch.randn(P, n, bs, H, G, generator=g).to(torch.float16)
    codes, params = codecs.int4_asym_layout(u, s16, z16)
    blk = bs * D // 2
    for pg in range(n):
        for h in range(H):
            kb = codes[0, pg, h * blk:(h + 1) * blk].numpy()
            vb = codes[1, pg, h * blk:(h + 1) * blk].numpy()
            for t in range(bs):
                for d in range(D):
                    kbyte = kb[t * D // 2 + d // 2]
                    assert ((kbyte >> 4) if d % 2 else (kbyte & 15)) == u[0, pg, t, h, d]
                    vbyte = vb[64 * (d // 8) + 32 * (t // 8) + 4 * (d % 8) + (t % 8) // 2]
                    assert ((vbyte >> 4) if t % 2 else (vbyte & 15)) == u[1, pg, t, h, d]
            for t in range(bs):
                for gg in range(G):
                    kw = int(params[0, pg, (h * bs + t) * G + gg])
                    vw = int(params[1, pg, (h * G + gg) * bs + t])
                    for w, p in ((kw, 0), (vw, 1)):
                        sb = np.array([w & 0xFFFF], np.uint16).view(np.float16)[0]
                        zb = np.array([w >> 16], np.uint16).view(np.float16)[0]
                        assert sb == s16[p, pg, t, h, gg].item() and zb == z16[p, pg, t, h, gg].item()
    u2, s2, z2 = codecs.int4_asym_unlayout(codes, params, bs, H, D)
    assert torch.equal(u2, u) and torch.equal(s2, s16) and torch.equal(z2, z16)


# ---------------------------------------------------------------- paging ----


def test_paging_gather_scatter():
    rng = np.random.default_rng(0)
    cache = rng.integers(0, 65536, size=(2, 40, 16, 2, 8), dtype=np.uint16)
    ids = rng.permutation(40)[:13]
    got = paging.gather(cache, ids)
    for j, b in enumerate(ids):
        assert np.array_equal(got[:, j], cache[:, b])
    target = np.full_like(cache, 0xBEEF)
    ids2 = rng.permutation(40)[:13]
    paging.scatter(target, ids2, got)
    for j, b in enumerate(ids2):
        assert np.array_equal(target[:, b], cache[:, ids[j]])
    untouched = np.setdiff1d(np.arange(40), ids2)
    assert np.all(target[:, untouched] == 0xBEEF)
    assert np.array_equal(paging.gather(target, ids2), got)


def test_slot_mapping_brute_force_and_quirks():
    """AMFReqMeta.make's slots (amf_kv_connector.py:90-115) against slots
    recomputed from (page, offset) pairs, and align_to_block_size's values
    (:72-74) worked by hand."""
    assert [paging.align_to_block_size(n, 16) for n in (0, 1, 15, 16, 17, 32, 33)] == \
        [-16, 0, 0, 0, 16, 16, 32]
    blocks = [7, 2, 9]
    slots = paging.slot_mapping(blocks, 4, 10)
    assert slots == [28, 29, 30, 31, 8, 9, 10, 11, 36, 37]
    for i, s in enumerate(slots):
        assert divmod(s, 4) == (blocks[i // 4], i % 4)
    assert paging.slot_mapping(blocks, 4, -4) == paging.slot_mapping(blocks, 4, 8)


def test_slot_gather_scatter_against_pages():
    """Whole-page slot lists move what the page gather / scatter moves; a
    single-slot mistake (offset from the wrong page) fails."""
    rng = np.random.default_rng(1)
    cache = rng.integers(0, 65536, size=(2, 12, 4, 3, 8), dtype=np.uint16)
    ids = [5, 0, 11]
    slots = paging.slot_mapping(ids, 4, 12)
    rows = paging.gather_slots(cache, slots)
    assert np.array_equal(rows.reshape(2, 3, 4, 3, 8), paging.gather(cache, ids))
    target = np.zeros_like(cache)
    paging.scatter_slots(target, slots, rows)
    assert np.array_equal(paging.gather(target, ids), paging.gather(cache, ids))
    assert np.all(np.delete(target, ids, axis=1) == 0)
    # unordered slots: every row lands where its slot says
    perm = rng.permutation(48)[:17]
    got = paging.gather_slots(cache, perm)
    for j, s in enumerate(perm):
        assert np.array_equal(got[:, j], cache[:, s // 4, s % 4])
    wrong = [(s // 4) * 4 + (s + 1) % 4 for s in slots]
    assert not np.array_equal(paging.gather_slots(cache, wrong), rows)


def test_prefix_hash_known_answers():
    """The SHA-256 digest of the empty message (published test vector), and
    the word packing: token 0x00636261 is the bytes b"abc\\x00", -1 is four
    0xff bytes, and tokens are taken mod 2**32."""
    assert paging.prefix_hash([]) == "e3b0c44298fc1c14"
    import hashlib

    assert paging.prefix_hash([0x00636261]) == hashlib.sha256(b"abc\x00").hexdigest()[:16]
    assert paging.prefix_hash([-1]) == hashlib.sha256(b"\xff" * 4).hexdigest()[:16]
    assert paging.prefix_hash([1 << 32 | 5]) == paging.prefix_hash([5])
    assert paging.prefix_hash([1, 2]) != paging.prefix_hash([2, 1])


# ------------------------------------------------------------- attention ----


def test_attention_two_formulations_agree():
    g = torch.Generator().manual_seed(14)
    B, Hq, Hkv, D, pool = 3, 8, 2, 32, 20
    q = torch.randn(B, Hq, D, generator=g).numpy()
    kp = torch.randn(pool, 16, Hkv, D, generator=g).numpy()
    vp = torch.randn(pool, 16, Hkv, D, generator=g).numpy()
    ctx = np.array([1, 37, 80])
    bt = np.stack([np.random.default_rng(b).permutation(pool)[:5] for b in range(B)])
    paged = attention.paged_decode_f64(q, kp, vp, bt, ctx)
    for b in range(B):
        n = ctx[b]
        K = kp[bt[b]].reshape(-1, Hkv, D)[:n].transpose(1, 0, 2)[None]
        V = vp[bt[b]].reshape(-1, Hkv, D)[:n].transpose(1, 0, 2)[None]
        dense = attention.dense_attention_f64(q[b][None, :, None], K, V)[0, :, 0]
        assert np.allclose(paged[b], dense, rtol=1e-12, atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(1)
    D = 16
    q = rng.standard_normal((1, 2, 1, D))
    v = rng.standard_normal((1, 2, 7, D))
    k_same = np.repeat(rng.standard_normal((1, 2, 1, D)), 7, axis=2)
    out = attention.dense_attention_f64(q, k_same, v)
    assert np.allclose(out[:, :, 0], v.mean(axis=2))          # equal keys: mean of V
    k = rng.standard_normal((1, 2, 7, D))
    mask = np.full((1, 1, 1, 7), -np.inf)
    mask[..., 4] = 0.0
    out = attention.dense_attention_f64(q, k, v, mask=mask)
    assert np.allclose(out[:, :, 0], v[:, :, 4])                # one visible key
    out1 = attention.dense_attention_f64(q, k[:, :, :1], v[:, :, :1])
    assert np.allclose(out1[:, :, 0], v[:, :, 0])               # T = 1
    assert not attention.dense_attention_f64(q, k[:, :, :0], v[:, :, :0]).any()


def test_reference_fallback_within_tolerance():
    """The reference's bf16 fallback path against fp64 (tests/test_kernels.py:
    54-75 tolerance class), on the decode shape."""
    g = torch.Generator().manual_seed(15)
    q = torch.randn(2, 8, 1, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 8, 256, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, 256, 128, generator=g).to(torch.bfloat16)
    ref = attention.dense_attention_f64(q.double().numpy(), k.double().numpy(), v.double().numpy())
    fb = attention.fallback_attention(q, k, v).float().numpy()
    assert np.abs(fb - ref).max() < 2e-2


# ------------------------------------------------------------------ AMFK ----


_U64 = (1 << 64) - 1


def test_fnv_goldens():
    """platform/tests/test_vllm_amf.py:63-122 (offset written in hex as
    amf_kv_manager.py:38's comment gives it)."""
    off, prime = 0x14650FB0739D0383, 1099511628211
    assert amfk.FNV_OFFSET == off and amfk.FNV_PRIME == prime
    golden_123 = (((((off ^ 1) * prime) & _U64 ^ 2) * prime) & _U64 ^ 3) * prime & _U64
    assert amfk.hash_tokens([1, 2, 3]) == golden_123
    assert amfk.hash_tokens([]) == off
    assert amfk.hash_tokens([0]) == (off * prime) & _U64
    assert amfk.hash_tokens([-1]) == ((off ^ 0xFFFFFFFF) * prime) & _U64
    assert amfk.hash_tenant("") == off
    h = amfk.hash_tenant("nebius")
    assert h not in (0, off) and h == amfk.hash_tenant("nebius")
    assert amfk.float_bits(0.0) == 0 and amfk.float_bits(1.0) == 0x3F800000
    assert amfk.float_bits(10000.0) == 0x461C4000


def test_fnv_pin_catches_published_offset():
    bad = 14695981039346656037
    assert amfk.hash_tokens([1, 2, 3]) != (((((bad ^ 1) * amfk.FNV_PRIME) & _U64 ^ 2)
                                            * amfk.FNV_PRIME) & _U64 ^ 3) * amfk.FNV_PRIME & _U64


def test_filename_golden():
    """platform/tests/test_vllm_amf.py:350-384."""
    name = amfk.key_filename(0x1234567890ABCDEF, 0xFEDCBA0987654321, 0xABCDEF0123456789, 65536, 1,
                             amfk.float_bits(10000.0), amfk.float_bits(1.0), 0, 0)
    assert name == ("amf_1234567890abcdef_fedcba0987654321_abcdef0123456789"
                    f"_65536_1_{0x461C4000}_{0x3F800000}"
                    "_0000000000000000_0000000000000000")
    assert name.startswith("amf_") and not name.endswith(".kv")


def test_amfk_header_layout():
    """tests/test_direct_kv.py:129-189 and core/amf_direct_kv.h:62-63."""
    hdr = amfk.pack_header(80, 85000, 4, 256, 2, 1 << 30, 0xDEADBEEFCAFEBABE, 0x0102030405060708)
    assert len(hdr) == 56 and amfk.LAYER.size == 32
    f = struct.unpack("<IIIIIIII QQQ", hdr)
    assert f == (0x414D464B, 1, 80, 85000, 4, 256, 2, 0, 1 << 30, 0xDEADBEEFCAFEBABE,
                 0x0102030405060708)
    assert hdr[:4] == b"KFMA"
    tab = amfk.layer_table([(100, 100), (64, 32)])
    assert tab == [(0, 100, 100, 100), (200, 64, 264, 32)]


# ------------------------------------------------------------------- gen ----


def test_gen_seeded_and_outliers():
    g1, g2 = torch.Generator().manual_seed(4), torch.Generator().manual_seed(4)
    a = gen.kv_values((2, 16, 2, 128), 128, g1, True)
    b = gen.kv_values((2, 16, 2, 128), 128, g2, True)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert len(gen.outlier_channels(128, torch.Generator().manual_seed(0))) == 3
    assert len(gen.outlier_channels(64, torch.Generator().manual_seed(0))) == 1
    bt = gen.block_table(100, 10, 7)
    assert bt.dtype == torch.int32 and len(set(bt.tolist())) == 10
