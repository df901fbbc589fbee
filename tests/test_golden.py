"""The committed fixtures of tests/golden/: the oracle still reproduces the
codec hashes and the reference's known answers (CPU), and the HIP kernels
reproduce the codec hashes through the C ABI (GPU)."""

from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

import pytest
import torch

from oracle import amfk

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_golden as mg  # noqa: E402

CODEC = json.load(open(os.path.join(HERE, "codec_golden.json")))
REF = json.load(open(os.path.join(HERE, "reference_vectors.json")))
IDS = [f"{e['format']}-{e['dtype']}" for e in CODEC["entries"]]


@pytest.mark.parametrize("entry", CODEC["entries"], ids=IDS)
def test_oracle_reproduces_codec_golden(entry):
    dtype = mg.DTYPES[entry["dtype"]]
    c, p, r = mg.oracle_case(entry["format"], mg.pages_for(entry["format"], dtype), dtype)
    assert (mg.sha(c), mg.sha(p), mg.sha(r)) == (entry["codes"], entry["params"], entry["restored"])


def test_oracle_matches_reference_known_answers():
    f = REF["fnv"]
    assert (amfk.FNV_OFFSET, amfk.FNV_PRIME) == (f["offset"], f["prime"])
    assert amfk.hash_tokens([1, 2, 3]) == f["tokens_1_2_3"]
    assert amfk.hash_tokens([0]) == f["tokens_0"]
    assert amfk.hash_tenant("") == f["tenant_empty"]
    assert amfk.float_bits(1.0) == REF["float_bits"]["1.0"]
    assert amfk.key_filename(*REF["filename"]["args"]) == REF["filename"]["expected"]
    h = REF["amfk_header"]
    assert amfk.pack_header(*h["fields"][2:7], h["fields"][8], h["fields"][9],
                            h["fields"][10]).hex() == h["bytes_hex"]
    assert amfk.HEADER.size == h["size"] and amfk.LAYER.size == h["layer_entry_size"]


def test_package_keys_match_reference_known_answers():
    from korith_vllm_ext.amf_kv_manager import amf_hash_tokens, amf_key_filename

    assert amf_hash_tokens([1, 2, 3]) == REF["fnv"]["tokens_1_2_3"]
    assert amf_key_filename(*REF["filename"]["args"]) == REF["filename"]["expected"]


@pytest.mark.gpu
@pytest.mark.parametrize("entry", CODEC["entries"], ids=IDS)
def test_hip_reproduces_codec_golden(entry):
    from korith_vllm_ext import _paged

    fmt, dtype = entry["format"], mg.DTYPES[entry["dtype"]]
    n, H, D = (mg.CASE[k] for k in ("n", "H", "D"))
    pages = mg.pages_for(fmt, dtype).cuda()
    lay = _paged.BlobLayout(fmt, 2, n, 16, H, D)
    blob = torch.zeros(lay.total_bytes, dtype=torch.uint8, device="cuda")
    _paged.quant_gather(lay, _paged.planes_view([pages[0], pages[1]]), None, [blob.data_ptr()], 2)
    out = torch.full_like(pages, -1.0)
    _paged.dequant_scatter(lay, [blob.data_ptr()], 2, _paged.planes_view([out[0], out[1]]), None)
    torch.cuda.synchronize()
    b = blob.cpu().numpy().tobytes()
    codes = b[:lay.data_bytes]
    if lay.shared_params:
        params = b[lay.scale_offset:lay.scale_offset + lay.shared_param_bytes]
    else:
        params = b"".join(b[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                          for p in range(2))
    restored = mg.tbytes(out.cpu())
    assert mg.sha(codes) == entry["codes"]
    assert mg.sha(params) == entry["params"]
    assert mg.sha(restored) == entry["restored"]
