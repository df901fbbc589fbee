"""oracle - CPU restatement of the reference's KV-materialization path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only to check results
(or, in bench.py, as the timed CPU baseline).  The product path
(axropus-deploy_amd/) never imports it and has no CPU fallback.

Modules
  codecs.py     FP8 / INT4 codecs: the reference formats restated with the same
                torch CPU op sequence (korith_vllm_ext/codecs/amf_codec.py), and
                the two new formats (FP8 per-(page, head), INT4 asym group-32)
                restated from their spec in include/amf_hip.h.
  paging.py     page gather / scatter (compressed_vram_pool.py, amf_kv_manager.py)
  attention.py  paged GQA decode attention over dequantized INT4 KV (fp64), and
                the reference's dense fallback (kernels/dispatch.py:117-152)
  e4m3.py       an independent e4m3fn encoder built from the OCP value table,
                used to pin torch's float8_e4m3fn cast
  gen.py        seeded synthetic inputs of the benchmark configurations
  amfk.py       AMFK snapshot header/table and FNV-1a keying (amf_kv_manager.py)

How each function is pinned (golden vectors, closed forms, brute force) is
listed in tests/test_oracle_pins.py; a function without such a check would be
marked "parity unpinned" there.
"""
