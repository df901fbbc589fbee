#!/usr/bin/env python3
"""bench.py - AMF KV materialization on one MI355X.

Headline (`value`): FP8 restore GB/s at the Llama-3-8B KV shape -- 32 layers,
8 KV heads, head_dim 128, 16-token pages; a 512-page (8192-token) prefix
stored as fp8_e4m3_ph (per-(page, head) fp32 scale) is dequantized and
scattered into a bf16 paged cache of 8192 pages through a seeded random block
table.  One step = one restore of all 32 layers (one kernel launch).

Also reported (same JSON line):
  int4_restore : int4_asym_g32 restore, 2048-page prefix into a 16384-page pool
  int4_decode  : paged GQA decode over INT4 KV, batch 32, Hq 32 / Hkv 8,
                 contexts U[1024, 32768], one layer call

GB/s = algorithmic bytes / mean kernel time (HIP events on the launch stream,
1 GB = 1e9 B).  Algorithmic bytes: restore = codes + params read + cache
bytes written; decode = 1280 B per context token (8 heads x (2 x 64 B codes
+ 2 x 16 B params)).  The CPU baseline is the reference's PyTorch op sequence
restated on the host (oracle/), timed on a bounded sample.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --profile {fp8_restore,int4_restore,decode_mfma,decode_valu}
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "axropus-deploy_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "KV restore GB/s (FP8/INT4 dequant+scatter); INT4 decode-attn tok/s; 1 GPU"
HBM_PEAK_GBS = 8000.0
DEV = torch.device("cuda")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ inputs --


def device_kv(shape, head_dim: int, seed: int, outliers: bool = True) -> torch.Tensor:
    """N(0,1) bf16 on the GPU with x20 on round(0.02 * head_dim) seeded channels."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32)
    if outliers:
        k = int(round(0.02 * head_dim))
        ch = torch.randperm(head_dim, generator=torch.Generator().manual_seed(seed))[:k]
        x[..., ch.to(DEV)] *= 20.0
    return x.to(torch.bfloat16)


def seeded_table(pool: int, n: int, seed: int) -> torch.Tensor:
    return torch.randperm(pool, generator=torch.Generator().manual_seed(seed))[:n].to(torch.int32)


def time_launches(fn, steps: int, warmup: int) -> float:
    """Mean milliseconds per call of fn (HIP events on torch's current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# ----------------------------------------------------------------- restore --


class RestoreCase:
    """A compressed prefix (one blob per layer) and a paged bf16 target cache."""

    def __init__(self, fmt: str, layers: int, heads: int, head_dim: int, pool: int, pages: int,
                 seed: int):
        from korith_vllm_ext import _paged

        self.fmt, self.layers, self.pages, self.pool = fmt, layers, pages, pool
        self.heads, self.head_dim, self.bs = heads, head_dim, 16
        self.layout = _paged.BlobLayout(fmt, 2, pages, 16, heads, head_dim)
        # Source prefix as an unpaged cache, quantized once (identity block ids).
        self.blobs = torch.empty(layers, self.layout.total_bytes, dtype=torch.uint8, device=DEV)
        for l in range(layers):
            src = device_kv((2, pages, 16, heads, head_dim), head_dim, seed * 1000 + l)
            view = _paged.cache_view([src])
            _paged.quant_gather(self.layout, view, None, [self.blobs[l].data_ptr()], 2)
            del src
        self.cache = [torch.empty(2, pool, 16, heads, head_dim, dtype=torch.bfloat16, device=DEV)
                      for _ in range(layers)]
        self.ids = seeded_table(pool, pages, seed + 7)
        self.launch = _paged.PreparedCodecLaunch(
            "restore", self.layout, [self.blobs[l].data_ptr() for l in range(layers)], 2,
            _paged.cache_view(self.cache), self.ids)
        torch.cuda.synchronize()

    @property
    def algo_bytes(self) -> int:
        lay = self.layout
        read = self.layers * (lay.data_bytes + lay.scale_bytes)
        written = self.layers * 2 * self.pages * lay.page_elems * 2
        return read + written

    def cpu_baseline(self, sample_layers: int, min_seconds: float = 10.0):
        """The reference restore op sequence on the host for `sample_layers`
        layers: per layer decompress_to(bf16) then chunked k_all[ids] = src
        (compressed_vram_pool.py:579-606), on a host copy of the blobs.

        Copies the inputs to the host now and returns a callable that times
        the restore when called, so the CPU work can run after every GPU
        measurement instead of idling the GPU between them."""
        from oracle import codecs as oc

        lay = self.layout
        ids = self.ids.long()
        blobs = [self.blobs[l].cpu() for l in range(sample_layers)]
        cache = [torch.empty(2, self.pool, 16, self.heads, self.head_dim, dtype=torch.bfloat16)
                 for _ in range(sample_layers)]
        for c in cache:
            c.zero_()

        def run():
            for l, blob in enumerate(blobs):
                codes = blob[:lay.data_bytes].view(2, self.pages, 16, self.heads, self.head_dim)
                if self.fmt == "fp8_e4m3_ph":
                    sc = torch.stack([blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                                      .view(torch.float32).view(self.pages, self.heads) for p in range(2)])
                    kv = oc.fp8_ph_decompress(codes, sc, torch.bfloat16)
                else:
                    cpl = lay.plane_code_bytes
                    c = torch.stack([blob[lay.code_offset(p):lay.code_offset(p) + cpl]
                                     .view(self.pages, -1) for p in range(2)])
                    pr = torch.stack([blob[lay.param_offset(p):lay.param_offset(p) + lay.plane_param_bytes]
                                      .view(torch.int32).view(self.pages, -1).to(torch.int64) & 0xFFFFFFFF
                                      for p in range(2)])
                    kv = oc.int4_asym_decompress(c, pr, 16, self.heads, self.head_dim, torch.bfloat16)
                for start in range(0, self.pages, 512):
                    end = min(start + 512, self.pages)
                    cache[l][0][ids[start:end]] = kv[0][start:end]
                    cache[l][1][ids[start:end]] = kv[1][start:end]

        sample_bytes = self.algo_bytes * sample_layers / self.layers
        n_layers = self.layers

        def timed() -> dict:
            times = []
            t_start = time.perf_counter()
            while len(times) < 3 or time.perf_counter() - t_start < min_seconds:
                t0 = time.perf_counter()
                run()
                times.append(time.perf_counter() - t0)
            t = statistics.median(times)
            return {"value": sample_bytes / t / 1e9, "unit": "GB/s", "seconds": t,
                    "sample": f"restore of {sample_layers} of {n_layers} layers, median of "
                              f"{len(times)} runs ({time.perf_counter() - t_start:.1f} s total)"}

        return timed

    def save_launch(self):
        """The save direction on the same shape: gather the prefix pages from
        the paged cache through the block table and quantize into the blobs."""
        from korith_vllm_ext import _paged

        return _paged.PreparedCodecLaunch(
            "save", self.layout, [self.blobs[l].data_ptr() for l in range(self.layers)], 2,
            _paged.cache_view(self.cache), self.ids)

    def pool_api(self, steps: int, warmup: int) -> dict:
        """Wall-clock ms per CompressedVRAMPool.put_from_vllm / restore_to_vllm
        call on this shape (host work included, tables cached after the first
        call), with the algorithmic GB/s of the same bytes."""
        from korith_vllm_ext.compressed_vram_pool import CompressedVRAMPool

        blk = 1 << 20
        per_layer = -(-self.layout.total_bytes // blk) * blk
        pool = CompressedVRAMPool(self.layers, per_layer, blk, default_format=self.fmt,
                                  device=DEV)
        src = seeded_table(self.pool, self.pages, 11).tolist()
        dst = self.ids.tolist()
        n_tok = self.pages * 16

        def wall(fn):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / steps

        put_ms = wall(lambda: pool.put_from_vllm("bench", self.cache, src, n_tok))
        rest_ms = wall(lambda: pool.restore_to_vllm("bench", self.cache, dst))
        del pool
        torch.cuda.empty_cache()
        return {"put_from_vllm_ms": round(put_ms, 4),
                "put_GB/s": round(self.algo_bytes / put_ms / 1e6, 1),
                "restore_to_vllm_ms": round(rest_ms, 4),
                "restore_GB/s": round(self.algo_bytes / rest_ms / 1e6, 1)}

    def free(self):
        del self.launch, self.cache, self.blobs
        torch.cuda.empty_cache()


# --------------------------------------------------------------- connector --


class ConnectorCase:
    """AMFKVConnector on the Llama-3-8B shape: a cold prefill of `tokens`
    prompt tokens saved from 32 layers of a paged bf16 cache, then a warm
    request restored into other pages through start_load_kv and the
    per-layer waits.  Also times the raw token-slot kernels on unordered
    slots (the general path)."""

    def __init__(self, fmt: str = "fp8_e4m3", layers: int = 32, heads: int = 8,
                 head_dim: int = 128, pool: int = 8192, pages: int = 512, seed: int = 12):
        from types import SimpleNamespace as NS

        from korith_vllm_ext.amf_kv_connector import AMFKVConnector, KVConnectorRole

        self.layers, self.heads, self.head_dim, self.pages = layers, heads, head_dim, pages
        self.fmt = fmt
        self.cache = [device_kv((2, pool, 16, heads, head_dim), head_dim, seed * 100 + l)
                      for l in range(layers)]
        self.target = [torch.empty_like(c) for c in self.cache]
        tokens = pages * 16 + 1
        self.prompt = list(range(tokens))
        self.cold = seeded_table(pool, pages + 1, seed).tolist()
        self.warm = seeded_table(pool, pages + 1, seed + 1).tolist()
        from korith_vllm_ext import _paged

        page = _paged.DENSE_PAGE_TOKENS[fmt]
        blob = _paged.BlobLayout(fmt, 2, -(-pages * 16 // page), page, heads, head_dim)
        extra = dict(num_layers=layers, num_kv_heads=heads, head_dim=head_dim,
                     bytes_per_layer=(-(-blob.total_bytes // (1 << 20)) + 1) << 20,
                     default_format=fmt, min_prefix_tokens=64)
        cfg = NS(cache_config=NS(block_size=16),
                 kv_transfer_config=NS(kv_connector_extra_config=extra))
        self.conn = AMFKVConnector(cfg, KVConnectorRole.WORKER)
        self.NS = NS

    def _sched(self, req_id, blocks):
        NS = self.NS
        return NS(scheduled_new_reqs=[NS(req_id=req_id, prompt_token_ids=self.prompt,
                                         block_ids=(blocks,))],
                  scheduled_cached_reqs=NS(req_ids=[], resumed_req_ids=set(),
                                           num_computed_tokens=[], new_block_ids=[]),
                  num_scheduled_tokens={})

    def _forward(self, caches):
        NS = self.NS
        return NS(attn_metadata=object(), virtual_engine=0, no_compile_layers={
            f"model.layers.{l}.self_attn.attn": NS(kv_cache=[c]) for l, c in enumerate(caches)})

    def save_meta(self):
        """Scheduler side of a cold request: hash, slots, store metadata."""
        return self.conn.build_connector_meta(self._sched("cold", self.cold))

    def load_meta(self):
        """Scheduler side of a warm request: hit, slots, load metadata."""
        c = self.conn
        c.update_state_after_alloc(self.NS(request_id="warm"), None, self.pages * 16)
        return c.build_connector_meta(self._sched("warm", self.warm))

    def save(self, meta):
        """Worker side of a cold prefill: every layer's save_kv_layer, then
        wait_for_save (the pool insert)."""
        c = self.conn
        c.bind_connector_metadata(meta)
        fwd = self._forward(self.cache)
        for name, layer in fwd.no_compile_layers.items():
            c.save_kv_layer(name, layer.kv_cache[0], None)
        c.wait_for_save()
        c.clear_connector_metadata()

    def load(self, meta):
        """Worker side of a warm request: start_load_kv and every layer's
        wait_for_layer_load."""
        c = self.conn
        c.bind_connector_metadata(meta)
        fwd = self._forward(self.target)
        c.start_load_kv(fwd)
        for name in fwd.no_compile_layers:
            c.wait_for_layer_load(name)
        c.wait_for_save()
        c.clear_connector_metadata()

    @property
    def tokens(self) -> int:
        return self.pages * 16

    def algo_bytes(self) -> int:
        """Codes + params read (restore) or written (save), plus the bf16 rows
        written (restore) or read (save)."""
        from korith_vllm_ext import _paged

        lay = _paged.BlobLayout(self.fmt, 2, self.pages, 16, self.heads, self.head_dim)
        return self.layers * (lay.data_bytes + lay.scale_bytes +
                              2 * self.tokens * self.heads * self.head_dim * 2)

    def slot_launch(self, seed: int = 5):
        """Raw token-slot gather of `tokens` unordered slots of every plane."""
        from korith_vllm_ext import _paged

        S = self.cache[0].shape[1] * 16
        slots = torch.randperm(S, generator=torch.Generator().manual_seed(seed))[:self.tokens]
        sm = _paged.SlotMap(slots)
        view = _paged.cache_view(self.cache)
        out = torch.empty(self.layers * 2, self.tokens, self.heads, self.head_dim,
                          dtype=torch.bfloat16, device=DEV)
        outs = [out[i].data_ptr() for i in range(out.shape[0])]
        row = self.heads * self.head_dim * 2
        bytes_moved = 2 * out.numel() * 2
        return (lambda: _paged.gather_slots(view, sm, self.tokens, outs, row)), bytes_moved, out

    def run(self, steps: int, warmup: int) -> dict:
        def wall(fn):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / steps

        meta_ms = wall(self.save_meta)
        smeta = self.save_meta()
        save_ms = wall(lambda: self.save(smeta))
        lmeta = self.load_meta()
        load_ms = wall(lambda: self.load(lmeta))
        algo = self.algo_bytes()
        fn, moved, keep = self.slot_launch()
        slot_ms = time_launches(fn, steps, warmup)
        del keep
        return {"workload": "connector_llama3_8b_8k", "format": self.fmt,
                "tokens": self.tokens, "layers": self.layers,
                "scheduler_meta_ms": round(meta_ms, 4),
                "save_ms": round(save_ms, 4), "save_GB/s": round(algo / save_ms / 1e6, 1),
                "load_ms": round(load_ms, 4), "load_GB/s": round(algo / load_ms / 1e6, 1),
                "slot_gather_unordered_ms": round(slot_ms, 4),
                "slot_gather_GB/s": round(moved / slot_ms / 1e6, 1),
                "slot_gather_frac": round(moved / slot_ms / 1e6 / HBM_PEAK_GBS, 4)}

    def free(self):
        del self.conn, self.cache, self.target
        torch.cuda.empty_cache()


# ------------------------------------------------------------------ decode --


class DecodeCase:
    """INT4 paged decode at batch 32, Hq 32 / Hkv 8, contexts U[1024, 32768]."""

    def __init__(self, batch=32, q_heads=32, kv_heads=8, ctx_lo=1024, ctx_hi=32768, seed=4):
        import amf_hip
        from korith_vllm_ext import _paged

        D = 128
        g = torch.Generator().manual_seed(seed)
        self.q = torch.randn(batch, q_heads, D, generator=g).to(torch.bfloat16).to(DEV)
        self.ctx = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g, dtype=torch.int32)
        pages = [(int(c) + 15) // 16 for c in self.ctx]
        self.pool = sum(pages)
        perm = torch.randperm(self.pool, generator=g).to(torch.int32)
        bt = torch.zeros(batch, max(pages), dtype=torch.int32)
        o = 0
        for b, n in enumerate(pages):
            bt[b, :n] = perm[o:o + n]
            o += n
        self.bt_cpu = bt
        self.bt = bt.to(DEV)
        self.dctx = self.ctx.to(DEV)
        self.batch, self.q_heads, self.kv_heads, self.D = batch, q_heads, kv_heads, D
        self.max_ctx = int(self.ctx.max())
        self.sum_ctx = int(self.ctx.sum())
        # INT4 pool: quantize seeded bf16 pages chunk by chunk.
        self.layout = _paged.BlobLayout("int4_asym_g32", 2, self.pool, 16, kv_heads, D)
        self.blob = torch.empty(self.layout.total_bytes, dtype=torch.uint8, device=DEV)
        chunk = 4096
        for c0 in range(0, self.pool, chunk):
            n = min(chunk, self.pool - c0)
            src = device_kv((2, n, 16, kv_heads, D), D, seed * 7919 + c0)
            part = _paged.BlobLayout("int4_asym_g32", 2, n, 16, kv_heads, D)
            tmp = torch.empty(part.total_bytes, dtype=torch.uint8, device=DEV)
            _paged.quant_gather(part, _paged.cache_view([src]), None, [tmp.data_ptr()], 2)
            lay = self.layout
            for p in range(2):
                cpp = lay.code_bytes_per_page
                self.blob[lay.code_offset(p) + c0 * cpp: lay.code_offset(p) + (c0 + n) * cpp] = \
                    tmp[part.code_offset(p): part.code_offset(p) + part.plane_code_bytes]
                ppp = lay.plane_param_bytes // self.pool
                self.blob[lay.param_offset(p) + c0 * ppp: lay.param_offset(p) + (c0 + n) * ppp] = \
                    tmp[part.param_offset(p): part.param_offset(p) + part.plane_param_bytes]
            del src, tmp
        self.out = torch.empty(batch, q_heads, D, dtype=torch.bfloat16, device=DEV)
        ws_bytes = amf_hip.decode_workspace_bytes(batch, q_heads, kv_heads, D, self.max_ctx)
        self.ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=DEV)
        self.amf_hip = amf_hip
        self._fn = amf_hip.load().amf_int4_paged_decode_attn
        torch.cuda.synchronize()

    def ptr(self, plane, kind):
        lay = self.layout
        off = lay.code_offset(plane) if kind == "codes" else lay.param_offset(plane)
        return self.blob.data_ptr() + off

    def launch(self, algo):
        h = self.amf_hip
        rc = self._fn(self.q.data_ptr(), h.DTYPE_BF16, self.out.data_ptr(), h.DTYPE_BF16,
                      self.ptr(0, "codes"), self.ptr(0, "params"), self.ptr(1, "codes"),
                      self.ptr(1, "params"), self.pool, self.bt.data_ptr(), self.bt.shape[1],
                      self.dctx.data_ptr(), self.batch, self.q_heads, self.kv_heads, self.D, 16,
                      self.max_ctx, 0.0, self.ws.data_ptr(), self.ws.numel() * 4, algo, None,
                      h.stream_handle(DEV))
        h.check("amf_int4_paged_decode_attn", rc)

    @property
    def algo_bytes(self) -> int:
        return 1280 * self.sum_ctx * self.kv_heads // 8


# -------------------------------------------------------------------- main --


def long_context_70b(steps: int, warmup: int) -> dict:
    """Llama-3-70B share on one GPU: FP8-PH restore of a 131072-token prefix
    (80 layers x 8192 pages, ~21.5 GB of blobs into a 43 GB bf16 cache) and
    INT4 decode at batch 8 x 131072 tokens, 64 query heads (GQA 8).  Skipped
    when the device lacks the ~70 GB it needs."""
    free, _ = torch.cuda.mem_get_info()
    if free < 80 * (1 << 30):
        log(f"70b workloads skipped: {free / 2**30:.0f} GiB free")
        return {"fp8_restore_70b": None, "decode_70b": None}
    out = {}
    log("70b fp8 restore: building inputs")
    case = RestoreCase("fp8_e4m3_ph", 80, 8, 128, 8192, 8192, 5)
    ms = time_launches(case.launch.launch, max(3, steps // 4), warmup)
    gbs = case.algo_bytes / (ms * 1e-3) / 1e9
    out["fp8_restore_70b"] = {"workload": "fp8_restore_llama3_70b_131k", "ms": round(ms, 4),
                              "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "algo_bytes": case.algo_bytes}
    log(f"70b fp8 restore: {ms:.3f} ms, {gbs:.1f} GB/s")
    case.free()
    del case
    log("70b decode: building inputs")
    dc = DecodeCase(8, 64, 8, 131072, 131072, 6)
    msd = time_launches(lambda: dc.launch(amf_hip_module().DECODE_MFMA), steps, warmup)
    gd = dc.algo_bytes / (msd * 1e-3) / 1e9
    out["decode_70b"] = {"workload": "decode_llama3_70b_b8_131k", "ms_per_layer_call": round(msd, 5),
                         "tok_per_s_per_layer": round(dc.batch / (msd * 1e-3), 1),
                         "tok_per_s_model_80_layers": round(dc.batch / (80 * msd * 1e-3), 1),
                         "GB/s": round(gd, 1), "frac": round(gd / HBM_PEAK_GBS, 4)}
    log(f"70b decode: {msd:.4f} ms, {gd:.1f} GB/s")
    del dc
    torch.cuda.empty_cache()
    return out


def amf_hip_module():
    import amf_hip

    return amf_hip


def profiled_traffic(name: str):
    """HBM bytes per launch recorded by the rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs of this workload (profiles/<name>.md, counters scaled by the
    page-copy calibration), or None when no summary is present."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def cpu_threads() -> int:
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return max(1, min(int(n or 1), 16))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    # 20 launches (about 6 ms of the headline kernel) bring the clocks to their
    # steady state; after 3 the first timed window still runs ~3% slower.
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--profile", choices=["fp8_restore", "int4_restore", "fp8_save", "int4_save",
                                          "fp8_tensor_save",
                                          "fp8_restore_70b", "decode_70b", "decode_mfma",
                                          "decode_valu", "copy", "slot_copy"], default=None,
                    help="run only this kernel loop (for rocprofv3)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: there is no multi-GPU path "
              "(the KV hot path shards by layer/head with no exchange).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    import amf_hip

    amf_hip.load()
    torch.set_num_threads(cpu_threads())

    if args.profile:
        if args.profile == "copy":
            # Calibration for the HBM byte counters: a raw page copy of exactly
            # 1 GiB read + 1 GiB written (2 planes of 16384 pages of 32 KiB).
            from korith_vllm_ext import _paged

            src = torch.empty(2, 16384, 16, 8, 128, dtype=torch.bfloat16, device=DEV).fill_(1.0)
            dst = torch.empty_like(src)
            view = _paged.cache_view([src])
            fn = lambda: _paged.gather_pages(view, None, [dst[0].data_ptr(), dst[1].data_ptr()],
                                             view.page_bytes, 16384)
            ms = time_launches(fn, args.steps, args.warmup)
            log(f"copy: {ms:.4f} ms/launch, 1 GiB read + 1 GiB written per launch, "
                f"{2 * 2**30 / ms / 1e6:.1f} GB/s")
            return 0
        if args.profile == "slot_copy":
            cc = ConnectorCase()
            fn, moved, keep = cc.slot_launch()
            ms = time_launches(fn, args.steps, args.warmup)
            log(f"slot_copy: {ms:.4f} ms/launch, {moved / ms / 1e6:.1f} GB/s")
            return 0
        if args.profile == "fp8_restore_70b":
            case = RestoreCase("fp8_e4m3_ph", 80, 8, 128, 8192, 8192, 5)
            ms = time_launches(case.launch.launch, args.steps, args.warmup)
            log(f"{args.profile}: {ms:.4f} ms/launch, {case.algo_bytes / ms / 1e6:.1f} GB/s")
            return 0
        if args.profile == "decode_70b":
            case = DecodeCase(8, 64, 8, 131072, 131072, 6)
            ms = time_launches(lambda: case.launch(amf_hip.DECODE_MFMA), args.steps, args.warmup)
            log(f"{args.profile}: {ms:.4f} ms/call, {case.algo_bytes / ms / 1e6:.1f} GB/s")
            return 0
        if args.profile in ("fp8_restore", "int4_restore", "fp8_save", "int4_save",
                            "fp8_tensor_save"):
            fmt = ("fp8_e4m3" if args.profile == "fp8_tensor_save" else
                   "fp8_e4m3_ph" if args.profile.startswith("fp8") else "int4_asym_g32")
            case = (RestoreCase(fmt, 32, 8, 128, 16384, 2048, 3) if fmt == "int4_asym_g32"
                    else RestoreCase(fmt, 32, 8, 128, 8192, 512, 2))
            launch = case.launch if args.profile.endswith("restore") else case.save_launch()
            ms = time_launches(launch.launch, args.steps, args.warmup)
            log(f"{args.profile}: {ms:.4f} ms/launch, {case.algo_bytes / ms / 1e6:.1f} GB/s")
        else:
            case = DecodeCase()
            algo = amf_hip.DECODE_MFMA if args.profile == "decode_mfma" else amf_hip.DECODE_VALU
            ms = time_launches(lambda: case.launch(algo), args.steps, args.warmup)
            log(f"{args.profile}: {ms:.4f} ms/call, {case.algo_bytes / ms / 1e6:.1f} GB/s")
        return 0

    # ---- headline: FP8 per-(page, head) restore, Llama-3-8B shape ----
    log("fp8 restore: building inputs")
    fp8 = RestoreCase("fp8_e4m3_ph", 32, 8, 128, 8192, 512, seed=2)
    ms = time_launches(fp8.launch.launch, args.steps, args.warmup)
    gbs = fp8.algo_bytes / (ms * 1e-3) / 1e9
    log(f"fp8 restore: {ms:.4f} ms, {gbs:.1f} GB/s")
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "fp8_restore_llama3_8b", "layers": 32, "kv_heads": 8,
                   "head_dim": 128, "block_size": 16, "prefix_pages": 512, "pool_pages": 8192,
                   "format": "fp8_e4m3_ph", "cache_dtype": "bf16", "parallelism": "none"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("fp8_dequant_scatter_llama3_8b_512p"),
                     "kernel": "fp8_dequant_scatter_kernel",
                     "algo_bytes_per_launch": fp8.algo_bytes},
    }
    cpu_timed = None if args.no_cpu_baseline else fp8.cpu_baseline(8)
    sv = fp8.save_launch()
    ms_s = time_launches(sv.launch, args.steps, args.warmup)
    result["fp8_save"] = {"workload": "fp8_save_llama3_8b", "ms": round(ms_s, 5),
                          "GB/s": round(fp8.algo_bytes / ms_s / 1e6, 2),
                          "frac": round(fp8.algo_bytes / ms_s / 1e6 / HBM_PEAK_GBS, 4)}
    del sv
    log(f"fp8 save: {ms_s:.4f} ms")
    log("fp8 restore: CompressedVRAMPool API wall clock")
    result["pool_api"] = fp8.pool_api(args.steps, args.warmup)
    log(f"pool api: {result['pool_api']}")
    fp8.free()
    del fp8

    if not args.no_secondary:
        log("int4 restore: building inputs")
        i4 = RestoreCase("int4_asym_g32", 32, 8, 128, 16384, 2048, seed=3)
        ms4 = time_launches(i4.launch.launch, args.steps, args.warmup)
        g4 = i4.algo_bytes / (ms4 * 1e-3) / 1e9
        log(f"int4 restore: {ms4:.4f} ms, {g4:.1f} GB/s")
        result["int4_restore"] = {"workload": "int4_restore_llama3_8b", "ms": round(ms4, 5),
                                  "GB/s": round(g4, 2), "frac": round(g4 / HBM_PEAK_GBS, 4),
                                  "algo_bytes": i4.algo_bytes}
        sv4 = i4.save_launch()
        ms4s = time_launches(sv4.launch, args.steps, args.warmup)
        result["int4_save"] = {"workload": "int4_save_llama3_8b", "ms": round(ms4s, 5),
                               "GB/s": round(i4.algo_bytes / ms4s / 1e6, 2),
                               "frac": round(i4.algo_bytes / ms4s / 1e6 / HBM_PEAK_GBS, 4)}
        del sv4
        log(f"int4 save: {ms4s:.4f} ms")
        i4.free()
        del i4

        log("int4 decode: building inputs")
        dc = DecodeCase()
        res = {}
        for name, algo in (("mfma", amf_hip.DECODE_MFMA), ("valu", amf_hip.DECODE_VALU)):
            msd = time_launches(lambda: dc.launch(algo), args.steps, args.warmup)
            res[name] = msd
        msd = res["mfma"]
        gd = dc.algo_bytes / (msd * 1e-3) / 1e9
        result["int4_decode"] = {
            "workload": "decode_llama3_8b", "batch": dc.batch, "sum_ctx": dc.sum_ctx,
            "ms_per_layer_call": round(msd, 5),
            "tok_per_s_per_layer": round(dc.batch / (msd * 1e-3), 1),
            "tok_per_s_model_32_layers": round(dc.batch / (32 * msd * 1e-3), 1),
            "kv_tok_per_s": round(dc.sum_ctx / (msd * 1e-3), 1),
            "GB/s": round(gd, 2), "frac": round(gd / HBM_PEAK_GBS, 4),
            "valu_ms": round(res["valu"], 5), "mfma_over_valu_speedup": round(res["valu"] / msd, 3),
        }
        log(f"int4 decode: mfma {msd:.4f} ms ({gd:.1f} GB/s), valu {res['valu']:.4f} ms")
        del dc
        torch.cuda.empty_cache()
        log("reference formats: restore and save at the Llama-3-8B shape")
        fmts = {}
        for fmt in ("fp8_e4m3", "int4_sym_block", "int4_sym"):
            rc = RestoreCase(fmt, 32, 8, 128, 8192, 512, seed=8)
            r_ms = time_launches(rc.launch.launch, args.steps, args.warmup)
            sv = rc.save_launch()
            s_ms = time_launches(sv.launch, args.steps, args.warmup)
            fmts[fmt] = {"restore_ms": round(r_ms, 5),
                         "restore_GB/s": round(rc.algo_bytes / r_ms / 1e6, 1),
                         "save_ms": round(s_ms, 5),
                         "save_GB/s": round(rc.algo_bytes / s_ms / 1e6, 1),
                         "algo_bytes": rc.algo_bytes}
            del sv
            rc.free()
        result["reference_formats_llama3_8b_512p"] = fmts
        log(f"reference formats: {fmts}")
        log("connector: save / load through AMFKVConnector")
        cc = ConnectorCase()
        result["connector"] = cc.run(args.steps, args.warmup)
        log(f"connector: {result['connector']}")
        cc.free()
        del cc
        result.update(long_context_70b(args.steps, args.warmup))
    if cpu_timed is not None:
        log("fp8 restore: CPU baseline (8 of 32 layers, >= 10 s)")
        cb = cpu_timed()
        result["cpu_baseline"] = {"value": round(cb["value"], 3), "unit": "GB/s",
                                  "cores": torch.get_num_threads(), "kind": "port",
                                  "sample": cb["sample"], "seconds": round(cb["seconds"], 3),
                                  "cpu": platform.processor() or platform.machine(),
                                  "torch": torch.__version__}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
