"""Seeded synthetic inputs of the benchmark configurations (test infrastructure).

Values are N(0, 1) drawn from torch.Generator('cpu'), cast to bf16.  Outlier
channels: round(0.02 * head_dim) head_dim channels chosen by randperm are
scaled x20 in every layer, head and token (K and V).  Block tables are seeded
randperm draws over the pool.

Workloads (layers, KV heads, head_dim, block_size 16):
  raw_qwen05b        24, 2, 64;   pool 4096, prefix 128 pages, no outliers
  fp8_llama3_8b      32, 8, 128;  pool 8192, prefix 512 pages
  int4_llama3_8b     32, 8, 128;  pool 16384, prefix 2048 pages
  decode_llama3_8b   B 32, Hq 32, Hkv 8, ctx U[1024, 32768]
  fp8_llama3_70b     80, 8, 128;  prefix 8192 pages
  decode_llama3_70b  B 8, Hq 64, Hkv 8, ctx 131072
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass(frozen=True)
class KVShape:
    layers: int
    kv_heads: int
    head_dim: int
    block_size: int
    pool_blocks: int
    prefix_blocks: int
    outliers: bool
    seed: int


WORKLOADS = {
    "raw_qwen05b": KVShape(24, 2, 64, 16, 4096, 128, False, 1),
    "fp8_llama3_8b": KVShape(32, 8, 128, 16, 8192, 512, True, 2),
    "int4_llama3_8b": KVShape(32, 8, 128, 16, 16384, 2048, True, 3),
    "fp8_llama3_70b": KVShape(80, 8, 128, 16, 8192, 8192, True, 5),
}


def outlier_channels(head_dim: int, g: torch.Generator) -> torch.Tensor:
    k = int(round(0.02 * head_dim))
    return torch.randperm(head_dim, generator=g)[:k]


def kv_values(shape, head_dim: int, g: torch.Generator, outliers: bool,
              dtype=torch.bfloat16) -> torch.Tensor:
    """N(0,1) of `shape` (last dim head_dim) with the x20 outlier channels."""
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    if outliers:
        ch = outlier_channels(head_dim, g)
        x[..., ch] *= 20.0
    return x.to(dtype)


def prefix_pages(s: KVShape, layers: Optional[int] = None, pages: Optional[int] = None,
                 dtype=torch.bfloat16) -> torch.Tensor:
    """[L, 2, n, bs, H, D] prefix KV (L, n default to the workload's)."""
    g = torch.Generator().manual_seed(s.seed)
    L = layers or s.layers
    n = pages or s.prefix_blocks
    return kv_values((L, 2, n, s.block_size, s.kv_heads, s.head_dim), s.head_dim, g, s.outliers,
                     dtype)


def block_table(pool: int, n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(pool, generator=g)[:n].to(torch.int32)


@dataclass(frozen=True)
class DecodeShape:
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    ctx_lo: int
    ctx_hi: int
    seed: int


DECODE_WORKLOADS = {
    "decode_llama3_8b": DecodeShape(32, 32, 8, 128, 16, 1024, 32768, 4),
    "decode_llama3_70b": DecodeShape(8, 64, 8, 128, 16, 131072, 131072, 6),
}


def decode_case(d: DecodeShape):
    """Returns (q bf16 [B, Hq, D], context_lens int32 [B], block_tables int32
    [B, max_pages], pool_pages).  Pages of all sequences come from one shared
    randperm over a pool of exactly sum(pages) pages."""
    g = torch.Generator().manual_seed(d.seed)
    q = torch.randn(d.batch, d.q_heads, d.head_dim, generator=g).to(torch.bfloat16)
    if d.ctx_lo == d.ctx_hi:
        ctx = torch.full((d.batch,), d.ctx_lo, dtype=torch.int32)
    else:
        ctx = torch.randint(d.ctx_lo, d.ctx_hi + 1, (d.batch,), generator=g, dtype=torch.int32)
    pages = [(int(c) + d.block_size - 1) // d.block_size for c in ctx]
    pool = sum(pages)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    max_pages = max(pages)
    bt = torch.zeros(d.batch, max_pages, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    return q, ctx, bt, pool


def decode_kv_pool(d: DecodeShape, pool: int, dtype=torch.bfloat16) -> torch.Tensor:
    """[2, pool, bs, Hkv, D] KV values of every pool page (x20 outlier channels)."""
    g = torch.Generator().manual_seed(d.seed + 1000)
    return kv_values((2, pool, d.block_size, d.kv_heads, d.head_dim), d.head_dim, g, True, dtype)
