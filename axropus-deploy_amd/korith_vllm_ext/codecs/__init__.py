"""Codec package: KV cache compression formats of the AMF VRAM pool.

Reference: korith_vllm_ext/codecs/__init__.py.  Every registered codec runs
on the GPU through libamf_hip.so.
"""

from __future__ import annotations

from .base import (
    ALL_FORMATS,
    FMT_BF16,
    FMT_FP8_E4M3,
    FMT_FP8_E4M3_PH,
    FMT_FP8_E5M2,
    FMT_FP16,
    FMT_INT2_SYM,
    FMT_INT4_ASYM_G32,
    FMT_INT4_BLOCK,
    FMT_INT4_SYM,
    FMT_NVFP4,
    FMT_RAW,
    FMT_TURBOQUANT,
    Codec,
    CompressedKV,
    get_codec,
    list_codecs,
    register_codec,
)
from .amf_codec import (
    FP8E4M3Codec,
    FP8PageHeadCodec,
    FP8ScaleSidecar,
    INT4AsymG32Codec,
    INT4PerBlockCodec,
    INT4PerChannelCodec,
    apply_fp8_scales,
)


def select_codec(hw_sm: int, accuracy_budget: float = 0.005, density_budget: float = 0.25) -> str:
    """Format choice by device generation and budgets, with the reference's
    decision table (codecs/__init__.py:40-67).  hw_sm is major * 10 + minor of
    torch.cuda.get_device_capability(); ROCm torch reports gfx950 as 95, which
    lands in the >= 90 row.  nvfp4 and turboquant are not registered in this
    build: get_codec() raises KeyError for them."""
    if hw_sm >= 100:
        if density_budget <= 0.20 and accuracy_budget >= 0.005:
            return FMT_TURBOQUANT
        return FMT_NVFP4
    if hw_sm >= 90:
        if density_budget <= 0.20:
            return FMT_TURBOQUANT
        if density_budget <= 0.25:
            return FMT_INT4_BLOCK
        return FMT_FP8_E4M3
    if hw_sm >= 80:
        return FMT_INT4_BLOCK
    return FMT_FP16


__all__ = [
    "ALL_FORMATS", "Codec", "CompressedKV", "FMT_BF16", "FMT_FP16", "FMT_FP8_E4M3",
    "FMT_FP8_E4M3_PH", "FMT_FP8_E5M2", "FMT_INT2_SYM", "FMT_INT4_ASYM_G32", "FMT_INT4_BLOCK",
    "FMT_INT4_SYM", "FMT_NVFP4", "FMT_RAW", "FMT_TURBOQUANT", "FP8E4M3Codec", "FP8PageHeadCodec",
    "FP8ScaleSidecar", "INT4AsymG32Codec", "INT4PerBlockCodec", "INT4PerChannelCodec",
    "apply_fp8_scales", "get_codec", "list_codecs", "register_codec", "select_codec",
]
