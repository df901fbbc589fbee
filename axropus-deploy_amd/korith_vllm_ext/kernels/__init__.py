"""Decode-attention kernels of the AMF path (reference: korith_vllm_ext/kernels/__init__.py)."""

from __future__ import annotations

from .dispatch import (
    KERNEL_DISPATCH,
    dense_attention,
    int4_sym_attention,
    dispatch_kernel,
    fallback_fp16_kernel,
    get_current_sm_version,
    hip_decode_attention,
    paged_int4_decode,
    register_kernel,
    try_load_cuda_extension,
)

__all__ = [
    "KERNEL_DISPATCH",
    "dense_attention",
    "int4_sym_attention",
    "dispatch_kernel",
    "fallback_fp16_kernel",
    "get_current_sm_version",
    "hip_decode_attention",
    "paged_int4_decode",
    "register_kernel",
    "try_load_cuda_extension",
]
