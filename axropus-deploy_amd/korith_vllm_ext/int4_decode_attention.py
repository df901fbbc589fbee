"""int4_decode_attention: the decode entry point (reference:
korith_vllm_ext/int4_decode_attention.py:6-9), dispatched for storage
"int4_sym" / active "fp8_e4m3" like the reference.

Positional use is unchanged: int4_decode_attention(q, k, v, scale=None,
mask=None).  Paged GQA decode over an INT4 page pool is selected by keyword:
int4_decode_attention(q, kv_pool, block_tables=..., context_lens=...)."""

from .kernels.dispatch import dispatch_kernel, fallback_fp16_kernel  # noqa: F401


def int4_decode_attention(*args, **kwargs):
    kernel = dispatch_kernel("int4_sym", "fp8_e4m3")
    return kernel(*args, **kwargs)
