"""codecs/base.py - codec interface, CompressedKV container and registry.

Same contract as the reference (korith_vllm_ext/codecs/base.py:26-158): a
Codec turns a raw KV tensor [..., tokens, heads, head_dim] into a
CompressedKV and back; codecs register under their format name.  Here every
codec runs on the GPU through libamf_hip.so; the container additionally keeps
the device blob the kernels wrote (`meta["_blob"]`) so decompression and the
VRAM pool read the codes where they lie.
"""

from __future__ import annotations

import abc
from dataclasses import dataclass, field
from typing import Any, Dict, List

import torch

FMT_FP16 = "fp16"
FMT_BF16 = "bf16"
FMT_FP8_E4M3 = "fp8_e4m3"
FMT_FP8_E5M2 = "fp8_e5m2"
FMT_INT4_SYM = "int4_sym"            # symmetric, one scale per head_dim channel
FMT_INT4_BLOCK = "int4_sym_block"    # symmetric, one scale per 128-token block
FMT_INT2_SYM = "int2_sym"
FMT_NVFP4 = "nvfp4"
FMT_TURBOQUANT = "turboquant"
# Formats added by this implementation (per-(page, head) FP8 scale and
# asymmetric 32-dim-group INT4; byte layouts in include/amf_hip.h).
FMT_FP8_E4M3_PH = "fp8_e4m3_ph"
FMT_INT4_ASYM_G32 = "int4_asym_g32"
# Raw bytes of an already 1-byte KV cache (no re-quantization).
FMT_RAW = "raw"

ALL_FORMATS = (
    FMT_FP16,
    FMT_BF16,
    FMT_FP8_E4M3,
    FMT_FP8_E5M2,
    FMT_INT4_SYM,
    FMT_INT4_BLOCK,
    FMT_INT2_SYM,
    FMT_NVFP4,
    FMT_TURBOQUANT,
    FMT_FP8_E4M3_PH,
    FMT_INT4_ASYM_G32,
)


@dataclass
class CompressedKV:
    """Compressed KV blob: packed payload, scales, and what restores it.

    ``data`` is the packed payload (float8_e4m3fn for the FP8 formats, uint8
    for the INT4 formats), ``scales`` the scale side table, ``shape`` the
    original tensor shape, ``dtype_original`` its dtype.
    """

    format: str
    data: torch.Tensor
    scales: torch.Tensor
    tensor_scale: float = 1.0
    shape: tuple = ()
    dtype_original: torch.dtype = torch.float16
    meta: Dict[str, Any] = field(default_factory=dict)

    def nbytes(self) -> int:
        total = self.data.numel() * self.data.element_size()
        if self.scales is not None:
            total += self.scales.numel() * self.scales.element_size()
        return total

    def original_bytes(self) -> int:
        numel = 1
        for d in self.shape:
            numel *= d
        return numel * torch.tensor([], dtype=self.dtype_original).element_size()


class Codec(abc.ABC):
    """A KV cache compression format (reference: codecs/base.py:89-133)."""

    FORMAT: str = ""

    @abc.abstractmethod
    def compress(self, raw_kv: torch.Tensor) -> CompressedKV:
        """raw_kv: [..., num_tokens, num_heads, head_dim] on the GPU."""

    @abc.abstractmethod
    def decompress_to(self, compressed: CompressedKV,
                      target_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """Back to a plain tensor of ``target_dtype`` and the original shape."""

    @abc.abstractmethod
    def memory_ratio(self) -> float:
        """Compressed size / FP16 size."""

    def compressed_bytes(self, numel: int) -> int:
        return int(round(numel * 2 * self.memory_ratio()))

    def supports_dtype(self, dtype: torch.dtype) -> bool:
        return dtype in (torch.float16, torch.bfloat16, torch.float32)

    def __repr__(self) -> str:
        return f"<Codec format={self.FORMAT} ratio={self.memory_ratio():.3f}>"


_REGISTRY: Dict[str, Codec] = {}


def register_codec(codec: Codec) -> None:
    if not codec.FORMAT:
        raise ValueError(f"Codec {codec!r} has no FORMAT string")
    _REGISTRY[codec.FORMAT] = codec


def get_codec(format: str) -> Codec:
    """Look up a registered codec; KeyError for unknown or unimplemented formats."""
    if format not in _REGISTRY:
        raise KeyError(f"Unknown codec format {format!r}. Registered: {list(_REGISTRY)}")
    return _REGISTRY[format]


def list_codecs() -> List[str]:
    return sorted(_REGISTRY.keys())
