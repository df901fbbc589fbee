"""Compatibility module: the codecs live in korith_vllm_ext.codecs
(reference: korith_vllm_ext/amf_codec.py re-exports them the same way)."""

from .codecs import *  # noqa: F401,F403
from .codecs import __all__  # noqa: F401
