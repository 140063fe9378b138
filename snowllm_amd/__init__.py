"""snowllm_amd: a gfx950 (MI355X) implementation of SnowLLM's speculative-decoding verify step.

`snowllm_amd.ops` mirrors the reference's operator names (snowllm.ops) for the verify path;
`snowllm_amd._capi` binds the kernel library libsnowverify.so.
"""
from .errors import SnowLLMError  # noqa: F401
