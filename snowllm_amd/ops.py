"""The operator namespace, laid out like `snowllm.ops` for the verify-step subset."""
from ._common import empty_bytes, synchronize  # noqa: F401
from .sampling import (SAMPLING_MAX_K, argmax, probabilities, sample,  # noqa: F401
                       sample_workspace_bytes)
from .metadata import spec_accept  # noqa: F401
from . import dflash  # noqa: F401
from .gemm import (Q4_K, Q8_0, gemm_kquant_a, gemm_kquant_a_ws_bytes,  # noqa: F401
                   gemm_kquant_shuffle_b, kquant_bytes,
                   gemm_kquant_prepare_a, gemm_kquant_a_prepared)
from .attention import (kv_pool_bytes, paged_attention_explicit,  # noqa: F401
                        paged_attention_scratch_bytes)
