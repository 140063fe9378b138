"""The operator namespace, laid out like `snowllm.ops` for the verify-step subset."""
from ._common import empty_bytes, synchronize  # noqa: F401
from .sampling import (SAMPLING_MAX_K, argmax, probabilities, sample,  # noqa: F401
                       sample_workspace_bytes)
from .metadata import spec_accept  # noqa: F401
from . import dflash  # noqa: F401
from .gemm import (Q4_K, Q8_0, gemm_kquant_a, gemm_kquant_a_ws_bytes,  # noqa: F401
                   gemm_kquant_shuffle_b, kquant_bytes, kquant_shuffle_stack,
                   gemm_kquant_prepare_a, gemm_kquant_a_prepared, gemm_kquant_a_noalloc)
from .attention import (kv_pool_bytes, paged_attention_explicit,  # noqa: F401
                        paged_attention_explicit_scratch_bytes, paged_attention, paged_attention_qk,
                        FUSED_QK_MAX_HALF,
                        paged_attention_scratch_bytes, paged_attention_varlen, attn_output_plan,
                        attn_output_shape, attn_output_gating, attn_output_project, rope_cos_sin,
                        qk_norm_rope_cache, paged_attention_prepare,
                        paged_attention_uses_prepared, PAGED_DECODE_MAX_Q_TOKENS, KV_BLOCK_SIZES,
                        paged_decode_num_slots, paged_decode_workspace_size,
                        paged_decode_plan_elems, paged_attn_decode_plan, paged_attn_decode,
                        prefill_q_plan)
from .inference import (KQuantProjWeight, KQuantExpertWeight, inference_qkv,  # noqa: F401
                        qkv_proj_scratch_bytes, inference_mlp, mlp_workspace_bytes,
                        inference_moe, inference_moe_norm, inference_moe_workspace_bytes,
                        moe_workspace_bytes, inference_head, lm_head_scratch_bytes,
                        moe_kquant_shuffle_gate_up, moe_kquant_shuffle_down,
                        moe_shuffle_router)
from .embedding import (lm_head_shuffle_weight, gather_embedding,  # noqa: F401
                        gather_embedding_q4_k, lm_head_kquant_shuffle_weight, lm_head_kquant,
                        lm_head)
from .dspark import (dspark_pack_weight, dspark_markov,  # noqa: F401
                     dspark_markov_workspace_bytes)
from .geometry import (build_geometry, select_geometry, active_geometry,  # noqa: F401
                       define_geometry)
