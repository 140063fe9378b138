// The model geometry the reference compiles into its library (snowllm/_capi.py:44-113): 37
// int64 fields in the reference's order. This build keeps it as run-time data, selected with
// snowllm_select_geometry or installed with snowverify_define_geometry.
#pragma once
#include <stdint.h>

// Field order of the reference's BuildGeometry (snowllm/_capi.py:44-64).
struct BuildGeometry {
  int64_t hidden, num_heads, num_kv_heads, head_size, block_size, vocab_size;
  int64_t qkv_proj_n, qkv_q_head_stride, qkv_off_scale, qkv_off_k, qkv_off_v;
  int64_t lin_num_k_heads, lin_num_v_heads, lin_head_k, lin_head_v, lin_key_dim;
  int64_t lin_value_dim, lin_conv_dim, lin_conv_k, lin_conv_state, lin_in_proj_n;
  int64_t lin_in_proj_n_pad;
  int64_t lin_in_proj_ba_n_pad, lin_off_qkv, lin_off_z, lin_off_b, lin_off_a;
  int64_t moe_num_experts, moe_shared_expert, moe_num_slabs, moe_topk, moe_topk_all;
  int64_t moe_inter, sampling_max_k, lm_head_decode_max_m, mlp_inter;
  int64_t mlp_gate_up_n;
};
static_assert(sizeof(BuildGeometry) == 37 * 8, "BuildGeometry layout");

// The active geometry (defined in layer.hip).
const BuildGeometry& active_geometry();
