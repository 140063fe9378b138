# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/_capi.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""ctypes binding of libsnowverify.so, the gfx950 verify-step kernel library.

Mirrors the loading pattern of the reference's binding (snowllm/_capi.py:144-194, 821-855):
torch's HIP runtime is loaded first so the kernel library binds to the same libamdhip64,
an ABI version is checked, every entry point gets an explicit signature, a nonzero status
becomes SnowLLMError, and the torch stream is always the last argument.

The library exports only the hot-path subset of the reference's C ABI under the same
symbol names and argument orders; it never poses as libsnowllm.so.
"""
import ctypes
import os
import pathlib
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_void_p

from .errors import SnowLLMError

__all__ = ["lib", "check", "synchronize", "assert_single_hip_runtime", "LIB_PATH", "ABI_VERSION"]

LIB_PATH = pathlib.Path(os.environ.get("SNOWVERIFY_LIB",
                                       pathlib.Path(__file__).resolve().parent / "libsnowverify.so"))
ABI_VERSION = 1


def _preload_hip_runtime() -> None:
    # Importing torch maps its bundled libamdhip64.so.7; the kernel library links the same
    # soname, so the dynamic linker reuses that runtime instead of /opt/rocm's copy.
    import torch  # noqa: F401
    lib_dir = pathlib.Path(torch.__file__).resolve().parent / "lib"
    hip = lib_dir / "libamdhip64.so"
    if hip.exists():
        ctypes.CDLL(str(hip), mode=ctypes.RTLD_GLOBAL)


def _load():
    if not LIB_PATH.exists():
        raise SnowLLMError(
            f"the kernel library {LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
            f"g.build()'` (or `python snowllm_amd/build.py`) first")
    _preload_hip_runtime()
    try:
        return ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    except OSError as exc:
        raise SnowLLMError(f"cannot load kernel library {LIB_PATH}: {exc}") from exc


lib = _load()

lib.snowllm_abi_version.restype = c_int
_got = lib.snowllm_abi_version()
if _got != ABI_VERSION:
    raise SnowLLMError(f"ABI mismatch: snowllm_amd expects {ABI_VERSION}, {LIB_PATH} provides {_got}. "
                       f"Rebuild the library.")


class Stream:
    pass


P, S = c_void_p, Stream
_SIGS = [
    ("snowllm_abi_version", c_int, []),
    ("snowllm_error_string", c_char_p, [c_int]),
    ("snowllm_synchronize", c_int, [S]),
    # acceptance
    ("snowllm_sampling_max_k", c_int64, []),
    ("snowllm_sampling_argmax", c_int, [P, P, c_int64, c_int64, S]),
    ("snowllm_spec_accept", c_int, [P] * 3 + [c_int64] * 4 + [S]),
    ("snowllm_sampling_workspace_bytes", c_int64, [c_int64] * 3),
    ("snowllm_sampling_softmax", c_int, [P, P, c_int64, c_int64, P, S]),
    ("snowllm_sampling_topk_topp", c_int, [P, P, P, c_int64, c_int64, c_int64, P, P, S]),
    ("snowllm_sampling_sample", c_int, [P] * 7 + [c_int64] * 4 + [S]),
    ("snowllm_sampling_penalties", c_int, [P, P, P, c_int, c_int, c_float, c_float, c_float, S]),
    ("snowllm_draft_reject", c_int, [P] * 10 + [c_int64] * 4 + [S]),
    ("snowverify_accept_reject", c_int, [P] * 10 + [c_int64] * 4 + [S]),
    ("snowverify_accept_greedy", c_int, [P] * 4 + [c_int64] * 3 + [S]),
    # DFlash 2 selector
    ("snowllm_draft_select_scratch_bytes", c_int64, [c_int64]),
    ("snowllm_draft_select", c_int, [P] * 7 + [c_int64] * 3 + [S]),
    ("snowllm_draft_sample", c_int, [P] * 12 + [c_int64] * 4 + [S]),
    ("snowverify_draft_select", c_int, [P] * 12 + [c_int64] * 4 + [S]),
    # GGUF k-quant GEMV
    ("snowllm_kquant_gguf_bytes", c_int64, [c_int, c_int64, c_int64]),
    ("snowllm_kquant_quant_bytes", c_int64, [c_int, c_int64, c_int64]),
    ("snowllm_kquant_meta_bytes", c_int64, [c_int, c_int64, c_int64]),
    ("snowllm_kquant_supported", c_int, [c_int]),
    ("snowllm_gemm_kquant_shuffle_b", c_int, [c_int, P, P, P, c_int64, c_int64, S]),
    ("snowverify_kquant_shuffle_split", c_int, [c_int, P, P, c_int64, P, P, c_int64, c_int64, S]),
    ("snowllm_gemm_kquant_a_ws_bytes", c_int64, [c_int64, c_int64]),
    ("snowllm_gemm_kquant_a", c_int, [c_int, P, P, P, P, c_int64, c_int64, c_int64, c_int, P, S]),
    ("snowverify_gemm_kquant_prepare_a", c_int, [P, c_int64, c_int64, P, S]),
    ("snowverify_gemm_kquant_a_prepared", c_int, [c_int, P, P, P, c_int64, c_int64, c_int64, c_int, P, S]),
    ("snowverify_gemm_kquant_a_prepared_ld", c_int,
     [c_int, P, P, P, c_int64, c_int64, c_int64, c_int64, c_int, P, S]),
    ("snowverify_gemm_kquant_a_noalloc", c_int, [c_int, P, P, P, P, c_int64, c_int64, c_int64, c_int, S]),
    ("snowverify_gemv_variant", None, [c_int]),
    # paged attention
    ("snowverify_paged_attention_scratch_bytes", c_int64, [c_int64] * 5),
    ("snowverify_paged_attention", c_int, [P] * 7 + [c_int64] * 7 + [c_float, P, c_int64, S]),
    ("snowverify_paged_attention_qk", c_int, [P] + [c_int64] * 4 + [P] * 4 + [c_int64] * 2 +
     [c_float] + [P] * 8 + [c_int64] * 7 + [c_float, P, c_int64, S]),
    ("snowverify_paged_attention_qk_ws", c_int, [P] + [c_int64] * 4 + [P] * 4 + [c_int64] * 2 +
     [c_float] + [P] * 8 + [c_int64] * 7 + [c_float, P, c_int64, P, S]),
    ("snowverify_attention_pages_per_split", c_int, [c_int]),
    ("snowverify_attention_d_split", c_int, [c_int]),
    ("snowverify_attention_ring", c_int, [c_int]),
    ("snowverify_attention_row_groups", c_int, [c_int]),
    # geometry-driven operator entry points (reference signatures)
    ("snowllm_qkv_proj_scratch_bytes", c_int64, [c_int64]),
    ("snowllm_attn_out_scale_oproj_scratch_bytes", c_int64, [c_int64]),
    ("snowllm_draft_paged_attn_num_slots", c_int64, [c_int64]),
    ("snowllm_draft_paged_attn_workspace_size", c_int64, [c_int64, c_int64]),
    ("snowllm_moe_router_shuffle_bytes", c_int64, [c_int64]),
    ("snowllm_inference_qkv", c_int, [P, P, P, P, c_float, P, P, c_int64, c_int, P, P, S]),
    ("snowllm_attn_output_plan", c_int, [c_int64, c_int, c_int, P]),
    ("snowllm_attn_output_gate", P, [P, c_int, c_int]),
    ("snowllm_attn_output_project", c_int, [P, P, c_int64, P, P, P, P, c_int, P, P, c_int64, c_int, c_int, S]),
    ("snowllm_paged_attention_scratch_bytes", c_int64, [c_int64, c_int64, c_int]),
    ("snowllm_paged_attention_varlen", c_int, [c_int, c_int64, c_int]),
    ("snowllm_paged_attention", c_int, [P, P, c_int64, S]),
    ("snowllm_paged_attention_prepared_bytes", c_int64, [c_int64, c_int64, c_int64, c_int]),
    ("snowllm_paged_attention_prepare", c_int, [P, P, c_int64, c_int64, c_int64, c_int64, S]),
    ("snowllm_paged_decode_max_q_tokens", c_int64, []),
    ("snowllm_paged_decode_num_slots", c_int64, [c_int64]),
    ("snowllm_paged_decode_workspace_size", c_int64, [c_int64, c_int64]),
    ("snowllm_paged_decode_plan_elems", c_int64, [c_int64, c_int64]),
    ("snowllm_paged_attn_decode_plan", c_int, [P, P, c_int64, c_int64, c_int64, c_int, S]),
    ("snowllm_paged_attn_decode", c_int, [P] * 7 + [c_int64] * 3 + [P, c_float] + [c_int64] * 4
     + [S]),
    ("snowllm_prefill_q_blocks", c_int64, [P, c_int64]),
    ("snowllm_prefill_q_block_map", None, [P, c_int64, P]),
    ("snowllm_kv_block_sizes", c_int64, [c_void_p, c_int64]),
    ("snowllm_moe_kquant_gate_up_quant_bytes", c_int64, [c_int, c_int64]),
    ("snowllm_moe_kquant_gate_up_meta_bytes", c_int64, [c_int, c_int64]),
    ("snowllm_moe_kquant_down_quant_bytes", c_int64, [c_int, c_int64]),
    ("snowllm_moe_kquant_down_meta_bytes", c_int64, [c_int, c_int64]),
    ("snowllm_moe_kquant_shuffle_gate_up", c_int, [c_int, P, P, P, P, c_int64, S]),
    ("snowllm_moe_kquant_shuffle_down", c_int, [c_int, P, P, P, c_int64, S]),
    ("snowllm_moe_shuffle_router_bytes", c_int64, []),
    ("snowllm_moe_shuffle_router", c_int, [P, P, P, S]),
    ("snowllm_moe_workspace_bytes", c_int64, [c_int64]),
    ("snowllm_inference_moe_workspace_bytes", c_int64, [c_int64, c_int64]),
    ("snowllm_inference_moe", c_int, [P] * 7 + [c_int64] * 3 + [S]),
    ("snowllm_inference_moe_norm", c_int, [P, P, P, P, c_float, P, P, P, P, c_int64, c_int64, S]),
    ("snowllm_fused_mlp_workspace_bytes", c_int64, [c_int64]),
    ("snowllm_inference_mlp", c_int, [P, P, P, P, c_int64, c_int, S]),
    ("snowllm_lm_head_scratch_bytes", c_int64, [c_int64]),
    ("snowllm_inference_head", c_int, [P, P, P, P, c_int64, S]),
    ("snowllm_shuffle_bytes", c_int64, [c_int64]),
    ("snowllm_lm_head_shuffle_weight", c_int, [P, P, S]),
    ("snowllm_lm_head", c_int, [P, P, P, c_int64, P, S]),
    ("snowllm_lm_head_kquant_gguf_bytes", c_int64, [c_int]),
    ("snowllm_lm_head_kquant_quant_bytes", c_int64, [c_int]),
    ("snowllm_lm_head_kquant_meta_bytes", c_int64, [c_int]),
    ("snowllm_lm_head_kquant_shuffle_weight", c_int, [c_int, P, P, P, S]),
    ("snowllm_lm_head_kquant", c_int, [c_int, P, P, P, P, c_int64, P, S]),
    ("snowllm_gather_embedding_q4_k", c_int, [P] * 3 + [c_int64] * 3 + [S]),
    ("snowllm_dspark_weight_bytes", c_int64, [c_int64] * 2),
    ("snowllm_dspark_pack_weight", c_int, [P, P, c_int64, c_int64, S]),
    ("snowllm_dspark_markov_workspace_bytes", c_int64, [c_int64] * 4),
    ("snowllm_dspark_markov", c_int, [P] * 10 + [c_int64] * 8 + [c_int, S]),
    ("snowllm_select_draft", c_int, [P]),
    ("snowllm_draft_count", c_int64, []),
    ("snowllm_draft_shape", c_int, [c_int, P]),
    ("snowllm_draft_name", c_int64, [c_int, c_char_p, c_int64]),
    ("snowllm_draft_projection_shape", c_int, [c_int, P]),
    ("snowllm_draft_projection_plan", c_int, [c_int, P, c_int64, P]),
    ("snowllm_draft_projections_workspace_bytes", c_int64, [c_int64]),
    ("snowllm_draft_projection", c_int, [c_int, P, P, P, P, c_int64, c_int64, S]),
    ("snowllm_draft_proj_shuffle_w", c_int, [c_int, P, P, S]),
    ("snowllm_draft_proj_shuffle_w_kquant", c_int, [c_int, c_int, P, P, P, S]),
    ("snowllm_rope_cos_sin", c_int, [P, P, P, P, c_int64, S]),
    ("snowllm_qk_norm_rope_cache", c_int, [P, c_int64, P, c_int64, P, c_int64] + [P] * 10 + [c_int64, c_float, c_int64, S]),
    # geometry and layer plumbing
    ("snowllm_model_config", None, [P]),
    ("snowllm_select_geometry", c_int, [c_int]),
    ("snowllm_active_geometry", c_int, []),
    ("snowllm_geometry_name", c_int64, [c_int, c_char_p, c_int64]),
    ("snowverify_define_geometry", c_int, [P]),
    ("snowverify_gather_embedding", c_int, [P, P, P, c_int64, c_int64, c_int64, c_int, S]),
    ("snowllm_gather_embedding", c_int, [P, P, P, c_int64, S]),
    ("snowverify_rmsnorm", c_int, [P, P, P, P, c_int64, c_int64, c_float, S]),
    ("snowllm_rmsnorm", c_int, [P, P, P, c_int64, c_float, S]),
    ("snowllm_rmsnorm_residual", c_int, [P, P, P, P, c_int64, c_float, S]),
    ("snowverify_rope_cos_sin", c_int, [P, P, P, P, c_int64, c_int64, S]),
    ("snowverify_qk_norm_rope_cache", c_int, [P, c_int64, P, P, P, P, P, P, P, P] + [c_int64] * 6
     + [c_float, S]),
    ("snowllm_resolve_slots", c_int, [P, c_int64, P, P, P, c_int64, c_int64, S]),
    ("snowllm_kv_pool_bytes", None, [c_int64, c_int64, c_int, P, P]),
    ("snowverify_swiglu", c_int, [P, c_int64, P, c_int64, c_int64, S]),
    ("snowverify_add_bf16", c_int, [P, P, P, c_int64, S]),
    ("snowverify_moe_route", c_int, [P, c_int64, c_int64, c_int64, c_int64, P, P, P, S]),
    # feed-forward
    ("snowverify_norm_prep", c_int, [P, P, P, P, P, P, c_int64, c_int64, c_float, S]),
    ("snowverify_norm_prep_moe", c_int, [P, P, c_int64] + [P] * 6 + [c_int64, c_int64, c_float, S]),
    ("snowverify_dense_bytes", c_int64, [c_int64, c_int64]),
    ("snowverify_dense_shuffle", c_int, [P, P, c_int64, c_int64, c_int, S]),
    ("snowverify_dense_gemv", c_int, [c_int, P, P, P, c_int64, c_int64, c_int64, c_int, S]),
    ("snowverify_gate_up_swiglu", c_int, [c_int, P, P, P, P, c_int64, c_int64, c_int64, S]),
    ("snowverify_moe_plan_bytes", c_int64, []),
    ("snowverify_moe_max_slots", c_int64, [c_int64, c_int64, c_int64, c_int]),
    ("snowverify_moe_plan", c_int, [P, c_int64, c_int64, c_int64, c_int, P, S]),
    ("snowverify_moe_route_plan", c_int, [P, c_int64, c_int64, c_int64, c_int64, P, P, P, P, S]),
    ("snowverify_norm_router_plan", c_int, [P] * 4 + [c_float] + [P] * 4 + [c_int64] * 4 +
     [P] * 4 + [S]),
    ("snowverify_moe_gate_up", c_int, [c_int] + [P] * 7 + [c_int64] * 5 + [S]),
    ("snowverify_moe_down", c_int, [c_int] + [P] * 10 + [c_int64] * 4 + [S]),
    ("snowverify_moe_gate_up_down", c_int, [c_int] + [P] * 15 + [c_int64] * 5 + [S]),
    ("snowverify_moe_sync_error", c_int, []),
    ("snowverify_moe_combine", c_int, [P, P, P, c_int64, c_int64, c_int64, S]),
    ("snowverify_moe_experts", c_int, [c_int] + [P] * 16 + [c_int64] * 5 + [S]),
]

_missing = []
for _name, _res, _args in _SIGS:
    try:
        _fn = getattr(lib, _name)
    except AttributeError:
        _missing.append(_name)
        continue
    _fn.restype = _res
    _fn.argtypes = [c_void_p if _a is S else _a for _a in _args]
if _missing:
    raise SnowLLMError(f"{LIB_PATH} is missing {len(_missing)} entry points this binding needs:\n  "
                       + "\n  ".join(_missing))

SYMBOLS = tuple(n for n, _, _ in _SIGS)
LAUNCHES = frozenset(n for n, _, a in _SIGS if a and S in a)


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib.snowllm_error_string(status).decode()
        raise SnowLLMError(f"{what}: hip status {status}: {msg}")


def synchronize(stream: int = 0) -> None:
    check(lib.snowllm_synchronize(stream), "synchronize")


def hip_runtimes() -> set[str]:
    try:
        lines = pathlib.Path("/proc/self/maps").read_text().splitlines()
    except OSError:
        return set()
    return {os.path.realpath(line.rsplit(" ", 1)[-1].strip())
            for line in lines if "libamdhip64.so" in line}


def assert_single_hip_runtime() -> None:
    paths = hip_runtimes()
    if len(paths) > 1:
        raise SnowLLMError("two HIP runtimes are loaded in this process -- torch's device pointers "
                           "are not valid in the kernels:\n  " + "\n  ".join(sorted(paths)))
