"""The model geometry (snowllm/_capi.py:44-113): the reference compiles it into its library;
here it is run-time data that the geometry-driven entry points read."""
import ctypes

from ._capi import SnowLLMError, lib

GEOMETRY_FIELDS = (
    "hidden", "num_heads", "num_kv_heads", "head_size", "block_size", "vocab_size",
    "qkv_proj_n", "qkv_q_head_stride", "qkv_off_scale", "qkv_off_k", "qkv_off_v",
    "lin_num_k_heads", "lin_num_v_heads", "lin_head_k", "lin_head_v", "lin_key_dim",
    "lin_value_dim", "lin_conv_dim", "lin_conv_k", "lin_conv_state", "lin_in_proj_n",
    "lin_in_proj_n_pad", "lin_in_proj_ba_n_pad", "lin_off_qkv", "lin_off_z", "lin_off_b",
    "lin_off_a", "moe_num_experts", "moe_shared_expert", "moe_num_slabs", "moe_topk",
    "moe_topk_all", "moe_inter", "sampling_max_k", "lm_head_decode_max_m", "mlp_inter",
    "mlp_gate_up_n")

GEO_QWEN36_35B_A3B = 0   # BASELINE configs 4 and 5
GEO_DENSE_8B = 100
GEO_CUSTOM = 1000        # installed by define_geometry


class BuildGeometry(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in GEOMETRY_FIELDS]


def build_geometry() -> BuildGeometry:
    g = BuildGeometry()
    lib.snowllm_model_config(ctypes.byref(g))
    return g


def select_geometry(geo: int) -> None:
    if lib.snowllm_select_geometry(int(geo)) != 0:
        raise SnowLLMError(f"this build carries no geometry {geo}")


def active_geometry() -> int:
    return int(lib.snowllm_active_geometry())


def define_geometry(**fields) -> None:
    """Install a geometry (id GEO_CUSTOM): unnamed fields are zero."""
    g = BuildGeometry(**{k: int(v) for k, v in fields.items()})
    if lib.snowverify_define_geometry(ctypes.byref(g)) != 0:
        raise SnowLLMError("invalid geometry")
