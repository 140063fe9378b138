# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/inference.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Geometry-driven operator entry points (mirrors snowllm/ops/inference.py:10-104): weights are
marshalled into the reference's _Weight descriptor and the shapes come from the active
geometry. The weights hold this library's repacked layouts (KQuantProjWeight from
gemm_kquant_shuffle_b, KQuantExpertWeight for an expert stack, dense 16-bit matrices repacked
by layers.dense_shuffle)."""
import ctypes
from typing import NamedTuple, Optional

import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream


class KQuantProjWeight(NamedTuple):
    """A repacked k-quant matrix (snowllm/ops/gemm.py; kind 2)."""
    quant: torch.Tensor
    meta: torch.Tensor
    fmt: int


class KQuantExpertWeight(NamedTuple):
    """The experts' repacked matrices of one layer back to back (kind 3): p0 = quant stack,
    p1 = meta stack."""
    p0: torch.Tensor
    p1: torch.Tensor
    p2: Optional[torch.Tensor]
    fmt: int


class _Weight(ctypes.Structure):  # snowllm/ops/inference.py:10-12
    _fields_ = [("data", ctypes.c_void_p * 3), ("scale", ctypes.c_void_p),
                ("kind", ctypes.c_int), ("fmt", ctypes.c_int)]


def _weight(w, scale=None):
    """snowllm/ops/inference.py:15-22."""
    if w is None:
        return _Weight((ctypes.c_void_p * 3)(), 0, -1, 0)
    if hasattr(w, "p0"):
        return _Weight((ctypes.c_void_p * 3)(*[_p(t) for t in (w.p0, w.p1, w.p2)]), 0, 3, w.fmt)
    if hasattr(w, "quant"):
        return _Weight((ctypes.c_void_p * 3)(_p(w.quant), _p(w.meta), 0), 0, 2, w.fmt)
    return _Weight((ctypes.c_void_p * 3)(_p(w), 0, 0), _p(scale), int(scale is not None), 0)


def _weights(*pairs):
    return (_Weight * len(pairs))(*[_weight(w, s) for w, s in pairs])


def _io(x, out):
    _chk(x, "hidden", torch.bfloat16, x.shape[0], x.shape[1])
    _chk(out, "output", torch.bfloat16, x.shape[0], out.shape[1])


def _norm(x, residual, gamma):
    """snowllm/ops/attention_full.py:578-585."""
    if gamma is None:
        return 0, 0
    _chk(gamma, "gamma", torch.bfloat16, x.shape[1])
    if residual is not None:
        _chk(residual, "residual", torch.bfloat16, *x.shape)
    return _p(residual), _p(gamma)


def qkv_proj_scratch_bytes(M: int) -> int:
    return int(lib.snowllm_qkv_proj_scratch_bytes(int(M)))


def inference_qkv(x, w, scale, v, kv, scratch, out, path, residual=None, gamma=None, eps=0.,
                  *, index_w=None, index_out=None):
    """QKV projection with the fused input norm (snowllm/ops/inference.py:34-43)."""
    _io(x, out)
    res_ptr, gamma_ptr = _norm(x, residual, gamma)
    if index_w is not None or index_out is not None:
        raise SnowLLMError("this build carries no attention indexer")
    weights = _weights((w, scale), (v, None), (kv, None))
    check(lib.snowllm_inference_qkv(weights, _p(x), res_ptr, gamma_ptr, eps, _p(scratch),
                                    _p(out), x.shape[0], int(path), None, None, _stream()),
          "inference_qkv")


def mlp_workspace_bytes(M: int) -> int:
    return int(lib.snowllm_fused_mlp_workspace_bytes(int(M)))


def inference_mlp(x, gate, down, out, scratch, decode, gate_scale=None, down_scale=None,
                  up=None):
    """Dense SwiGLU MLP (snowllm/ops/inference.py:46-51)."""
    _io(x, out)
    weights = _weights((gate, gate_scale), (up, None), (down, down_scale))
    check(lib.snowllm_inference_mlp(weights, _p(x), _p(out), _p(scratch), x.shape[0],
                                    int(decode), _stream()), "inference_mlp")


def moe_workspace_bytes(rows: int) -> int:
    return int(lib.snowllm_moe_workspace_bytes(int(rows)))


def inference_moe_workspace_bytes(rows: int) -> int:
    return int(lib.snowllm_inference_moe_workspace_bytes(int(rows), 0))


def inference_moe(x, router, gate, down, shared_gate, shared_down, out, scratch, gate_scale=None,
                  down_scale=None, *, token_ids=None, tid2eid=None):
    """MoE block on normalised rows (snowllm/ops/inference.py:60-76)."""
    _io(x, out)
    weights = _weights((gate, gate_scale), (down, down_scale), (shared_gate, None),
                       (shared_down, None))
    need = inference_moe_workspace_bytes(x.shape[0])
    capacity = 0 if scratch is None else scratch.nbytes
    if capacity < need:
        raise SnowLLMError(f"MoE needs {need} scratch bytes")
    check(lib.snowllm_inference_moe(weights, _p(x), _p(router), _p(token_ids), _p(tid2eid),
                                    _p(out), _p(scratch), capacity, x.shape[0], 0, _stream()),
          "inference_moe")


def inference_moe_norm(x, residual, gamma, eps, hidden_row, router, gate, down, shared_gate,
                       shared_down, out, scratch, gate_scale=None, down_scale=None):
    """Post-attention norm + MoE block (snowllm/ops/inference.py:82-95)."""
    _io(x, out)
    M, H = x.shape
    _chk(residual, "residual", torch.bfloat16, M, H)
    _chk(gamma, "gamma", torch.bfloat16, H)
    _chk(hidden_row, "hidden scratch", torch.bfloat16, M, H)
    weights = _weights((gate, gate_scale), (down, down_scale), (shared_gate, None),
                       (shared_down, None))
    capacity = 0 if scratch is None else scratch.nbytes
    if capacity < inference_moe_workspace_bytes(M):
        raise SnowLLMError("MoE scratch is too small")
    check(lib.snowllm_inference_moe_norm(weights, _p(x), _p(residual), _p(gamma), eps,
                                         _p(hidden_row), _p(router), _p(out), _p(scratch),
                                         capacity, M, _stream()), "inference_moe_norm")


def _expert_blocks(t, what, want):
    if t.device.type != "cuda" or t.dtype != torch.uint8 or not t.is_contiguous():
        raise SnowLLMError(f"{what}: contiguous uint8 GGUF blocks on the GPU expected")
    if t.numel() != want:
        raise SnowLLMError(f"{what}: {t.numel()} GGUF bytes, the active geometry needs {want}")


def moe_kquant_shuffle_gate_up(gate, up, fmt: int, num_experts: int) -> KQuantExpertWeight:
    """ffn_gate_exps / ffn_up_exps GGUF blocks [E, F, H] -> the experts' packed gate/up stack
    (snowllm/ops/moe.py:136-145); F = moe_inter and H = hidden of the active geometry."""
    from .gemm import kquant_bytes
    g = _geometry()
    want = num_experts * kquant_bytes(fmt, g.moe_inter, g.hidden)[2]
    _expert_blocks(gate, "gate blocks", want)
    _expert_blocks(up, "up blocks", want)
    quant = torch.empty(lib.snowllm_moe_kquant_gate_up_quant_bytes(fmt, num_experts),
                        dtype=torch.uint8, device="cuda")
    meta = torch.empty(lib.snowllm_moe_kquant_gate_up_meta_bytes(fmt, num_experts),
                       dtype=torch.uint8, device="cuda")
    check(lib.snowllm_moe_kquant_shuffle_gate_up(fmt, _p(gate), _p(up), _p(quant), _p(meta),
                                                 num_experts, _stream()),
          "moe_kquant_shuffle_gate_up")
    return KQuantExpertWeight(quant, meta, None, fmt)


def moe_kquant_shuffle_down(down, fmt: int, num_experts: int) -> KQuantExpertWeight:
    """ffn_down_exps GGUF blocks [E, H, F] -> the experts' packed down stack
    (snowllm/ops/moe.py:148-160)."""
    from .gemm import kquant_bytes
    g = _geometry()
    _expert_blocks(down, "down blocks", num_experts * kquant_bytes(fmt, g.hidden, g.moe_inter)[2])
    quant = torch.empty(lib.snowllm_moe_kquant_down_quant_bytes(fmt, num_experts),
                        dtype=torch.uint8, device="cuda")
    meta = torch.empty(lib.snowllm_moe_kquant_down_meta_bytes(fmt, num_experts),
                       dtype=torch.uint8, device="cuda")
    check(lib.snowllm_moe_kquant_shuffle_down(fmt, _p(down), _p(quant), _p(meta), num_experts,
                                              _stream()), "moe_kquant_shuffle_down")
    return KQuantExpertWeight(quant, meta, None, fmt)


def moe_shuffle_router(router, bias=None) -> torch.Tensor:
    """bf16 router [E + 1, H] (routed experts, then the shared expert's gate) -> the router
    GEMV's layout (snowllm/ops/moe.py:81-86). A bias is not supported."""
    g = _geometry()
    _chk(router, "router", torch.bfloat16, g.moe_num_experts + 1, g.hidden)
    if bias is not None:
        raise SnowLLMError("router bias: not supported by this library")
    out = torch.empty(lib.snowllm_moe_shuffle_router_bytes(), dtype=torch.uint8, device="cuda")
    check(lib.snowllm_moe_shuffle_router(_p(router), None, _p(out), _stream()),
          "moe_shuffle_router")
    return out


def _geometry():
    from .geometry import build_geometry
    return build_geometry()


def lm_head_scratch_bytes(M: int) -> int:
    return int(lib.snowllm_lm_head_scratch_bytes(int(M)))


def inference_head(x, w, out, scratch):
    """LM head (snowllm/ops/inference.py:98-104)."""
    _chk(x, "hidden", torch.bfloat16, x.shape[0], x.shape[1])
    _chk(out, "logits", torch.float32, x.shape[0], out.shape[1])
    weight = _weight(w)
    check(lib.snowllm_inference_head(ctypes.byref(weight), _p(x), _p(out), _p(scratch),
                                     x.shape[0], _stream()), "inference_head")
