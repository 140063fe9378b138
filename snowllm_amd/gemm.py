# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/gemm.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""GGUF k-quant GEMM operators (snowllm/ops/gemm.py:130-163).

Format ids follow the reference (ops/moe.py:189-190): 4 = Q4_K, 8 = Q8_0.
"""
import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream, empty_bytes

Q4_K, Q8_0 = 4, 8


def kquant_bytes(fmt: int, N: int, K: int) -> tuple[int, int, int]:
    return (lib.snowllm_kquant_quant_bytes(fmt, N, K), lib.snowllm_kquant_meta_bytes(fmt, N, K),
            lib.snowllm_kquant_gguf_bytes(fmt, N, K))


def gemm_kquant_shuffle_b(fmt: int, b_gguf: torch.Tensor, N: int,
                          K: int) -> tuple[torch.Tensor, torch.Tensor]:
    quant_bytes, meta_bytes, gguf_bytes = kquant_bytes(fmt, N, K)
    if quant_bytes < 0 or meta_bytes < 0:
        raise SnowLLMError(f"gemm_kquant_shuffle_b: format {fmt} with N={N}, K={K} is not supported "
                           f"(N must be a multiple of 16 and K of 256)")
    _chk(b_gguf, "b_gguf", torch.uint8)
    if b_gguf.numel() != gguf_bytes:
        raise SnowLLMError(f"gemm_kquant_shuffle_b: expected {gguf_bytes} bytes of GGUF blocks for "
                           f"a [{N}, {K}] weight at format {fmt}, got {b_gguf.numel()}")
    quant, meta = empty_bytes(quant_bytes), empty_bytes(meta_bytes)
    check(lib.snowllm_gemm_kquant_shuffle_b(fmt, _p(b_gguf), _p(quant), _p(meta), N, K, _stream()),
          "gemm_kquant_shuffle_b")
    return quant, meta


def kquant_shuffle_stack(fmt: int, b_gguf: torch.Tensor, count: int, N: int,
                         K: int) -> tuple[torch.Tensor, torch.Tensor]:
    """`count` [N, K] GGUF weights stored one after another (an expert stack [E, N, K]) ->
    (quant, meta) with each weight repacked on its own, weight e at e * (quant bytes - 4) and
    e * meta bytes: the layout of snowllm_moe_kquant_shuffle_gate_up / _down, which the MoE
    kernels read (Q6_K's per-matrix tail of fp16 scales makes it differ from one repack of
    the [count * N, K] matrix)."""
    quant_bytes, meta_bytes, gguf_bytes = kquant_bytes(fmt, N, K)
    if quant_bytes < 0 or meta_bytes < 0 or count <= 0:
        raise SnowLLMError(f"kquant_shuffle_stack: format {fmt}, {count} x [{N}, {K}] is not "
                           f"supported")
    _chk(b_gguf, "b_gguf", torch.uint8)
    if b_gguf.numel() != count * gguf_bytes:
        raise SnowLLMError(f"kquant_shuffle_stack: expected {count * gguf_bytes} bytes, got "
                           f"{b_gguf.numel()}")
    if fmt != 6:
        # no per-matrix tail: the stack repacks as one matrix, to the same bytes
        return gemm_kquant_shuffle_b(fmt, b_gguf, count * N, K)
    qs = quant_bytes - 4   # the 4 slack bytes behind each weight are read, never written
    quant, meta = empty_bytes(count * qs + 4), empty_bytes(count * meta_bytes)
    for e in range(count):
        check(lib.snowllm_gemm_kquant_shuffle_b(fmt, _p(b_gguf) + e * gguf_bytes,
                                                _p(quant) + e * qs, _p(meta) + e * meta_bytes,
                                                N, K, _stream()), "kquant_shuffle_stack")
    return quant, meta


def gemm_kquant_a_ws_bytes(M: int, K: int) -> int:
    return int(lib.snowllm_gemm_kquant_a_ws_bytes(int(M), int(K)))


def gemm_kquant_a(fmt: int, a: torch.Tensor, quant: torch.Tensor, meta: torch.Tensor,
                  c: torch.Tensor, M: int, N: int, K: int, ws: torch.Tensor) -> None:
    """C[M, N] = A[M, K] @ W[N, K]^T with W dequantised on the fly (fp32 accumulate)."""
    _chk(a, "a", torch.bfloat16, M, K)
    _chk(ws, "ws", torch.uint8, gemm_kquant_a_ws_bytes(M, K))
    bf16 = c.dtype is torch.bfloat16
    _chk(c, "c", torch.bfloat16 if bf16 else torch.float32, M, N)
    check(lib.snowllm_gemm_kquant_a(fmt, _p(a), _p(quant), _p(meta), _p(c), M, N, K, bf16, _p(ws),
                                    _stream()), "gemm_kquant_a")


def gemm_kquant_prepare_a(a: torch.Tensor, ws: torch.Tensor) -> None:
    """Convert activations into the operand workspace once (extension; no reference
    counterpart): lets several weights sharing one input skip the conversion."""
    M, K = a.shape
    _chk(a, "a", torch.bfloat16, M, K)
    _chk(ws, "ws", torch.uint8, gemm_kquant_a_ws_bytes(M, K))
    check(lib.snowverify_gemm_kquant_prepare_a(_p(a), M, K, _p(ws), _stream()), "gemm_kquant_prepare_a")


def gemm_kquant_a_prepared(fmt: int, quant: torch.Tensor, meta: torch.Tensor, c: torch.Tensor,
                           M: int, N: int, K: int, ws: torch.Tensor, col: int = None) -> None:
    """gemm_kquant_a on a workspace filled by gemm_kquant_prepare_a (extension). col: write
    columns [col, col + N) of a wider c [M, ldc] (snowverify_gemm_kquant_a_prepared_ld)."""
    _chk(ws, "ws", torch.uint8, gemm_kquant_a_ws_bytes(M, K))
    bf16 = c.dtype is torch.bfloat16
    if col is None:
        _chk(c, "c", torch.bfloat16 if bf16 else torch.float32, M, N)
        check(lib.snowverify_gemm_kquant_a_prepared(fmt, _p(quant), _p(meta), _p(c), M, N, K, bf16,
                                                 _p(ws), _stream()), "gemm_kquant_a_prepared")
        return
    ldc = c.shape[-1] if c.dim() == 2 else -1
    _chk(c, "c", torch.bfloat16 if bf16 else torch.float32, M, ldc)
    if col < 0 or col + N > ldc:
        raise SnowLLMError(f"gemm_kquant_a_prepared: columns [{col}, {col + N}) outside c's {ldc}")
    check(lib.snowverify_gemm_kquant_a_prepared_ld(fmt, _p(quant), _p(meta),
                                                   _p(c) + col * c.element_size(), ldc, M, N, K,
                                                   bf16, _p(ws), _stream()),
          "gemm_kquant_a_prepared")


GEMM_NOALLOC_MAX_M, GEMM_NOALLOC_MAX_K = 64, 16384


def gemm_kquant_a_noalloc(fmt: int, a: torch.Tensor, quant: torch.Tensor, meta: torch.Tensor,
                          c: torch.Tensor, M: int, N: int, K: int) -> None:
    """gemm_kquant_a without a workspace and without any allocation (extension, for callers
    that cannot allocate): M <= 64, K <= 16384; the library's per-GPU operand array is shared,
    so calls that overlap on one GPU race."""
    if M > GEMM_NOALLOC_MAX_M or K > GEMM_NOALLOC_MAX_K:
        raise SnowLLMError(f"gemm_kquant_a_noalloc: M={M}, K={K} exceed its workspace "
                           f"(M <= {GEMM_NOALLOC_MAX_M}, K <= {GEMM_NOALLOC_MAX_K})")
    _chk(a, "a", torch.bfloat16, M, K)
    bf16 = c.dtype is torch.bfloat16
    _chk(c, "c", torch.bfloat16 if bf16 else torch.float32, M, N)
    check(lib.snowverify_gemm_kquant_a_noalloc(fmt, _p(a), _p(quant), _p(meta), _p(c), M, N, K,
                                               bf16, _stream()), "gemm_kquant_a_noalloc")
