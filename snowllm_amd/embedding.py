# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/embedding.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Embedding gather and LM head operators with the reference's names and arguments
(snowllm/ops/embedding.py:12-73): a bf16 or Q4_K embedding table, a bf16 or k-quant head.
Shapes come from the active geometry (vocab_size, hidden)."""
import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream
from .geometry import build_geometry
from .inference import KQuantExpertWeight


def lm_head_shuffle_weight(w: torch.Tensor) -> torch.Tensor:
    """bf16 head [vocab, hidden] -> the head GEMV's layout."""
    g = build_geometry()
    _chk(w, "lm_head w", torch.bfloat16, g.vocab_size, g.hidden)
    out = torch.empty(lib.snowllm_shuffle_bytes(w.numel() * w.element_size()), dtype=torch.uint8,
                      device="cuda")
    check(lib.snowllm_lm_head_shuffle_weight(_p(w), _p(out), _stream()), "lm_head_shuffle_weight")
    return out


def gather_embedding(input_ids: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> None:
    M = input_ids.numel()
    _chk(input_ids, "input_ids", torch.int64)
    _chk(weight, "embed weight", torch.bfloat16)
    _chk(out, "out", torch.bfloat16, M, weight.shape[1])
    check(lib.snowllm_gather_embedding(_p(input_ids), _p(weight), _p(out), M, _stream()),
          "gather_embedding")


def gather_embedding_q4_k(input_ids: torch.Tensor, weight: torch.Tensor,
                          out: torch.Tensor) -> None:
    """Rows of a Q4_K table weight [vocab, hidden / 256 * 144] (uint8) -> bf16 out [rows, hidden]."""
    if out.ndim != 2 or weight.ndim != 2:
        raise SnowLLMError("Q4_K embedding: weight and out must be matrices")
    rows, hidden = out.shape
    if hidden <= 0 or hidden % 256 or weight.shape[0] <= 0:
        raise SnowLLMError(f"Q4_K embedding: hidden {hidden} must be a positive multiple of 256")
    _chk(input_ids, "Q4_K embedding ids", torch.int64, rows)
    _chk(out, "Q4_K embedding output", torch.bfloat16, rows, hidden)
    _chk(weight, "Q4_K embedding weight", torch.uint8, weight.shape[0], hidden // 256 * 144)
    check(lib.snowllm_gather_embedding_q4_k(_p(input_ids), _p(weight), _p(out), rows,
                                            weight.shape[0], hidden, _stream()),
          "gather_embedding_q4_k")


def lm_head_kquant_shuffle_weight(blocks: torch.Tensor, fmt: int) -> KQuantExpertWeight:
    """Q4_K / Q8_0 GGUF blocks of the head [vocab, hidden] -> packed (quant, meta)."""
    want = lib.snowllm_lm_head_kquant_gguf_bytes(fmt)
    if want <= 0:
        raise SnowLLMError(f"lm_head: format {fmt} is not supported for the active geometry")
    _chk(blocks, "lm_head blocks", torch.uint8)
    if blocks.numel() != want:
        raise SnowLLMError(f"lm_head: {blocks.numel()} bytes of blocks, the format wants {want}")
    quant = torch.empty(lib.snowllm_lm_head_kquant_quant_bytes(fmt), dtype=torch.uint8,
                        device="cuda")
    meta = torch.empty(lib.snowllm_lm_head_kquant_meta_bytes(fmt), dtype=torch.uint8,
                       device="cuda")
    check(lib.snowllm_lm_head_kquant_shuffle_weight(fmt, _p(blocks), _p(quant), _p(meta),
                                                    _stream()), "lm_head_kquant_shuffle_weight")
    return KQuantExpertWeight(quant, meta, None, fmt)


def lm_head_kquant(hidden: torch.Tensor, w: KQuantExpertWeight, logits: torch.Tensor,
                   scratch: torch.Tensor) -> None:
    g = build_geometry()
    _chk(hidden, "hidden", torch.bfloat16, hidden.shape[0], g.hidden)
    _chk(logits, "logits", torch.float32, hidden.shape[0], g.vocab_size)
    check(lib.snowllm_lm_head_kquant(w.fmt, _p(hidden), _p(w.p0), _p(w.p1), _p(logits),
                                     hidden.shape[0], _p(scratch), _stream()), "lm_head_kquant")


def lm_head(hidden: torch.Tensor, w: torch.Tensor, logits: torch.Tensor,
            scratch: torch.Tensor = None) -> None:
    g = build_geometry()
    _chk(hidden, "hidden", torch.bfloat16, hidden.shape[0], g.hidden)
    _chk(logits, "logits", torch.float32, hidden.shape[0], g.vocab_size)
    check(lib.snowllm_lm_head(_p(hidden), _p(w), _p(logits), hidden.shape[0], _p(scratch),
                              _stream()), "lm_head")
