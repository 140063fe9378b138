# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/sampling.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Sampling operators: argmax, temperature/top-k/top-p probabilities, sampling.

Signatures and argument meanings follow snowllm/ops/sampling.py:28-91.
"""
import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream, empty

SAMPLING_MAX_K = int(lib.snowllm_sampling_max_k())


def sample_workspace_bytes(batch, vocab, width):
    return int(lib.snowllm_sampling_workspace_bytes(batch, vocab, width))


def sample(logits: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor,
           temperature: torch.Tensor, width: int, generator: torch.Generator | None = None,
           uniform: torch.Tensor | None = None, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Per-row top-k/top-p sample: pick = #(u >= cumsum(values)) (ops/sampling.py:34-62)."""
    B, V = logits.shape
    _chk(logits, "logits", torch.float32, B, V)
    _chk(top_k, "top_k", torch.int32, B)
    _chk(top_p, "top_p", torch.float32, B)
    _chk(temperature, "temperature", torch.float32, B)
    width = int(width)
    workspace_bytes = sample_workspace_bytes(B, V, width)
    if workspace is None:
        workspace = empty(workspace_bytes, dtype=torch.uint8)
    _chk(workspace, "sampling workspace", torch.uint8)
    if workspace.nbytes < workspace_bytes:
        raise ValueError(f"sampling needs {workspace_bytes} workspace bytes")
    if out is None:
        out = empty(B, dtype=torch.int64)
    _chk(out, "sample output", torch.int64, B)
    if uniform is None:
        uniform = torch.rand(B, dtype=torch.float32, device="cuda", generator=generator)
    _chk(uniform, "uniform", torch.float32, B)
    if B == 0:
        return out
    check(lib.snowllm_sampling_sample(_p(logits), _p(top_k), _p(top_p), _p(temperature),
          _p(uniform), _p(out), _p(workspace), workspace.nbytes, B, V, width, _stream()),
          "sampling_sample")
    return out


def argmax(logits: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row argmax; NaN counts as -inf and ties go to the first index (ops/sampling.py:65-72)."""
    B, V = logits.shape
    _chk(logits, "logits", torch.float32, B, V)
    tok = empty(B, dtype=torch.int64) if out is None else out
    _chk(tok, "argmax output", torch.int64, B)
    check(lib.snowllm_sampling_argmax(_p(logits), _p(tok), B, V, _stream()), "argmax")
    return tok


def probabilities(logits, top_k, top_p, temperature, width, out, indices, workspace):
    """Temperature softmax, then top-k/top-p candidates (ops/sampling.py:75-91).

    Rows with top_k covering the vocabulary and top_p >= 1 come back in vocabulary order;
    other rows come back sorted by probability (ties to the lower id), padded with (0, -1).
    """
    rows, vocab = logits.shape
    _chk(logits, "logits", torch.float32, rows, vocab)
    _chk(top_k, "top_k", torch.int32, rows)
    _chk(top_p, "top_p", torch.float32, rows)
    _chk(temperature, "temperature", torch.float32, rows)
    _chk(out, "probabilities", torch.float32, rows, width)
    _chk(indices, "indices", torch.int64, rows, width)
    _chk(workspace, "sampling workspace", torch.uint8)
    if workspace.nbytes < sample_workspace_bytes(rows, vocab, width):
        raise SnowLLMError("sampling probability workspace is too small")
    dense = workspace.view(torch.float32)[:rows * vocab].view(rows, vocab)
    check(lib.snowllm_sampling_softmax(_p(logits), _p(dense), rows, vocab, _p(temperature),
                                       _stream()), "sampling_softmax")
    check(lib.snowllm_sampling_topk_topp(_p(dense), _p(out), _p(indices), rows, vocab, width,
                                         _p(top_k), _p(top_p), _stream()), "sampling_topk_topp")


def penalties(logits, ids, counts, presence, frequency, repetition):
    """Repetition / frequency / presence penalties on one logit row for the listed token ids
    and their output counts (ops/sampling.py:94-100)."""
    _chk(logits, "penalty logits", torch.float32, logits.numel())
    _chk(ids, "penalty token IDs", torch.int64, ids.numel())
    _chk(counts, "penalty counts", torch.int32, ids.numel())
    check(lib.snowllm_sampling_penalties(_p(logits), _p(ids), _p(counts), ids.numel(),
                                         logits.numel(), presence, frequency, repetition,
                                         _stream()), "sampling_penalties")
