# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/metadata.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Greedy prefix acceptance (snowllm/ops/metadata.py:244-251)."""
import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _chk_rows, _p, _stream, empty


def spec_accept(tokens, drafts, *, out=None):
    """accepted[b] = 1 + number of leading j with tokens[b, j] == drafts[b, j]."""
    b, t = tokens.shape
    _chk_rows(tokens, "verified tokens", torch.int64)
    _chk_rows(drafts, "draft tokens", torch.int64)
    if drafts.shape != (b, t - 1):
        raise SnowLLMError("draft and verify token shapes differ")
    if out is None:
        out = empty(b, dtype=torch.int64, device=tokens.device)
    _chk(out, "accepted lengths", torch.int64, b)
    check(lib.snowllm_spec_accept(_p(tokens), _p(drafts), _p(out), b, t, tokens.stride(0),
                                  drafts.stride(0), _stream()), "spec_accept")
    return out
