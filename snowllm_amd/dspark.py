# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/dspark.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""The DSpark Markov head operators with the reference's names and arguments
(snowllm/ops/dspark.py:10-16, 53-77)."""
import torch

from ._capi import check, lib
from ._common import _chk, _chk_rows, _p, _stream
from .errors import SnowLLMError

MAX_BATCH = 16


def dspark_pack_weight(raw: torch.Tensor) -> torch.Tensor:
    """bf16 [n, k] -> the Markov head's packed W2, viewed as bf16 [n, k]."""
    n, k = raw.shape
    _chk(raw, "DSpark raw weight", torch.bfloat16, n, k)
    need = lib.snowllm_dspark_weight_bytes(n, k)
    if need <= 0:
        raise SnowLLMError(f"DSpark weight [{n}, {k}]: k must be a positive multiple of 8")
    packed = torch.empty(need, dtype=torch.uint8, device=raw.device).view(torch.bfloat16).view(n, k)
    check(lib.snowllm_dspark_pack_weight(_p(raw), _p(packed), n, k, _stream()), "dspark_pack_weight")
    return packed


def dspark_markov_workspace_bytes(b: int, v: int, rank: int, block: int) -> int:
    return int(lib.snowllm_dspark_markov_workspace_bytes(int(b), int(v), int(rank), int(block)))


def dspark_markov(base, w1, w2, anchor, block, *, pre_head=None, conf_weight=None,
                  conf_bias=None, confidence=None, workspace=None, out=None, fp32_bias=False):
    """The Markov walk over a block of draft rows: out [b, block] i64 (and confidence
    [b, block] f32 when given). base f32 [b * block, >= V] rows, w1 bf16 [V, rank], w2 packed by
    dspark_pack_weight, anchor i64 [b]."""
    b = anchor.numel()
    v, rank = w1.shape
    _chk_rows(base, "DSpark base logits", torch.float32)
    if base.shape[0] != b * block or base.shape[1] < v:
        raise SnowLLMError("DSpark logits and block shapes differ")
    _chk(w1, "DSpark Markov W1", torch.bfloat16, v, rank)
    _chk(w2, "DSpark packed W2", torch.bfloat16, v, rank)
    _chk(anchor, "DSpark anchors", torch.int64, b)
    if b > MAX_BATCH or b * rank > 4096:
        raise SnowLLMError(f"DSpark Markov head: at most {MAX_BATCH} requests per call and "
                           f"requests x rank <= 4096")
    h = ps = 0
    if confidence is not None:
        if pre_head is None or conf_weight is None:
            raise SnowLLMError("DSpark confidence needs pre_head and weights")
        _chk_rows(pre_head, "DSpark pre-head", torch.bfloat16)
        h, ps = pre_head.shape[1], pre_head.stride(0)
        if pre_head.shape[0] != b * block:
            raise SnowLLMError("DSpark pre-head row count differs")
        _chk(conf_weight, "DSpark confidence weights", torch.float32, h + rank)
        if conf_bias is not None:
            _chk(conf_bias, "DSpark confidence bias", torch.float32, conf_bias.numel())
            if conf_bias.numel() != 1:
                raise SnowLLMError("DSpark confidence bias must be scalar")
        _chk(confidence, "DSpark confidence output", torch.float32, b, block)
    need = dspark_markov_workspace_bytes(b, v, rank, block)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=base.device)
    _chk(workspace, "DSpark Markov workspace", torch.uint8)
    if workspace.numel() < need:
        raise SnowLLMError("DSpark Markov workspace too small")
    if out is None:
        out = torch.empty(b, block, dtype=torch.int64, device=base.device)
    _chk(out, "DSpark output", torch.int64, b, block)
    ptrs = [_p(t) for t in (base, w1, w2, anchor, pre_head, conf_weight, conf_bias, out,
                            confidence, workspace)]
    check(lib.snowllm_dspark_markov(*ptrs, b, v, rank, block, base.stride(0), h, ps,
                                    workspace.numel(), int(fp32_bias), _stream()),
          "dspark_markov")
    return out
