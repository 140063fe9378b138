"""DFlash acceptance: rejection sampling of a draft prefix (snowllm/ops/dflash.py:201-219)."""
import torch

from ._capi import check, lib
from ._common import _chk, _p, _stream


def reject(probabilities, indices, drafts, candidate_ids, q, slots, valid, uniform, out, accepted):
    """Accept drafts while u*q(d) < p(d); then draw the correction from max(p - q, 0).

    probabilities/indices: [b*(k+1), p_width] target candidates; candidate_ids/q:
    [S, k, q_width] draft candidates indexed by the stable request slot; valid=0 means the
    draft proposal is stale (q treated as 1 for acceptance, one-hot for the residual).
    """
    b, length = drafts.shape
    width = length + 1
    p_width, q_width = probabilities.shape[1], q.shape[2]
    _chk(probabilities, "target probabilities", torch.float32, b * width, p_width)
    _chk(indices, "target indices", torch.int64, b * width, p_width)
    _chk(drafts, "drafts", torch.int64, b, length)
    _chk(candidate_ids, "candidate_ids", torch.int64, q.shape[0], length, q_width)
    _chk(q, "draft probabilities", torch.float32, *candidate_ids.shape)
    _chk(slots, "request slots", torch.int32, b)
    _chk(valid, "valid proposals", torch.int32, b)
    _chk(uniform, "uniform", torch.float32, b, width)
    _chk(out, "verified tokens", torch.int64, b, width)
    _chk(accepted, "accepted", torch.int64, b)
    check(lib.snowllm_draft_reject(
        _p(probabilities), _p(indices), _p(drafts), _p(candidate_ids), _p(q), _p(slots),
        _p(valid), _p(uniform), _p(out), _p(accepted), b, width, p_width, q_width, _stream()),
        "draft_reject")
