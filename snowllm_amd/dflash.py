# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/dflash.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""DFlash 2 selector and acceptance (snowllm/ops/dflash.py:159-219): the candidate walk that
proposes a draft path, and rejection sampling of a draft prefix."""
import ctypes
import enum

import torch

from ._capi import check, lib
from ._common import _chk, _p, _stream
from .errors import SnowLLMError

# The DFlash 2 draft geometry's selector (tests/test_dflash_sampling.py:24): codebook rank and
# candidates per position. Ranks 64, 128 and 512 use the extension entry.
SELECTOR_RANK = 256
SELECTOR_TOP_K = 16


def select_scratch_bytes(n: int) -> int:
    """Scratch of select_path for n = b * ell logit rows (snowllm/ops/dflash.py:159-161)."""
    return lib.snowllm_draft_select_scratch_bytes(int(n))


def select_path(hp: torch.Tensor, logits: torch.Tensor, pred_cb: torch.Tensor,
                succ_cb: torch.Tensor, anchor: torch.Tensor, path: torch.Tensor,
                scratch: torch.Tensor, *, temperature=None, uniform=None, slots=None,
                candidate_ids=None, probabilities=None) -> None:
    """The candidate walk that replaces argmax on a DFlash 2 draft's logits
    (snowllm/ops/dflash.py:164-198): without temperature a greedy walk writing path only;
    with it, per-row greedy or sampling walks that also store the 16 candidates and their
    probabilities at each request's stable slot."""
    b, ell = path.shape
    n, v = logits.shape
    if n != b * ell:
        raise SnowLLMError(f"the selector was given {n} logit rows for {b}x{ell} positions")
    rank = hp.shape[1] if hp.dim() == 2 else -1
    _chk(hp, "hp", torch.bfloat16, n, rank)
    _chk(logits, "logits", torch.float32, n, v)
    _chk(pred_cb, "pred_cb", torch.bfloat16, v, rank)
    _chk(succ_cb, "succ_cb", torch.bfloat16, v, rank)
    _chk(anchor, "anchor", torch.int64, b)
    _chk(path, "path", torch.int64, b, ell)
    _chk(scratch, "scratch", torch.uint8)
    if scratch.numel() < select_scratch_bytes(n):
        raise SnowLLMError("selector scratch is too small")
    if temperature is None:
        if rank == SELECTOR_RANK:
            check(lib.snowllm_draft_select(_p(hp), _p(logits), _p(pred_cb), _p(succ_cb),
                                           _p(anchor), _p(path), _p(scratch), b, ell, v,
                                           _stream()), "draft_select")
        else:
            check(lib.snowverify_draft_select(_p(hp), _p(logits), _p(pred_cb), _p(succ_cb),
                                              _p(anchor), None, None, None, _p(path), None, None,
                                              _p(scratch), b, ell, v, rank, _stream()),
                  "draft_select")
        return
    _chk(temperature, "temperature", torch.float32, b)
    _chk(uniform, "uniform", torch.float32, b, ell)
    _chk(slots, "slots", torch.int32, b)
    _chk(candidate_ids, "candidate_ids", torch.int64)
    _chk(probabilities, "probabilities", torch.float32, *candidate_ids.shape)
    if tuple(candidate_ids.shape[1:]) != (ell, SELECTOR_TOP_K):
        raise SnowLLMError("selector probability pool has the wrong block or candidate count")
    if rank == SELECTOR_RANK:
        check(lib.snowllm_draft_sample(
            _p(hp), _p(logits), _p(pred_cb), _p(succ_cb), _p(anchor), _p(temperature),
            _p(uniform), _p(slots), _p(path), _p(candidate_ids), _p(probabilities), _p(scratch),
            b, ell, v, SELECTOR_TOP_K, _stream()), "draft_sample")
    else:
        check(lib.snowverify_draft_select(
            _p(hp), _p(logits), _p(pred_cb), _p(succ_cb), _p(anchor), _p(temperature),
            _p(uniform), _p(slots), _p(path), _p(candidate_ids), _p(probabilities), _p(scratch),
            b, ell, v, rank, _stream()), "draft_sample")


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


def accept_reject(logits, drafts, candidate_ids, q, slots, valid, uniform, out, accepted, *,
                  temperature=None):
    """Extension: rejection-sampling acceptance straight from the target logits [b*(k+1), V]
    (three launches, no dense probabilities), for requests whose candidate lists are the whole vocabulary (top-k >= V,
    top-p 1): the same results, bit for bit, as probabilities + reject on those rows.
    temperature [b*(k+1)] or None (1). Returns False when the shape is beyond the fused
    kernel's limits (nothing launched); the caller then takes probabilities + reject."""
    b, length = drafts.shape
    width = length + 1
    rows, V = logits.shape
    _chk(logits, "logits", torch.float32, b * width, V)
    if temperature is not None:
        _chk(temperature, "temperature", torch.float32, b * width)
    _chk(drafts, "drafts", torch.int64, b, length)
    _chk(candidate_ids, "candidate_ids", torch.int64, q.shape[0], length, q.shape[2])
    _chk(q, "draft probabilities", torch.float32, *candidate_ids.shape)
    _chk(slots, "request slots", torch.int32, b)
    _chk(valid, "valid proposals", torch.int32, b)
    _chk(uniform, "uniform", torch.float32, b, width)
    _chk(out, "verified tokens", torch.int64, b, width)
    _chk(accepted, "accepted", torch.int64, b)
    rc = lib.snowverify_accept_reject(_p(logits), _p(temperature), _p(drafts), _p(candidate_ids),
                                      _p(q), _p(slots), _p(valid), _p(uniform), _p(out),
                                      _p(accepted), b, width, V, q.shape[2], _stream())
    if rc == NOT_SUPPORTED:
        return False
    check(rc, "accept_reject")
    return True


def accept_greedy(logits, drafts, tokens, accepted):
    """Extension: tokens [b, k+1] = argmax of each logit row, accepted [b] = 1 + leading
    matches with drafts [b, k], in one launch. Returns False beyond the fused kernel's
    limits (nothing launched)."""
    b, length = drafts.shape
    width = length + 1
    rows, V = logits.shape
    _chk(logits, "logits", torch.float32, b * width, V)
    _chk(drafts, "drafts", torch.int64, b, length)
    _chk(tokens, "tokens", torch.int64, b, width)
    _chk(accepted, "accepted", torch.int64, b)
    rc = lib.snowverify_accept_greedy(_p(logits), _p(drafts), _p(tokens), _p(accepted), b, width,
                                      V, _stream())
    if rc == NOT_SUPPORTED:
        return False
    check(rc, "accept_greedy")
    return True


NOT_SUPPORTED = 801  # hipErrorNotSupported


# ---- draft shape and the selector's hidden projection (snowllm/ops/dflash.py:21-135) -------
class Proj(enum.IntEnum):
    """Projection ids of the DFlash draft (snowllm/ops/dflash.py:21-29); this build computes
    SELECTOR_HIDDEN."""
    FC = 0
    CTX_KV = 1
    QKV = 2
    O = 3  # noqa: E741
    GATE_UP = 4
    DOWN = 5
    CONV = 6
    SELECTOR_HIDDEN = 7


DRAFT_SHAPE_FIELDS = ("hidden", "num_layers", "num_heads", "num_kv_heads", "head_size",
                      "intermediate", "num_taps")


class DraftShape(ctypes.Structure):   # snowllm/_capi.py:67-72
    _fields_ = [(n, ctypes.c_int64) for n in DRAFT_SHAPE_FIELDS]


_selected = None


def select(geo) -> None:
    """Install the draft's shape (any object with the DraftShape fields)."""
    global _selected
    shape = DraftShape(*(int(getattr(geo, n, 0) or 0) for n in DRAFT_SHAPE_FIELDS))
    if lib.snowllm_select_draft(ctypes.byref(shape)) != 0:
        raise SnowLLMError(f"draft shape not supported (hidden {shape.hidden} must be a positive "
                           f"multiple of 256)")
    _selected = geo


def selected():
    if _selected is None:
        raise SnowLLMError("no DFlash draft is selected; call select(geometry) first")
    return _selected


def proj_shape(which: Proj) -> tuple:
    nk = (ctypes.c_int64 * 2)()
    check(lib.snowllm_draft_projection_shape(int(which), nk), "draft_projection_shape")
    return tuple(nk)


def proj_plan(which: Proj, w, m: int) -> tuple:
    from .inference import _weight
    plan = (ctypes.c_int64 * 3)()
    weight = _weight(w)
    check(lib.snowllm_draft_projection_plan(int(which), ctypes.byref(weight), int(m), plan),
          "draft_projection_plan")
    return tuple(plan)


def proj_workspace_bytes(which: Proj, w, m: int) -> int:
    return proj_plan(which, w, m)[2]


def projections_workspace_bytes(m: int) -> int:
    return int(lib.snowllm_draft_projections_workspace_bytes(int(m)))


def proj_shuffle_w(which: Proj, w: torch.Tensor) -> torch.Tensor:
    n, k = proj_shape(which)
    _chk(w, f"draft {which.name} w", torch.bfloat16, n, k)
    buf = torch.empty(lib.snowllm_shuffle_bytes(w.numel() * w.element_size()), dtype=torch.uint8,
                      device="cuda")
    check(lib.snowllm_draft_proj_shuffle_w(int(which), _p(w), _p(buf), _stream()),
          "draft_proj_shuffle_w")
    return buf


def proj_shuffle_w_kquant(which: Proj, blocks: torch.Tensor, fmt: int):
    from .inference import KQuantProjWeight
    n, k = proj_shape(which)
    _chk(blocks, f"draft {which.name} blocks", torch.uint8)
    want = lib.snowllm_kquant_gguf_bytes(fmt, n, k)
    if blocks.numel() != want:
        raise SnowLLMError(f"draft {which.name}: expected {want} bytes of GGUF blocks for a "
                           f"[{n}, {k}] weight at format {fmt}, got {blocks.numel()}")
    quant = torch.empty(lib.snowllm_kquant_quant_bytes(fmt, n, k), dtype=torch.uint8, device="cuda")
    meta = torch.empty(lib.snowllm_kquant_meta_bytes(fmt, n, k), dtype=torch.uint8, device="cuda")
    check(lib.snowllm_draft_proj_shuffle_w_kquant(int(which), fmt, _p(blocks), _p(quant),
                                                  _p(meta), _stream()),
          "draft_proj_shuffle_w_kquant")
    return KQuantProjWeight(quant, meta, fmt)


def proj(which: Proj, a: torch.Tensor, w_shuffled, a_scratch, out: torch.Tensor) -> None:
    """out [m, n] bf16 = a [m, k] W^T for a repacked bf16 or k-quant draft weight."""
    from .inference import _weight
    m = a.shape[0]
    weight = _weight(w_shuffled)
    n, k, need = proj_plan(which, w_shuffled, m)
    _chk(a, "a", torch.bfloat16, m, k)
    _chk(out, "out", torch.bfloat16, m, n)
    capacity = 0 if a_scratch is None else a_scratch.nbytes
    if capacity < need:
        raise SnowLLMError(f"draft projection needs {need} scratch bytes, got {capacity}")
    check(lib.snowllm_draft_projection(int(which), ctypes.byref(weight), _p(a), _p(out),
                                       _p(a_scratch), capacity, m, _stream()), "draft_projection")
