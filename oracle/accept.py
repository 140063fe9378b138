"""ctypes binding of the C acceptance oracle (accept.c). Test infrastructure only.

Functions take and return numpy arrays. See accept.c for the canonical arithmetic and the
reference lines each function restates.
"""
import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    if not LIB.exists():
        build()
    return ctypes.CDLL(str(LIB))


_lib = _load()
_P = ctypes.c_void_p
_I = ctypes.c_int64
for name, res, args in [
    ("oc_exp", ctypes.c_float, [ctypes.c_float]),
    ("oc_fix", ctypes.c_uint64, [ctypes.c_float]),
    ("oc_unfix", ctypes.c_float, [ctypes.c_uint64]),
    ("oc_scale_floor", ctypes.c_uint64, [ctypes.c_float, ctypes.c_uint64]),
    ("oc_argmax", None, [_P, _P, _I, _I]),
    ("oc_spec_accept", None, [_P, _P, _P, _I, _I, _I, _I]),
    ("oc_softmax", None, [_P, _P, _I, _I, _P]),
    ("oc_topk_topp", ctypes.c_int, [_P, _P, _P, _I, _I, _I, _P, _P]),
    ("oc_pick_rows", None, [_P, _P, _I, _I, _P, _P]),
    ("oc_penalties", None, [_P, _P, _P, _I, _I, ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    ("oc_reject", None, [_P] * 10 + [_I] * 4),
    ("oc_round_bf16", ctypes.c_float, [ctypes.c_float]),
    ("oc_select_dot", ctypes.c_float, [_P, _P, _P, _I, ctypes.c_int]),
    ("oc_select", None, [_P] * 11 + [_I] * 4),
]:
    fn = getattr(_lib, name)
    fn.restype = res
    fn.argtypes = args


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def exp(x: float) -> float:
    return float(_lib.oc_exp(ctypes.c_float(x)))


def exp_array(x) -> np.ndarray:
    x = _c(x, np.float32)
    return np.array([_lib.oc_exp(ctypes.c_float(float(v))) for v in x.ravel()],
                    dtype=np.float32).reshape(x.shape)


def argmax(logits) -> np.ndarray:
    x = _c(logits, np.float32)
    B, V = x.shape
    out = np.empty(B, dtype=np.int64)
    _lib.oc_argmax(_ptr(x), _ptr(out), B, V)
    return out


def spec_accept(tokens, drafts) -> np.ndarray:
    t = _c(tokens, np.int64)
    d = _c(drafts, np.int64)
    b, T = t.shape
    out = np.empty(b, dtype=np.int64)
    _lib.oc_spec_accept(_ptr(t), _ptr(d), _ptr(out), b, T, T, max(T - 1, 1))
    return out


def softmax(logits, temperature=None) -> np.ndarray:
    x = _c(logits, np.float32)
    rows, vocab = x.shape
    out = np.empty_like(x)
    t = None if temperature is None else _c(temperature, np.float32)
    _lib.oc_softmax(_ptr(x), _ptr(out), rows, vocab, _ptr(t))
    return out


def topk_topp(dense, width, top_k=None, top_p=None):
    p = _c(dense, np.float32)
    rows, vocab = p.shape
    values = np.empty((rows, width), dtype=np.float32)
    ids = np.empty((rows, width), dtype=np.int64)
    k = None if top_k is None else _c(top_k, np.int32)
    tp = None if top_p is None else _c(top_p, np.float32)
    unsupported = _lib.oc_topk_topp(_ptr(p), _ptr(values), _ptr(ids), rows, vocab, width,
                                    _ptr(k), _ptr(tp))
    return values, ids, bool(unsupported)


def probabilities(logits, top_k, top_p, temperature, width):
    """softmax + topk_topp, the composition ops.sampling.probabilities performs."""
    return topk_topp(softmax(logits, temperature), width, top_k, top_p)[:2]


def pick_rows(values, ids, uniform) -> np.ndarray:
    v = _c(values, np.float32)
    i = _c(ids, np.int64)
    u = _c(uniform, np.float32)
    rows, width = v.shape
    out = np.empty(rows, dtype=np.int64)
    _lib.oc_pick_rows(_ptr(v), _ptr(i), rows, width, _ptr(u), _ptr(out))
    return out


def sample(logits, top_k, top_p, temperature, uniform, width) -> np.ndarray:
    values, ids = probabilities(logits, top_k, top_p, temperature, width)
    return pick_rows(values, ids, uniform)


def reject(p, ids, drafts, cand, q, slots, valid, uniform):
    p = _c(p, np.float32)
    ids = _c(ids, np.int64)
    drafts = _c(drafts, np.int64)
    cand = _c(cand, np.int64)
    q = _c(q, np.float32)
    slots = _c(slots, np.int32)
    valid = _c(valid, np.int32)
    uniform = _c(uniform, np.float32)
    b, length = drafts.shape
    width = length + 1
    p_width = p.shape[-1]
    q_width = q.shape[-1]
    out = np.empty((b, width), dtype=np.int64)
    acc = np.empty(b, dtype=np.int64)
    _lib.oc_reject(_ptr(p), _ptr(ids), _ptr(drafts), _ptr(cand), _ptr(q), _ptr(slots),
                   _ptr(valid), _ptr(uniform), _ptr(out), _ptr(acc), b, width, p_width, q_width)
    return out, acc


def _bf16_bits(a) -> np.ndarray:
    """bf16 data as uint16 words (accepts a torch bf16 tensor or uint16 words)."""
    if hasattr(a, "view") and str(getattr(a, "dtype", "")) == "torch.bfloat16":
        import torch
        return a.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    return _c(a, np.uint16)


def round_bf16(x: float) -> float:
    return float(_lib.oc_round_bf16(ctypes.c_float(x)))


def select_dot(pred_row, hp_row, succ_row, sampling: bool) -> float:
    p, h, s = _bf16_bits(pred_row), _bf16_bits(hp_row), _bf16_bits(succ_row)
    return float(_lib.oc_select_dot(_ptr(p), _ptr(h), _ptr(s), p.shape[-1], int(sampling)))


def select(hp, logits, pred, succ, anchor, temperature=None, uniform=None, slots=None,
           n_slots=None):
    """The DFlash 2 candidate walk (accept.c: oc_select). Returns path [b, ell] and, when a
    temperature is given, candidate ids and probabilities [n_slots, ell, 16] (zero-filled
    outside the written slots)."""
    h = _bf16_bits(hp)
    x = _c(logits, np.float32)
    pr, sc = _bf16_bits(pred), _bf16_bits(succ)
    a = _c(anchor, np.int64)
    b = a.shape[0]
    n, V = x.shape
    ell = n // b
    R = h.shape[-1]
    path = np.empty((b, ell), dtype=np.int64)
    t = u = s = cand = q = None
    if temperature is not None:
        t = _c(temperature, np.float32)
        u = _c(uniform, np.float32)
        s = _c(slots, np.int32)
        S = int(n_slots if n_slots is not None else s.max() + 1)
        cand = np.zeros((S, ell, 16), dtype=np.int64)
        q = np.zeros((S, ell, 16), dtype=np.float32)
    _lib.oc_select(_ptr(h), _ptr(x), _ptr(pr), _ptr(sc), _ptr(a), _ptr(t), _ptr(u), _ptr(s),
                   _ptr(path), _ptr(cand), _ptr(q), b, ell, V, R)
    return path, cand, q


def penalties(logits, ids, counts, presence, frequency, repetition):
    """accept.c: oc_penalties on a copy of one logit row."""
    x = _c(logits, np.float32).copy()
    i = _c(ids, np.int64)
    c = _c(counts, np.int32)
    _lib.oc_penalties(_ptr(x), _ptr(i), _ptr(c), i.shape[0], x.shape[0], presence, frequency,
                      repetition)
    return x
