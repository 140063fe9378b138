"""Pins the C acceptance oracle (oracle/accept.c) to mathematics and to the reference's own
torch semantics. CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import reference as R


def ulp_diff(a: float, b: float) -> int:
    ia = np.array([a], dtype=np.float32).view(np.int32)[0]
    ib = np.array([b], dtype=np.float32).view(np.int32)[0]
    return abs(int(ia) - int(ib))


def test_canon_exp_matches_exp_within_two_ulp():
    xs = np.concatenate([np.linspace(-86.0, 0.0, 20001, dtype=np.float32),
                         -np.logspace(-8, 1.9, 2001).astype(np.float32), [0.0, -0.0]])
    worst = 0
    for x in xs:
        want = np.float32(math.exp(float(x)))
        worst = max(worst, ulp_diff(A.exp(float(x)), float(want)))
    assert worst <= 2, worst
    assert A.exp(-86.5) == 0.0 and A.exp(float("-inf")) == 0.0 and A.exp(float("nan")) == 0.0


def test_fixed_point_helpers():
    assert A._lib.oc_fix(1.0) == 1 << 44
    assert A._lib.oc_fix(0.0) == 0 and A._lib.oc_fix(-1.0) == 0
    assert A._lib.oc_fix(2.0 ** -45) == 0
    assert A._lib.oc_unfix(1 << 44) == 1.0
    # round-to-nearest-even on the 24-bit boundary: 2^24 + 1 -> 2^24, 2^24 + 3 -> 2^24 + 4
    assert A._lib.oc_unfix((1 << 24) + 1) == np.float32(2.0 ** 24) * np.float32(2.0 ** -44)
    assert A._lib.oc_unfix((1 << 24) + 3) == np.float32(2.0 ** 24 + 4) * np.float32(2.0 ** -44)
    # floor(u * R) exactly: u = 0.5 -> R // 2; u = 0.75, R = 2^62 + 3
    assert A._lib.oc_scale_floor(0.5, 1001) == 500
    assert A._lib.oc_scale_floor(0.75, (1 << 62) + 3) == ((1 << 62) + 3) * 3 // 4
    assert A._lib.oc_scale_floor(0.0, 12345) == 0


@pytest.mark.parametrize("rows,vocab", [(3, 67), (9, 1027), (2, 151936)])
def test_softmax_matches_float64_softmax(rows, vocab):
    g = torch.Generator().manual_seed(rows * vocab)
    x = torch.randn(rows, vocab, generator=g) * 2.0
    t = torch.tensor([1.0, 0.65, 1.3][:rows] + [1.0] * max(0, rows - 3))
    got = A.softmax(x.numpy(), t.numpy())
    want = (x.double() / t.double()[:, None]).softmax(-1).numpy()
    assert np.abs(got - want).max() <= 2e-6 * want.max()
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=1e-5)


def test_argmax_reference_patterns():
    # tests/test_sampling_argmax.py:19-30 patterns
    for rows, vocab in [(1, 248320), (3, 1027), (3, 31), (0, 248320)]:
        g = torch.Generator().manual_seed(1743 + rows)
        logits = torch.randn(rows, vocab, generator=g)
        for pattern in ("random", "ties", "nan", "negative-inf"):
            if pattern == "ties":
                logits.fill_(-1)
                logits[:, [min(vocab - 1, 31), min(vocab - 1, 1024), vocab - 1]] = 5
            elif pattern == "nan":
                logits.fill_(float("nan"))
                if rows:
                    logits[0, vocab - 1] = 7
            elif pattern == "negative-inf":
                logits.fill_(float("-inf"))
            want = logits.nan_to_num(nan=float("-inf"), posinf=float("inf"),
                                     neginf=float("-inf")).argmax(-1)
            got = A.argmax(logits.numpy())
            assert np.array_equal(got, want.numpy()), pattern


def test_spec_accept_brute_force():
    T = 9
    for pattern in range(1 << (T - 1)):
        drafts = np.arange(1, T, dtype=np.int64)[None]
        tokens = np.zeros((1, T), dtype=np.int64)
        tokens[0, :T - 1] = np.where([(pattern >> j) & 1 for j in range(T - 1)], drafts[0], -5)
        lead = 0
        while lead < T - 1 and (pattern >> lead) & 1:
            lead += 1
        assert A.spec_accept(tokens, drafts)[0] == 1 + lead


def _rejection_case(width, length, seed):
    # the reference's own rejection test inputs (tests/test_dflash_sampling.py:122-143)
    g = torch.Generator().manual_seed(seed)
    batch, candidates = 37, 7
    vocab = max(width, candidates) + 5
    p_ids = torch.stack([torch.randperm(vocab, generator=g)[:width] for _ in range(batch * (length + 1))])
    p = torch.randn(batch * (length + 1), width, generator=g).softmax(-1)
    q_ids = torch.stack([torch.randperm(vocab, generator=g)[:candidates] for _ in range(batch * length)])
    q_ids = q_ids.view(batch, length, candidates)
    q = torch.randn(batch, length, candidates, generator=g).softmax(-1)
    slots = torch.randperm(batch, generator=g)
    drafts = q_ids[slots, :, 0].clone()
    valid = (torch.arange(batch) % 3 != 0).int()
    uniform = torch.rand(batch, length + 1, generator=g)
    uniform[::4, :-1] = 0
    return p, p_ids, drafts, q_ids, q, slots, valid, uniform


@pytest.mark.parametrize("width,length", [(4, 3), (20, 3), (1024, 3), (20, 7)])
def test_reject_matches_reference_reject(width, length):
    p, p_ids, drafts, q_ids, q, slots, valid, uniform = _rejection_case(width, length, 73 + width)
    batch = drafts.shape[0]
    want, kept = R.reference_reject(p.view(batch, length + 1, width),
                                    p_ids.view(batch, length + 1, width), drafts, q_ids, q,
                                    slots, valid, uniform)
    got, acc = A.reject(p.numpy(), p_ids.numpy(), drafts.numpy(), q_ids.numpy(), q.numpy(),
                        slots.int().numpy(), valid.numpy(), uniform.numpy())
    assert np.array_equal(acc, kept.numpy())
    assert np.array_equal(got, want.numpy())


def test_reject_distribution_invariants():
    # tests/test_dflash_sampling.py:146-167: first emitted token ~ p; acceptance = sum min(p,q)
    batch, width = 40000, 4
    target = np.array([.1, .2, .3, .4], dtype=np.float32)
    draft = np.array([.45, .35, .2, 0.], dtype=np.float32)
    g = torch.Generator().manual_seed(5)
    p = np.tile(target, (batch * 2, 1))
    ids = np.tile(np.arange(width), (batch * 2, 1))
    q = np.tile(draft, (batch, 1, 1))
    q_ids = np.tile(np.arange(width), (batch, 1, 1))
    tokens = torch.multinomial(torch.from_numpy(draft), batch, replacement=True, generator=g).view(batch, 1).numpy()
    slots = np.arange(batch, dtype=np.int32)
    valid = np.ones(batch, dtype=np.int32)
    uniform = torch.rand(batch, 2, generator=g).numpy()
    out, acc = A.reject(p, ids, tokens, q_ids, q, slots, valid, uniform)
    observed = np.bincount(out[:, 0], minlength=4) / batch
    assert np.abs(observed - target).max() < .01
    assert abs((acc == 2).mean() - np.minimum(target, draft).sum()) < .01


def test_reject_full_vocab_matches_reference_identity():
    # BASELINE config 1 shapes (V = 151936, k = 8) through the identity form of reference_reject
    V, k = 151936, 8
    g = torch.Generator().manual_seed(10)
    target = torch.randn(k + 1, V, generator=g) * 2.0
    draft = torch.randn(k, V, generator=g) * 2.0
    p = torch.from_numpy(A.softmax(target.numpy()))
    q = torch.from_numpy(A.softmax(draft.numpy()))
    drafts = torch.multinomial(q, 1, generator=torch.Generator().manual_seed(0)).view(1, k)
    for trial in range(4):
        uniform = torch.rand(1, k + 1, generator=torch.Generator().manual_seed(1 + trial))
        want, kept = R.reference_reject_identity(p[None], drafts, q[None], uniform)
        ids = np.tile(np.arange(V, dtype=np.int64), (k + 1, 1))
        got, acc = A.reject(p.numpy(), ids, drafts.numpy(), ids[:k][None], q.numpy()[None],
                            np.zeros(1, np.int32), np.ones(1, np.int32), uniform.numpy())
        assert np.array_equal(acc, kept.numpy()) and np.array_equal(got, want.numpy())


def test_probabilities_match_reference_target_probabilities():
    # tests/test_dflash_sampling.py:190-217
    g = torch.Generator().manual_seed(73)
    params = [(0., 1, 1.), (.65, 20, .95), (1.3, 0, .8), (1., 3, .5)]
    logits = torch.randn(4, 67, generator=g)
    temp = torch.tensor([t if t > 0 else 1.0 for t, _, _ in params])
    top_k = torch.tensor([1 if t <= 0 else (k if 0 < k <= 67 else 67) for t, k, _ in params], dtype=torch.int32)
    top_p = torch.tensor([p for _, _, p in params])
    values, ids = A.probabilities(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(), 67)
    actual = torch.zeros(4, 67).scatter_add_(1, torch.from_numpy(ids).clamp_min(0), torch.from_numpy(values))
    expected = R.target_probabilities(logits, torch.tensor([t for t, _, _ in params]), top_k, top_p)
    assert ((actual - expected).norm() / expected.norm()).item() < 1e-5
    uniform = np.array([.17, .37, .67, .87], dtype=np.float32)
    picked = (torch.from_numpy(uniform)[:, None] >= torch.from_numpy(values).cumsum(-1)).sum(-1).clamp_max(66)
    want = torch.from_numpy(ids).gather(1, picked[:, None]).view(-1)
    assert np.array_equal(A.pick_rows(values, ids, uniform), want.numpy())


def test_wide_lists_match_reference_target_probabilities():
    """Lists of any width: top-k beyond 1024 and top-p over the whole vocabulary
    (snowllm/engine/request.py:29-35 gives top_k 0 the whole vocabulary), against the
    reference test's torch semantics (tests/test_dflash_sampling.py:199-209) at V = 151,936:
    the same distribution, the same number of kept tokens, and the kept ids in the order of
    torch's stable descending sort of the probabilities."""
    V = 151936
    g = torch.Generator().manual_seed(5)
    params = [(1., 0, .9), (1., 2000, 1.), (.8, 5000, .7), (1.3, 1500, .95)]
    logits = torch.randn(len(params), V, generator=g) * 2
    temp = torch.tensor([t for t, _, _ in params])
    top_k = torch.tensor([k if 0 < k <= V else V for _, k, _ in params], dtype=torch.int32)
    top_p = torch.tensor([p for _, _, p in params])
    values, ids = A.probabilities(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(), V)
    actual = torch.zeros(len(params), V).scatter_add_(
        1, torch.from_numpy(ids).clamp_min(0), torch.from_numpy(values))
    expected = R.target_probabilities(logits, temp, top_k, top_p)
    for i, (t, k, p) in enumerate(params):
        err = ((actual[i] - expected[i]).norm() / expected[i].norm()).item()
        assert err < 1e-6, (i, err)
        kept = int((expected[i] > 0).sum())
        assert int((torch.from_numpy(values[i]) > 0).sum()) == kept
        order = torch.sort((logits[i] / t).softmax(-1), descending=True, stable=True).indices
        assert np.array_equal(ids[i, :kept], order[:kept].numpy()), i
        width = k if 0 < k <= V else V
        assert (ids[i, width:] == -1).all() and (values[i, kept:] == 0).all()


def test_lists_narrower_than_top_k_are_marked():
    """A row whose top-k does not fit the list width is written as (NaN, -2) and reported."""
    logits = np.random.default_rng(1).standard_normal((2, 300)).astype(np.float32)
    dense = A.softmax(logits)
    values, ids, bad = A.topk_topp(dense, 40, np.array([50, 10], np.int32),
                                   np.array([1., .9], np.float32))
    assert bad and (ids[0] == -2).all() and np.isnan(values[0]).all()
    assert (ids[1, :10] >= 0).all() and (ids[1, 10:] == -1).all()


def test_banned_ngram_tokens_known_answers():
    # the reference's own cases (tests/test_mineru.py:123-128)
    from snowllm_amd.ngram import banned_ngram_tokens
    assert banned_ngram_tokens([1, 2, 3, 1, 2], 3) == [3]
    assert banned_ngram_tokens([1, 2, 3, 1, 4], 3) == []
    assert banned_ngram_tokens([3, 1, 3], 1) == [1, 3]
    assert banned_ngram_tokens([1, 2], 0) == []
    assert banned_ngram_tokens([1, 2], 4) == []
    # brute force over short streams
    rng = np.random.default_rng(2)
    for _ in range(200):
        toks = rng.integers(0, 4, rng.integers(0, 9)).tolist()
        size = int(rng.integers(0, 5))
        want = set()
        if size > 0 and len(toks) >= size - 1:
            tail = toks[len(toks) - (size - 1):] if size > 1 else []
            for i in range(len(toks) - size + 1):
                if toks[i:i + size - 1] == tail:
                    want.add(toks[i + size - 1])
        assert banned_ngram_tokens(toks, size) == sorted(want), (toks, size)


def test_penalties_known_answers():
    # tests/test_runtime_buffers.py:136-143: repetition 2 turns a listed logit of 8 into 4
    x = np.full(16, 8.0, np.float32)
    got = A.penalties(x, np.array([1, 2]), np.array([0, 1], np.int32), 0.0, 0.0, 2.0)
    assert got[1] == 4.0 and got[2] == 4.0 and got[0] == 8.0 and got[3] == 8.0
    # exactly representable cases pin the formula: repetition divides positive and multiplies
    # non-positive logits (prompt ids included, count 0), frequency scales with the count,
    # presence needs a count
    x = np.array([3.0, -3.0, 3.0, -1.0, 5.0, 0.0], np.float32)
    ids = np.array([0, 1, 2, 3, 5, 99])
    counts = np.array([0, 0, 3, 2, 1, 4], np.int32)
    got = A.penalties(x, ids, counts, 0.5, 0.25, 1.5)
    want = np.array([2.0, -4.5, 2.0 - 0.75 - 0.5, -1.5 - 0.5 - 0.5, 5.0, 0.0 - 0.25 - 0.5],
                    np.float32)
    assert np.array_equal(got, want)
    # ids outside the vocabulary are skipped, repetition 1 leaves the sign rule out
    got = A.penalties(np.array([1.0, -2.0], np.float32), np.array([-1, 1, 7]),
                      np.array([5, 2, 1], np.int32), 1.0, 0.5, 1.0)
    assert np.array_equal(got, np.array([1.0, -4.0], np.float32))
