"""Pins of the selector oracle (oracle/accept.c: oc_select) on the CPU.

The expected values restate the reference's own checks: the torch formula of
tests/test_dflash_sampling.py:44-75 (mixed greedy / sampling walk with codebooks) and the
stable-sort reference of tests/test_dflash_selector_topk.py:42-61 (zero codebooks, ties, NaN).
The two arithmetic pieces the oracle adds -- bf16 rounding and the lane-tree dot product --
are pinned against torch's bf16 conversion and an fp64 sum."""
import numpy as np
import pytest
import torch

from oracle import accept as A

K = 16


def test_round_bf16_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, generator=g) * torch.exp(torch.randn(4096, generator=g) * 8)
    # exact halfway cases in both directions (ties to even)
    halves = torch.tensor([1.00390625, 1.01171875, -1.00390625, 3.0e38, 1e-40, 0.0, -0.0])
    for v in torch.cat([x, halves]).tolist():
        want = torch.tensor([v], dtype=torch.float32).bfloat16().float().item()
        got = A.round_bf16(v)
        assert got == want or (np.isnan(got) and np.isnan(want)), v


@pytest.mark.parametrize("rank", [64, 256, 512])
def test_select_dot_against_fp64(rank):
    g = torch.Generator().manual_seed(rank)
    pred, hp, succ = ((torch.randn(rank, generator=g) * .2).bfloat16() for _ in range(3))
    exact = (pred.double() * hp.double() * succ.double()).sum().item()
    got = A.select_dot(pred, hp, succ, sampling=False)
    # products are exact in binary32; only the 255 additions round
    assert abs(got - exact) <= 1e-6 * (pred.double().abs() * hp.double().abs() * succ.double().abs()).sum().item()
    # the sampling form: bf16(sum(bf16(pred * hp) * succ)), the torch bf16 product path
    prod = pred * hp
    want = (succ.float() * prod.float()).double().sum()
    got_s = A.select_dot(pred, hp, succ, sampling=True)
    assert got_s == A.round_bf16(got_s)
    assert abs(got_s - want.item()) <= 2 ** -7 * abs(want.item()) + 1e-30


def _reference_walk(hidden, logits, pred, succ, anchor, temp, uniform):
    """tests/test_dflash_sampling.py:44-75, check(): the reference's own expected values."""
    batch = anchor.shape[0]
    length = logits.shape[0] // batch
    values, candidates = logits.topk(K, dim=-1)
    expected, probabilities = [], []
    for b in range(batch):
        previous, tokens, qs = anchor[b], [], []
        for j in range(length):
            row = b * length + j
            if temp[b] == 0:
                correction = (pred[previous].float() * hidden[row].float()
                              * succ[candidates[row]].float()).sum(-1)
            else:
                product = pred[previous] * hidden[row]
                correction = (succ[candidates[row]].float() * product.float()).sum(-1).bfloat16().float()
            scores = values[row] + correction
            if temp[b] == 0:
                picked = scores.argmax()
                probs = torch.nn.functional.one_hot(picked, K).float()
            else:
                probs = (scores / temp[b]).softmax(-1)
                picked = (uniform[b, j] >= probs.cumsum(-1)).sum().clamp_max(K - 1)
            previous = candidates[row, picked]
            tokens.append(previous)
            qs.append(probs)
        expected.append(torch.stack(tokens))
        probabilities.append(torch.stack(qs))
    return torch.stack(expected), candidates, torch.stack(probabilities)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_matches_reference_walk(seed):
    torch.manual_seed(seed)
    batch, length, vocab, rank = 3, 7, 67, 256
    hidden = (torch.randn(batch * length, rank) * .2).bfloat16()
    logits = torch.randn(batch * length, vocab)
    pred = (torch.randn(vocab, rank) * .2).bfloat16()
    succ = (torch.randn(vocab, rank) * .2).bfloat16()
    anchor = torch.tensor([5, 21, 51])
    temp = torch.tensor([0., 1., .65])
    uniform = torch.rand(batch, length)
    slots = torch.tensor([4, 0, 2], dtype=torch.int32)
    path, cand, q = A.select(hidden, logits.numpy(), pred, succ, anchor.numpy(), temp.numpy(),
                             uniform.numpy(), slots.numpy(), n_slots=5)
    want_path, want_cand, want_q = _reference_walk(hidden, logits, pred, succ, anchor, temp, uniform)
    assert np.array_equal(path, want_path.numpy())
    s = slots.long().numpy()
    assert np.array_equal(cand[s], want_cand.view(batch, length, K).numpy())
    assert np.allclose(q[s], want_q.numpy(), atol=.003, rtol=0)
    assert not q[1].any() and not q[3].any()  # slots nobody owns stay as they were


@pytest.mark.parametrize("vocab,rows", [(67, 3), (248320, 3), (248320, 17)])
def test_oracle_matches_stable_sort_reference(vocab, rows):
    """tests/test_dflash_selector_topk.py:42-61 with zero codebooks."""
    torch.manual_seed(1743)
    pred = torch.zeros(vocab, 256, dtype=torch.bfloat16)
    hidden = torch.zeros(rows, 256, dtype=torch.bfloat16)
    anchor = np.zeros(1, dtype=np.int64)
    uniform = np.full((1, rows), .371, dtype=np.float32)
    slots = np.array([1], dtype=np.int32)
    logits = torch.empty(rows, vocab)
    for pattern in ["random", "ties", "nan-mix"]:
        logits.normal_()
        if pattern == "ties":
            logits.zero_()
            logits[:, ::2] = -0.
        elif pattern == "nan-mix":
            logits[:, ::257] = float("nan")
        clean = logits.nan_to_num(nan=-float("inf"))
        expected_ids = clean.argsort(dim=-1, descending=True, stable=True)[:, :K]
        expected_values = clean.gather(1, expected_ids)
        for temperature in [0., .7]:
            expected_q = (torch.nn.functional.one_hot(torch.zeros(rows, dtype=torch.int64), K).float()
                          if temperature == 0 else (expected_values / temperature).softmax(-1))
            picked = (torch.full((rows, 1), .371) >= expected_q.cumsum(-1)).sum(-1).clamp_max(K - 1)
            expected_path = expected_ids.gather(1, picked[:, None]).view(1, rows)
            path, cand, q = A.select(hidden, logits.numpy(), pred, pred, anchor,
                                     np.array([temperature], np.float32), uniform, slots, n_slots=3)
            assert np.array_equal(cand[1], expected_ids.numpy()), (pattern, temperature)
            assert np.allclose(q[1], expected_q.numpy(), atol=1e-6, rtol=0)
            assert np.array_equal(path, expected_path.numpy())
