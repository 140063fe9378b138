"""Pins of the DSpark Markov oracle (oracle/dspark.py) on the CPU: the PyTorch procedure of the
reference's own test (tests/test_lfm2_dspark_reference.py:143-152) on the same inputs, a
hand-computed case, invariants, and the single rounding fp64 -> bf16 against exact rationals."""
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dspark as D


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _exact_bf16(x: float) -> float:
    """Nearest bf16 (ties to even) of a finite double, by rational arithmetic."""
    if x == 0:
        return 0.0
    q = Fraction(x)
    e = max(abs(q).numerator.bit_length() - abs(q).denominator.bit_length(), -140)
    while Fraction(2) ** e > abs(q):
        e -= 1
    while Fraction(2) ** (e + 1) <= abs(q):
        e += 1
    quantum = Fraction(2) ** max(e - 7, -133)
    return float(round(q / quantum) * quantum)   # round() on a Fraction ties to even


def test_round_f64_to_bf16_single_rounding():
    cases = [1 + 2 ** -8,               # a tie: to even (1.0)
             1 + 3 * 2 ** -8,           # a tie: to even (1 + 2^-6)
             1 + 2 ** -8 + 2 ** -30,    # just above the tie: up; via fp32 it would tie to 1.0
             -(1 + 2 ** -8 + 2 ** -30), 1 - 2 ** -10, 3.0e38, 2.0 ** -130 * 1.3, 0.0]
    got = D.round_f64_to_bf16(np.array(cases))
    assert got[0] == 1.0 and got[1] == 1 + 2 ** -6 and got[2] == 1 + 2 ** -7
    assert got[3] == -(1 + 2 ** -7)
    for x, y in zip(cases, got):
        assert y == _exact_bf16(x), x
    rng = np.random.default_rng(0)
    xs = rng.standard_normal(3000) * np.exp2(rng.integers(-60, 60, 3000))
    got = D.round_f64_to_bf16(xs)
    for x, y in zip(xs.tolist(), got.tolist()):
        assert y == _exact_bf16(x), x
    # values a bf16 holds exactly come back unchanged, and match torch's fp32 -> bf16
    v = torch.randn(1000).bfloat16().float()
    assert np.array_equal(D.round_f64_to_bf16(v.double().numpy()), v.numpy())


def test_hand_computed_case():
    W1 = torch.tensor([[1, 0], [0, 1], [1, 1], [0, 0]], dtype=torch.bfloat16)
    W2 = torch.tensor([[1, 0], [0, 1], [0, 0], [2, 0]], dtype=torch.bfloat16)
    base = np.array([[0, .5, .2, .1], [.3, 0, 0, 0]], np.float32)
    path, _ = D.markov(base, _bits(W1), _bits(W2), np.array([0]), 2)
    # row 0: latent W1[0] = (1, 0), bias = (1, 0, 0, 2) -> (1, .5, .2, 2.1) -> 3
    # row 1: latent W1[3] = 0 -> base row -> 0
    assert path.tolist() == [[3, 0]]
    # an anchor outside the table gives no bias
    path, _ = D.markov(base, _bits(W1), _bits(W2), np.array([7]), 2)
    assert path.tolist() == [[1, 1]]


def _reference_procedure(base, W1, W2, anchor, block, hidden, conf_w, conf_b):
    """tests/test_lfm2_dspark_reference.py:143-152, request by request, in torch on the CPU."""
    paths, confs = [], []
    for r, a in enumerate(anchor.tolist()):
        previous, path, conf = torch.tensor([a]), [], []
        for j in range(block):
            row = r * block + j
            latent = W1[previous]
            bias = F.linear(latent, W2)
            conf.append(F.linear(torch.cat((hidden[row], latent[0])).float(), conf_w.view(1, -1),
                                 conf_b.view(1)).sigmoid())
            previous = (base[row].float() + bias[0].float()).argmax().view(1)
            path.append(int(previous))
        paths.append(path)
        confs.append(torch.cat(conf))
    return np.array(paths), torch.stack(confs).double().numpy()


@pytest.mark.parametrize("V,rank,b,block,seed", [(4096, 256, 1, 8, 0), (1000, 64, 3, 5, 1),
                                                 (2048, 128, 2, 16, 2)])
def test_matches_the_reference_procedure(V, rank, b, block, seed):
    g = torch.Generator().manual_seed(seed)
    # bias of the same spread as the logits, so that the Markov term decides the path
    W1 = (torch.randn(V, rank, generator=g) * .25).bfloat16()
    W2 = (torch.randn(V, rank, generator=g) * .25 * (256 / rank) ** .5).bfloat16()
    base = torch.randn(b * block, V, generator=g)
    anchor = torch.randint(0, V, (b,), generator=g)
    H = 64
    hidden = torch.randn(b * block, H, generator=g).bfloat16()
    conf_w = torch.randn(H + rank, generator=g) * .1
    conf_b = torch.tensor(.3)
    want_path, want_conf = _reference_procedure(base, W1, W2, anchor, block, hidden, conf_w,
                                                conf_b)
    path, conf = D.markov(base.numpy(), _bits(W1), _bits(W2), anchor.numpy(), block,
                          pre_head=_bits(hidden), conf_w=conf_w.numpy(), conf_b=float(conf_b))
    assert np.array_equal(path, want_path)
    assert np.abs(conf - want_conf).max() < 1e-5
    # the Markov term matters here: the path without it (W2 = 0) differs, and so does a walk
    # that keeps the anchor's latent for every row
    flat, _ = D.markov(base.numpy(), _bits(W1), _bits(torch.zeros_like(W2)), anchor.numpy(), block)
    assert not np.array_equal(flat, want_path)
    stuck = np.array([[D.ord_argmax(base[r * block + j].numpy() + D.round_f64_to_bf16(
        D.bf16_bits_to_f32(_bits(W2)).astype(np.float64) @ D.bf16_bits_to_f32(
            _bits(W1[int(anchor[r])])).astype(np.float64))) for j in range(block)]
        for r in range(b)])
    assert not np.array_equal(stuck, want_path)


def test_invariants():
    g = torch.Generator().manual_seed(7)
    V, rank, block = 512, 32, 6
    W1 = torch.randn(V, rank, generator=g).bfloat16()
    base = torch.randn(2 * block, V, generator=g)
    base[3, 100] = float("nan")                 # NaN is never the maximum
    base[4, :] = -1.0
    base[4, [40, 41]] = 5.0                     # a tie goes to the lower index
    zero = torch.zeros(V, rank, dtype=torch.bfloat16)
    path, _ = D.markov(base.numpy(), _bits(W1), _bits(zero), np.array([1, 2]), block)
    want = [[D.ord_argmax(base[r * block + j].numpy()) for j in range(block)] for r in range(2)]
    assert path.tolist() == want
    assert path[0, 4] == 40
    # fp32 bias keeps more of the sum than the bf16 one, and both agree where the sum is a
    # bf16 value already (an integer matrix of small entries)
    Wi = torch.randint(-2, 3, (V, rank), generator=g).bfloat16()   # |sum| <= 128: bf16-exact
    Li = torch.randint(-2, 3, (V, rank), generator=g).bfloat16()
    a, _ = D.markov(base.numpy(), _bits(Li), _bits(Wi), np.array([5, 9]), block)
    b, _ = D.markov(base.numpy(), _bits(Li), _bits(Wi), np.array([5, 9]), block, fp32_bias=True)
    assert np.array_equal(a, b)
