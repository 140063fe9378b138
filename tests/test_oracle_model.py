"""Pins of the CPU layer reference (oracle/model.py) by properties the reference's semantics
fix, each chosen so that a plausible slip (a sign, a swapped half, a dropped term, a wrong
mask bit) fails: known answers of the rotate-half RoPE convention, RMSNorm invariants,
attention against the independent dense restatement in oracle/reference.py, routing against
brute force, and the Q4_K repack view used by the layer reference."""
import itertools
import math

import numpy as np
import torch

from oracle import model as RM
from oracle import reference as R


def test_rope_rotate_half_known_answers():
    D, half = 16, 4  # partial rotary: dims [0, 8) rotate in (i, i + 4) pairs, [8, 16) untouched
    theta = math.pi / 2
    cos = torch.tensor([[math.cos(theta)] * half], dtype=torch.float32)
    sin = torch.tensor([[math.sin(theta)] * half], dtype=torch.float32)
    x = torch.zeros(1, 1, D)
    x[0, 0, 0] = 1.0                       # e_0 -> +e_half under rotate_half (x1 -> (-x2, x1))
    out = RM.rope(x, cos, sin, half)
    assert torch.allclose(out[0, 0, half], torch.tensor(1.0), atol=1e-6)
    assert abs(out[0, 0, 0].item()) < 1e-6
    x = torch.zeros(1, 1, D)
    x[0, 0, half] = 1.0                    # e_half -> -e_0
    out = RM.rope(x, cos, sin, half)
    assert torch.allclose(out[0, 0, 0], torch.tensor(-1.0), atol=1e-6)
    x = torch.randn(3, 2, D)
    pos = torch.tensor([0, 5, 17])
    inv = 1.0 / (1e4 ** (torch.arange(half, dtype=torch.float32) / half))
    c, s = RM.rope_tables(pos, inv)
    out = RM.rope(x, c, s, half)
    assert torch.equal(out[0], x[0])                       # position 0 is the identity
    assert torch.equal(out[..., 2 * half:], x[..., 2 * half:])  # pass-through dims
    n_in = x[..., :half] ** 2 + x[..., half:2 * half] ** 2
    n_out = out[..., :half] ** 2 + out[..., half:2 * half] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)  # pairwise rotation


def test_rmsnorm_invariants():
    x = torch.randn(5, 256) * 3
    y = RM.rmsnorm(x, torch.ones(256), 0.0)
    assert torch.allclose(y.square().mean(-1), torch.ones(5), rtol=1e-2)
    assert torch.equal(RM.rmsnorm(4 * x, torch.ones(256), 0.0), y)  # scale invariance (2^k)
    g = torch.linspace(0.5, 1.5, 256)
    assert torch.allclose(RM.rmsnorm(x, g, 0.0), RM.bf(y * g), rtol=1e-2, atol=1e-2)


def test_masked_attention_matches_dense_restatement():
    g = torch.Generator().manual_seed(3)
    T, Hq, Hkv, D, ctx = 5, 8, 2, 32, 40
    q = torch.randn(T, Hq, D, generator=g)
    k = torch.randn(ctx + T, Hkv, D, generator=g)
    v = torch.randn(ctx + T, Hkv, D, generator=g)
    parents = [-1, 0, 1, 0, 3]
    masks = []
    for i, p in enumerate(parents):
        masks.append((1 << i) | (masks[p] if p >= 0 else 0))
    vis = RM.visibility(ctx, masks)
    # the ancestor mask: row 3's parent is row 0, so it must not see rows 1 and 2
    assert vis[3, ctx:].tolist() == [True, False, False, True, False]
    got = RM.masked_attention(q, k, v, vis, D ** -0.5)
    want = R.dense_attention(q, k, v, D ** -0.5, vis)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-5)
    causal = RM.visibility(ctx, [(2 << t) - 1 for t in range(T)])
    assert torch.equal(causal[:, ctx:], torch.ones(T, T, dtype=torch.bool).tril())


def test_route_brute_force():
    g = torch.Generator().manual_seed(5)
    E, K = 6, 2
    logits = torch.randn(4, E + 1, generator=g)
    ids, w, gate = RM.route(logits, E, K)
    for r in range(4):
        p = torch.softmax(logits[r, :E].double(), -1).numpy()
        best = max(itertools.combinations(range(E), K), key=lambda c: sum(p[list(c)]))
        assert sorted(ids[r].tolist()) == sorted(best)
        assert np.isclose(w[r].sum().item(), 1.0, atol=1e-6)
        assert np.allclose(w[r].double().numpy(), p[ids[r].numpy()] / p[list(best)].sum(), rtol=1e-5)
        assert np.isclose(gate[r].item(), 1 / (1 + math.exp(-logits[r, E].item())), rtol=1e-6)
