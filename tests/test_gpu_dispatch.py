"""The acceptance straight from the logits (snowverify_accept_reject / _greedy) and the verify
dispatch (snowllm/engine/dflash_sampling.py:
54-69) against the C oracle, bit-exact: accept lengths, emitted ids (and, for the dispatch,
the branch each batch takes)."""
import numpy as np
import pytest
import torch

from oracle import accept as A

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _selector_lists(S, length, V, g, width=16):
    """Draft candidate lists as the selector writes them: unique ids, probabilities that sum
    to one per row."""
    cand = torch.stack([torch.stack([torch.randperm(V, generator=g)[:width] for _ in range(length)])
                        for _ in range(S)])
    q = torch.rand(S, length, width, generator=g) + 0.05
    q = q / q.sum(-1, keepdim=True)
    return cand.long(), q.float()


def _oracle_reject(logits, temp, drafts, cand, q, slots, valid, uniform):
    p = A.softmax(logits, temp)
    ident = np.tile(np.arange(logits.shape[1]), (logits.shape[0], 1))
    return A.reject(p, ident, drafts, cand, q, slots, valid, uniform)


CASES = [
    # b, width, V, q kind, temperature
    (1, 9, 151936, "selector", 1.0),
    (1, 9, 151936, "vocab", 1.0),
    (3, 5, 4096, "selector", 0.7),
    (2, 9, 248320, "selector", 1.3),
    (2, 1, 20000, "selector", 1.0),
    (4, 3, 67, "selector", 1.0),
]


@pytest.mark.parametrize("b,width,V,qkind,T", CASES)
def test_fused_reject_equals_oracle(gpu, b, width, V, qkind, T):
    from snowllm_amd import ops
    from snowllm_amd.dflash import accept_reject
    length = width - 1
    g = torch.Generator().manual_seed(V + b * 7 + width)
    S = b + 2
    logits = torch.randn(b * width, V, generator=g) * 2
    temp = torch.full((b * width,), T)
    if qkind == "vocab":
        q = torch.softmax(torch.randn(S, max(length, 1), V, generator=g) * 2, -1)[:, :length]
        cand = torch.arange(V).repeat(S, length, 1)
    else:
        cand, q = _selector_lists(S, length, V, g) if length else (
            torch.zeros(S, 0, 16, dtype=torch.int64), torch.zeros(S, 0, 16))
    slots = torch.randperm(S, generator=g)[:b].int()
    valid = torch.tensor([1, 0, 1, 1][:b], dtype=torch.int32)
    for mode in ("sampled", "argmax", "u0", "oob"):
        drafts = torch.randint(0, V, (b, length), generator=g)
        if mode == "argmax" and length:   # target argmax drafts, so prefixes get accepted
            drafts = logits.view(b, width, V)[:, :length].argmax(-1)
        if mode == "oob" and length:      # ids outside the vocabulary are never accepted
            drafts[:, 0] = -1
            drafts[:, -1] = V + 5
        uniform = torch.rand(b, width, generator=g)
        if mode == "u0":
            uniform[:, :length] = 0.0     # u = 0 accepts every draft with p > 0
        _say(f"fused reject b={b} width={width} V={V} q={qkind} T={T} {mode}")
        out = torch.full((b, width), -7, dtype=torch.int64, device="cuda")
        acc = torch.full((b,), -7, dtype=torch.int64, device="cuda")
        args = [x.cuda() for x in (drafts, cand, q.contiguous(), slots, valid, uniform)]
        assert accept_reject(logits.cuda(), *args, out, acc, temperature=temp.cuda())
        torch.cuda.synchronize()
        want_out, want_acc = _oracle_reject(logits.numpy(), temp.numpy(), drafts.numpy(),
                                            cand.numpy(), q.contiguous().numpy(), slots.numpy(),
                                            valid.numpy(), uniform.numpy())
        assert np.array_equal(out.cpu().numpy(), want_out), mode
        assert np.array_equal(acc.cpu().numpy(), want_acc), mode
        # and the multi-launch form on the same inputs
        p = torch.empty(b * width, V, device="cuda")
        ids = torch.empty(b * width, V, dtype=torch.int64, device="cuda")
        ws = torch.empty(ops.sample_workspace_bytes(b * width, V, V), dtype=torch.uint8,
                         device="cuda")
        kmax = torch.full((b * width,), ops.SAMPLING_MAX_K, dtype=torch.int32, device="cuda")
        ops.probabilities(logits.cuda(), kmax, torch.ones(b * width, device="cuda"), temp.cuda(),
                          V, p, ids, ws)
        out2 = torch.empty_like(out)
        acc2 = torch.empty_like(acc)
        ops.dflash.reject(p, ids, *args, out2, acc2)
        torch.cuda.synchronize()
        assert torch.equal(out2, out) and torch.equal(acc2, acc), mode


def test_fused_reject_graph_replays(gpu):
    """The arrival counters advance across captured replays: each replay with new uniforms
    matches the oracle."""
    from snowllm_amd.dflash import accept_reject
    b, width, V = 1, 9, 151936
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(b * width, V, generator=g) * 2).cuda()
    cand, q = _selector_lists(2, width - 1, V, g)
    drafts = logits.view(b, width, V)[:, :width - 1].argmax(-1)
    slots = torch.zeros(b, dtype=torch.int32, device="cuda")
    valid = torch.ones(b, dtype=torch.int32, device="cuda")
    uniform = torch.empty(b, width, device="cuda")
    out = torch.empty(b, width, dtype=torch.int64, device="cuda")
    acc = torch.empty(b, dtype=torch.int64, device="cuda")
    cand, q = cand.cuda(), q.cuda()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        accept_reject(logits, drafts, cand, q, slots, valid, uniform, out, acc)
    for i in range(4):
        _say(f"fused reject graph replay {i}")
        u = torch.rand(b, width, generator=g)
        uniform.copy_(u)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_out, want_acc = _oracle_reject(logits.cpu().numpy(), None, drafts.cpu().numpy(),
                                            cand.cpu().numpy(), q.cpu().numpy(),
                                            slots.cpu().numpy(), valid.cpu().numpy(), u.numpy())
        assert np.array_equal(out.cpu().numpy(), want_out)
        assert np.array_equal(acc.cpu().numpy(), want_acc)


@pytest.mark.parametrize("b,width,V", [(1, 9, 151936), (3, 5, 248320), (5, 1, 4096), (2, 9, 67)])
def test_fused_greedy_equals_oracle(gpu, b, width, V):
    from snowllm_amd.dflash import accept_greedy
    length = width - 1
    g = torch.Generator().manual_seed(V + b)
    for pattern in ("random", "ties", "nan"):
        logits = torch.randn(b * width, V, generator=g)
        if pattern == "ties":
            logits.fill_(-1)
            logits[:, [min(V - 1, 31), min(V - 1, 20000), V - 1]] = 5
        elif pattern == "nan":
            logits[:, ::3] = float("nan")
        top = torch.from_numpy(A.argmax(logits.numpy())).view(b, width)
        drafts = top[:, :length].clone()
        if length:
            drafts[0, length // 2] += 1   # a mismatch in the middle for the first request
        _say(f"fused greedy b={b} width={width} V={V} {pattern}")
        tokens = torch.full((b, width), -7, dtype=torch.int64, device="cuda")
        acc = torch.full((b,), -7, dtype=torch.int64, device="cuda")
        assert accept_greedy(logits.cuda(), drafts.cuda(), tokens, acc)
        torch.cuda.synchronize()
        assert torch.equal(tokens.cpu(), top)
        assert np.array_equal(acc.cpu().numpy(), A.spec_accept(top.numpy(), drafts.numpy()))


def test_verify_dispatch_branches_bit_exact(gpu):
    """snowllm/engine/dflash_sampling.py:54-69 on three batches: all greedy, all sampling over
    the whole vocabulary, and a mixed batch (greedy, whole vocabulary, top-k/top-p) with one
    stale proposal -- each against the oracle."""
    from snowllm_amd.dflash_sampling import DFlashAcceptance, SamplingParams, VerifyRequest
    V, width = 4096, 9
    length = width - 1
    acc = DFlashAcceptance(max_seqs=4, block=width, vocab=V, seed=5)
    g = torch.Generator().manual_seed(11)
    cand, q = _selector_lists(4, length, V, g)
    acc.candidates.copy_(cand)
    acc.q.copy_(q)
    batches = {
        "greedy": [SamplingParams(0.0), SamplingParams(-1.0)],
        "fused": [SamplingParams(1.0), SamplingParams(0.8, top_k=0), SamplingParams(1.2)],
        "lists": [SamplingParams(0.0), SamplingParams(1.0), SamplingParams(0.7, top_k=50, top_p=0.9)],
    }
    for want_path, params in batches.items():
        count = len(params)
        logits = torch.randn(count * width, V, generator=g) * 2
        top = torch.from_numpy(A.argmax(logits.numpy())).view(count, width)
        drafts = top[:, :length].clone()
        drafts[:, 3] = torch.randint(0, V, (count,), generator=g)
        batch = [VerifyRequest(slot=s, params=p, drafts=tuple(drafts[i].tolist()))
                 for i, (s, p) in enumerate(zip([2, 0, 3], params))]
        acc.remember(batch, [r.drafts for r in batch])
        if count > 1:   # a stale proposal: the slot remembers other drafts
            acc.proposals[batch[1].slot] = tuple(range(length))
        _say(f"dispatch {want_path}: {count} requests")
        tokens, accepted = acc.verify(logits.cuda(), batch, drafts.cuda())
        torch.cuda.synchronize()
        assert acc.path == want_path
        if want_path == "greedy":
            assert torch.equal(tokens.cpu(), top)
            assert np.array_equal(accepted.cpu().numpy(), A.spec_accept(top.numpy(), drafts.numpy()))
            continue
        rows = [r for r in batch for _ in range(width)]
        ks = np.array([r.params.kernel_top_k() for r in rows], np.int32)
        tp = np.array([r.params.top_p for r in rows], np.float32)
        tt = np.array([r.params.kernel_temperature() for r in rows], np.float32)
        wp = min(int(ks.max()), V)
        p, ids = A.probabilities(logits.numpy(), ks, tp, tt, wp)
        valid = np.array([int(r.drafts == acc.proposals[r.slot]) for r in batch], np.int32)
        slots = np.array([r.slot for r in batch], np.int32)
        u = acc.verify_uniform[:count * width].view(count, width).cpu().numpy()
        want_out, want_acc = A.reject(p, ids, drafts.numpy(), cand.numpy(), q.numpy(), slots,
                                      valid, u)
        assert np.array_equal(tokens.cpu().numpy(), want_out), want_path
        assert np.array_equal(accepted.cpu().numpy(), want_acc), want_path
        assert valid.tolist()[1] == 0
