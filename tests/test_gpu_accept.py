"""GPU parity of the acceptance kernels against the C oracle (bit-exact) and the reference's
torch semantics. Shapes follow the reference's own tests and BASELINE config 1."""
import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import reference as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("rows,vocab,offset", [(b, 248320, 0) for b in (1, 3, 9, 17)]
                         + [(3, 248320, 1), (3, 1027, 0), (3, 31, 0), (0, 248320, 0)])
def test_argmax(gpu, rows, vocab, offset):
    from snowllm_amd import ops
    # tests/test_sampling_argmax.py:13-43 (patterns, graph capture, output bounds)
    g = torch.Generator().manual_seed(1743 + rows)
    storage = torch.randn(rows * vocab + offset, generator=g).cuda()
    logits = storage[offset:].view(rows, vocab)
    allocation = torch.full((rows + 32,), -73, dtype=torch.int64, device="cuda")
    output = allocation[:rows]
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
        expected = torch.from_numpy(A.argmax(logits.cpu().numpy()))
        for capture in (False, True):
            _say(f"argmax {rows}x{vocab} offset={offset} {pattern} graph={capture}")
            output.fill_(-73)
            if capture and rows:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    ops.argmax(logits, out=output)
                graph.replay()
            else:
                ops.argmax(logits, out=output)
            torch.cuda.synchronize()
            assert torch.equal(output.cpu(), expected), (pattern, capture)
            assert bool((allocation[rows:] == -73).all())


def test_spec_accept(gpu):
    from snowllm_amd import ops
    g = torch.Generator().manual_seed(3)
    b, T = 37, 9
    drafts_full = torch.randint(0, 50, (b, T + 3), generator=g)
    tokens_full = torch.randint(0, 50, (b, T + 5), generator=g)
    for i in range(b):  # force varied leading-match lengths
        n = i % T
        tokens_full[i, :n] = drafts_full[i, :n]
    tokens = tokens_full.cuda()[:, :T]
    drafts = drafts_full.cuda()[:, :T - 1]
    got = ops.spec_accept(tokens, drafts).cpu().numpy()
    want = A.spec_accept(tokens_full[:, :T].numpy(), drafts_full[:, :T - 1].numpy())
    assert np.array_equal(got, want)
    # and against the reference's CPU loop
    _, acc = R.reference_greedy(torch.nn.functional.one_hot(tokens_full[:, :T].reshape(-1), 64).float(),
                                drafts_full[:, :T - 1])
    assert np.array_equal(got, acc.numpy())


@pytest.mark.parametrize("rows,vocab", [(4, 67), (9, 1027), (17, 151936), (3, 248320)])
def test_softmax_bit_exact(gpu, rows, vocab):
    from snowllm_amd import ops
    from snowllm_amd._capi import check, lib
    _say(f"softmax {rows}x{vocab}")
    g = torch.Generator().manual_seed(rows + vocab)
    x = torch.randn(rows, vocab, generator=g) * 2.0
    x[0, :5] = float("-inf")
    if rows > 2:
        x[2, 7] = float("nan")
    t = torch.rand(rows, generator=g) + 0.5
    t[0] = 1.0
    t[1] = 0.0  # temperature <= 0 counts as 1
    ws = torch.empty(ops.sample_workspace_bytes(rows, vocab, vocab), dtype=torch.uint8, device="cuda")
    xd, td = x.cuda(), t.cuda()
    check(lib.snowllm_sampling_softmax(xd.data_ptr(), ws.data_ptr(), rows, vocab, td.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream), "softmax")
    got = ws.view(torch.float32)[:rows * vocab].view(rows, vocab).cpu().numpy()
    want = A.softmax(x.numpy(), t.numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("vocab,width,params", [
    (67, 67, [(0., 1, 1.), (.65, 20, .95), (1.3, 0, .8), (1., 3, .5)]),
    (151936, 1024, [(1., 1024, 1.), (.7, 16, 1.), (1., 50, .9), (0., 1, 1.)]),
    (151936, 151936, [(1., 0, 1.), (1., 0, 1.)]),
])
def test_probabilities_bit_exact(gpu, vocab, width, params):
    from snowllm_amd import ops
    _say(f"probabilities V={vocab} width={width}")
    rows = len(params)
    g = torch.Generator().manual_seed(vocab + width)
    logits = torch.randn(rows, vocab, generator=g) * 2.0
    temp = torch.tensor([t if t > 0 else 1.0 for t, _, _ in params])
    top_k = torch.tensor([1 if t <= 0 else (k if 0 < k <= ops.SAMPLING_MAX_K else ops.SAMPLING_MAX_K)
                          for t, k, _ in params], dtype=torch.int32)
    top_p = torch.tensor([p for _, _, p in params])
    out = torch.empty(rows, width, device="cuda")
    idx = torch.empty(rows, width, dtype=torch.int64, device="cuda")
    ws = torch.empty(ops.sample_workspace_bytes(rows, vocab, width), dtype=torch.uint8, device="cuda")
    ops.probabilities(logits.cuda(), top_k.cuda(), top_p.cuda(), temp.cuda(), width, out, idx, ws)
    want_v, want_i = A.probabilities(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(), width)
    got_v, got_i = out.cpu().numpy(), idx.cpu().numpy()
    assert np.array_equal(got_i, want_i)
    assert np.array_equal(got_v.view(np.uint32), want_v.view(np.uint32))
    if vocab == 67:  # tests/test_dflash_sampling.py:190-209
        actual = torch.zeros(rows, vocab).scatter_add_(1, torch.from_numpy(got_i).clamp_min(0),
                                                       torch.from_numpy(got_v))
        expected = R.target_probabilities(logits, torch.tensor([t for t, _, _ in params]), top_k, top_p)
        assert ((actual - expected).norm() / expected.norm()).item() < 1e-5


def test_sample_bit_exact(gpu):
    from snowllm_amd import ops
    g = torch.Generator().manual_seed(11)
    rows, vocab = 6, 151936
    logits = torch.randn(rows, vocab, generator=g) * 2.0
    temp = torch.tensor([1.0, .7, 1.0, 1.2, 1.0, 1.0])
    top_k = torch.tensor([20, 1024, 1, 5, 64, 3], dtype=torch.int32)
    top_p = torch.tensor([1.0, .9, 1.0, .5, .95, 1.0])
    for trial in range(3):
        uniform = torch.rand(rows, generator=g)
        if trial == 2:
            uniform[0] = 0.0
            uniform[1] = 0.99999994
        width = 1024
        got = ops.sample(logits.cuda(), top_k.cuda(), top_p.cuda(), temp.cuda(), width,
                         uniform=uniform.cuda()).cpu().numpy()
        want = A.sample(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(), uniform.numpy(), width)
        assert np.array_equal(got, want), trial


def _rejection_case(width, length, seed):
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
def test_reject_reference_cases(gpu, width, length):
    from snowllm_amd import ops
    _say(f"reject width={width} block={length + 1}")
    p, p_ids, drafts, q_ids, q, slots, valid, uniform = _rejection_case(width, length, 73 + width)
    batch = drafts.shape[0]
    want, kept = R.reference_reject(p.view(batch, length + 1, width), p_ids.view(batch, length + 1, width),
                                    drafts, q_ids, q, slots, valid, uniform)
    actual = torch.empty(batch, length + 1, dtype=torch.int64, device="cuda")
    accepted = torch.empty(batch, dtype=torch.int64, device="cuda")
    args = [t.cuda() for t in (p, p_ids, drafts, q_ids, q, slots.int(), valid, uniform)]
    ops.dflash.reject(*args, actual, accepted)
    assert torch.equal(accepted.cpu(), kept)
    assert torch.equal(actual.cpu(), want)


def test_reject_distribution(gpu):
    from snowllm_amd import ops
    batch, width = 40000, 4
    target = torch.tensor([.1, .2, .3, .4])
    draft = torch.tensor([.45, .35, .2, 0.])
    g = torch.Generator().manual_seed(9)
    p = target.repeat(batch * 2, 1).cuda()
    ids = torch.arange(width).repeat(batch * 2, 1).cuda()
    q = draft.repeat(batch, 1, 1).cuda()
    q_ids = torch.arange(width).repeat(batch, 1, 1).cuda()
    tokens = torch.multinomial(draft, batch, replacement=True, generator=g).view(batch, 1).cuda()
    slots = torch.arange(batch, dtype=torch.int32, device="cuda")
    valid = torch.ones(batch, dtype=torch.int32, device="cuda")
    uniform = torch.rand(batch, 2, generator=g).cuda()
    out = torch.empty(batch, 2, dtype=torch.int64, device="cuda")
    accepted = torch.empty(batch, dtype=torch.int64, device="cuda")
    ops.dflash.reject(p, ids, tokens, q_ids, q, slots, valid, uniform, out, accepted)
    observed = out[:, 0].bincount(minlength=4).float().cpu() / batch
    assert (observed - target).abs().max() < .01
    assert abs((accepted == 2).float().mean().item() - torch.minimum(target, draft).sum().item()) < .01
    want, acc = A.reject(p.cpu().numpy(), ids.cpu().numpy(), tokens.cpu().numpy(), q_ids.cpu().numpy(),
                         q.cpu().numpy(), slots.cpu().numpy(), valid.cpu().numpy(), uniform.cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), want) and np.array_equal(accepted.cpu().numpy(), acc)


def config1_inputs():
    """target [9, V], draft [8, V] ~ N(0, 2^2) (seeds 10, 11); draft tokens
    from the draft softmax (seed 0); uniforms U(0,1) [1, 9] (seed 1)."""
    V, k = 151936, 8
    target = torch.randn(k + 1, V, generator=torch.Generator().manual_seed(10)) * 2.0
    draft = torch.randn(k, V, generator=torch.Generator().manual_seed(11)) * 2.0
    drafts = torch.multinomial(draft.softmax(-1), 1, generator=torch.Generator().manual_seed(0)).view(1, k)
    uniform = torch.rand(1, k + 1, generator=torch.Generator().manual_seed(1))
    return target, draft, drafts, uniform


def test_config1_rejection_full_vocab(gpu):
    from snowllm_amd import ops
    target, draft, drafts, uniform = config1_inputs()
    V, k = target.shape[1], drafts.shape[1]
    ws_t = torch.empty(ops.sample_workspace_bytes(k + 1, V, V), dtype=torch.uint8, device="cuda")
    ws_q = torch.empty(ops.sample_workspace_bytes(k, V, V), dtype=torch.uint8, device="cuda")
    ones = lambda n: torch.ones(n, device="cuda")
    kmax = lambda n: torch.full((n,), ops.SAMPLING_MAX_K, dtype=torch.int32, device="cuda")
    p = torch.empty(k + 1, V, device="cuda")
    pid = torch.empty(k + 1, V, dtype=torch.int64, device="cuda")
    q = torch.empty(k, V, device="cuda")
    qid = torch.empty(k, V, dtype=torch.int64, device="cuda")
    ops.probabilities(target.cuda(), kmax(k + 1), ones(k + 1), ones(k + 1), V, p, pid, ws_t)
    ops.probabilities(draft.cuda(), kmax(k), ones(k), ones(k), V, q, qid, ws_q)
    out = torch.empty(1, k + 1, dtype=torch.int64, device="cuda")
    acc = torch.empty(1, dtype=torch.int64, device="cuda")
    for trial in range(6):
        u = uniform if trial == 0 else torch.rand(1, k + 1, generator=torch.Generator().manual_seed(100 + trial))
        if trial == 5:
            u[0, :-1] = 0.0  # accept everything the target supports, then a bonus draw
        ops.dflash.reject(p, pid, drafts.cuda(), qid.view(1, k, V), q.view(1, k, V),
                          torch.zeros(1, dtype=torch.int32, device="cuda"),
                          torch.ones(1, dtype=torch.int32, device="cuda"), u.cuda(), out, acc)
        pn, qn = p.cpu().numpy(), q.cpu().numpy()
        assert np.array_equal(pn, A.softmax(target.numpy()))
        want, wacc = A.reject(pn, pid.cpu().numpy(), drafts.numpy(), qid.cpu().numpy()[None],
                              qn[None], np.zeros(1, np.int32), np.ones(1, np.int32), u.numpy())
        assert np.array_equal(out.cpu().numpy(), want), trial
        assert np.array_equal(acc.cpu().numpy(), wacc), trial
        rwant, racc = R.reference_reject_identity(torch.from_numpy(pn)[None], drafts,
                                                  torch.from_numpy(qn)[None], u)
        assert torch.equal(out.cpu(), rwant) and torch.equal(acc.cpu(), racc), trial


def test_config1_greedy(gpu):
    from snowllm_amd import ops
    target, draft, drafts, uniform = config1_inputs()
    # make the first three drafts agree with the target argmax so the prefix scan has work
    am = target.argmax(-1)
    drafts = drafts.clone()
    drafts[0, :3] = am[:3]
    tokens = ops.argmax(target.cuda())
    acc = ops.spec_accept(tokens.view(1, -1), drafts.cuda())
    tv, racc = R.reference_greedy(target, drafts)
    assert torch.equal(tokens.cpu().view(1, -1), tv)
    assert torch.equal(acc.cpu(), racc) and int(acc[0]) == 4


def test_reject_graph_replay(gpu):
    from snowllm_amd import ops
    p, p_ids, drafts, q_ids, q, slots, valid, uniform = _rejection_case(20, 3, 5)
    batch, length = drafts.shape
    args = [t.cuda() for t in (p, p_ids, drafts, q_ids, q, slots.int(), valid, uniform)]
    out = torch.empty(batch, length + 1, dtype=torch.int64, device="cuda")
    acc = torch.empty(batch, dtype=torch.int64, device="cuda")
    graph = torch.cuda.CUDAGraph()
    ops.dflash.reject(*args, out, acc)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        ops.dflash.reject(*args, out, acc)
    for fill in (.97, .03, None):
        if fill is None:
            args[7].copy_(uniform.cuda())
        else:
            args[7].fill_(fill)
        graph.replay()
        torch.cuda.synchronize()
        want, wacc = A.reject(*[a.cpu().numpy() for a in args])
        assert np.array_equal(out.cpu().numpy(), want) and np.array_equal(acc.cpu().numpy(), wacc)
