"""Sampling lists of any width, penalties, n-gram masks, slot resolution and the verify
dispatch's fallbacks on the GPU, through the C ABI, against the C oracle (bit-exact) and the
reference tests' own expectations (tests/test_runtime_buffers.py:108-152,
tests/test_dflash_sampling.py:190-217, snowllm/engine/spec_decode.py:183)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import accept as A

pytestmark = pytest.mark.gpu
V = 151936


def _say(msg):
    print(msg, flush=True)


def _params(params, vocab):
    from snowllm_amd import ops
    temp = torch.tensor([t if t > 0 else 1.0 for t, _, _ in params])
    top_k = torch.tensor([1 if t <= 0 else (k if 0 < k <= ops.SAMPLING_MAX_K else ops.SAMPLING_MAX_K)
                          for t, k, _ in params], dtype=torch.int32)
    top_p = torch.tensor([p for _, _, p in params])
    return temp, top_k, top_p


@pytest.mark.parametrize("width,params", [
    # whole vocabulary under top-p (top_k 0), wide top-k with and without top-p, short lists
    # and identity rows in the same launch
    (V, [(1., 0, .9), (1., 2000, 1.), (.8, 5000, .7), (1., 0, 1.), (.7, 16, 1.), (0., 1, 1.),
         (1.3, 0, .5)]),
    (2000, [(1., 2000, 1.), (1., 1500, .95), (.7, 16, .8), (1., 1025, 1.)]),
    (V, [(1., 0, 0.0), (1., 0, 1e-9), (1., V - 1, .999)]),
])
def test_wide_probabilities_bit_exact(gpu, width, params):
    from snowllm_amd import ops
    _say(f"wide probabilities width={width} rows={len(params)}")
    rows = len(params)
    g = torch.Generator().manual_seed(width + rows)
    logits = torch.randn(rows, V, generator=g) * 2.0
    temp, top_k, top_p = _params(params, V)
    out = torch.empty(rows, width, device="cuda")
    idx = torch.empty(rows, width, dtype=torch.int64, device="cuda")
    ws = torch.empty(ops.sample_workspace_bytes(rows, V, width), dtype=torch.uint8, device="cuda")
    ops.probabilities(logits.cuda(), top_k.cuda(), top_p.cuda(), temp.cuda(), width, out, idx, ws)
    want_v, want_i = A.probabilities(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(),
                                     width)
    got_v, got_i = out.cpu().numpy(), idx.cpu().numpy()
    for r in range(rows):
        assert np.array_equal(got_i[r], want_i[r]), r
        assert np.array_equal(got_v[r].view(np.uint32), want_v[r].view(np.uint32)), r
    assert not (got_i == -2).any()


def test_wide_sample_bit_exact(gpu):
    from snowllm_amd import ops
    rows = 5
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(rows, V, generator=g) * 2.0
    temp = torch.tensor([1.0, .8, 1.0, 1.2, 1.0])
    top_k = torch.tensor([ops.SAMPLING_MAX_K, 2000, ops.SAMPLING_MAX_K, 30000, 5],
                         dtype=torch.int32)
    top_p = torch.tensor([.9, 1.0, .6, .95, 1.0])
    for trial in range(3):
        uniform = torch.rand(rows, generator=g)
        if trial == 2:
            uniform[0], uniform[1] = 0.0, 0.99999994
        _say(f"wide sample trial {trial}")
        got = ops.sample(logits.cuda(), top_k.cuda(), top_p.cuda(), temp.cuda(), V,
                         uniform=uniform.cuda()).cpu().numpy()
        want = A.sample(logits.numpy(), top_k.numpy(), top_p.numpy(), temp.numpy(),
                        uniform.numpy(), V)
        assert np.array_equal(got, want), trial


def test_penalties_kernel_bit_exact(gpu):
    from snowllm_amd.sampling import penalties
    g = torch.Generator().manual_seed(3)
    vocab = 4099
    for presence, frequency, repetition in [(.4, .2, 1.3), (-.2, .1, .9), (0., 0., 2.), (1.5, -.7, 1.)]:
        x = torch.randn(vocab, generator=g) * 3
        ids = torch.randperm(vocab, generator=g)[:700].long()
        ids[::97] = torch.tensor([-5, vocab, vocab + 3] * 3)[:ids[::97].numel()]
        counts = torch.randint(0, 4, (700,), generator=g, dtype=torch.int32)
        d = x.cuda()
        penalties(d, ids.cuda(), counts.cuda(), presence, frequency, repetition)
        want = A.penalties(x.numpy(), ids.numpy(), counts.numpy(), presence, frequency, repetition)
        assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _sampler(rows, vocab, **kw):
    from snowllm_amd.sampler import Sampler
    s = Sampler(frozenset(), seed=kw.pop("seed", 123))
    s.reserve(rows, vocab, **kw)
    return s


def test_sampler_penalties_match_independent_rows(gpu):
    """tests/test_runtime_buffers.py:108-132: the batched penalties of verify rows equal the
    penalties applied row by row with each row's own ids and counts."""
    from collections import Counter
    from snowllm_amd.sampler import SamplingParams
    from snowllm_amd.sampling import penalties
    s = _sampler(6, 31, max_tokens=17, max_requests=2)
    a = SimpleNamespace(params=SamplingParams(presence_penalty=.4, frequency_penalty=.2,
                                              repetition_penalty=1.3),
                        prompt=[1, 2, 1], out=[3, 3], drafts=[4, 1, 5])
    b = SimpleNamespace(params=SamplingParams(presence_penalty=-.2, frequency_penalty=.1,
                                              repetition_penalty=.9),
                        prompt=[6, 7], out=[], drafts=[8])
    rows = [a, b, a, b, a, a]
    logits = torch.arange(6 * 31, dtype=torch.float32, device="cuda").view(6, 31) / 10 - 9
    expected = logits.clone()
    depths = {}
    for i, r in enumerate(rows):
        depth = depths.get(id(r), 0)
        depths[id(r)] = depth + 1
        counts = Counter(r.out)
        counts.update(r.drafts[:depth])
        ids = sorted(set(r.prompt) | counts.keys())
        penalties(expected[i], torch.tensor(ids, dtype=torch.int64, device="cuda"),
                  torch.tensor([counts.get(t, 0) for t in ids], dtype=torch.int32, device="cuda"),
                  r.params.presence_penalty, r.params.frequency_penalty,
                  r.params.repetition_penalty)
    s.prepare(logits, rows)
    assert torch.equal(logits, expected)


def test_sampler_future_drafts_not_penalised(gpu):
    # tests/test_runtime_buffers.py:136-143
    from snowllm_amd.sampler import SamplingParams
    s = _sampler(3, 16, max_tokens=9, max_requests=1)
    row = SimpleNamespace(params=SamplingParams(repetition_penalty=2), prompt=[1], out=[],
                          drafts=[2, 3])
    logits = torch.full((3, 16), 8., device="cuda")
    s.prepare(logits, [row] * 3)
    values = logits.cpu().tolist()
    assert [values[i][2] for i in range(3)] == [8., 4., 4.]
    assert [values[i][3] for i in range(3)] == [8., 8., 4.]


def test_sampler_penalty_overflow_rejected(gpu):
    # tests/test_runtime_buffers.py:145-152
    from snowllm_amd.errors import SnowLLMError
    from snowllm_amd.sampler import SamplingParams
    s = _sampler(1, 16, max_tokens=8)
    logits = torch.ones(1, 16, device="cuda")
    row = SimpleNamespace(params=SamplingParams(repetition_penalty=1.1), prompt=list(range(9)),
                          out=[], drafts=[])
    with pytest.raises(SnowLLMError):
        s.sample(logits, [row])
    assert torch.equal(logits, torch.ones(1, 16, device="cuda"))


def test_sampler_ngram_masks_and_sample_bit_exact(gpu):
    """Sampler.sample / probabilities: penalties, then the n-gram bans of each verify depth
    (snowllm/engine/sampler.py:146-168), then the lists -- the oracle on the same steps."""
    from snowllm_amd.ngram import banned_ngram_tokens
    from snowllm_amd.sampler import SamplingParams
    vocab = 5000
    g = torch.Generator().manual_seed(21)
    a = SimpleNamespace(params=SamplingParams(temperature=.9, top_k=0, top_p=.9,
                                              repetition_penalty=1.2, presence_penalty=.3,
                                              no_repeat_ngram_size=2),
                        prompt=[5, 6, 7, 5], out=[6, 9], drafts=[5, 6])
    b = SimpleNamespace(params=SamplingParams(temperature=1.1, top_k=1500, top_p=1.0,
                                              no_repeat_ngram_size=1),
                        prompt=[1, 2, 3], out=[], drafts=[4])
    rows = [a, a, a, b, b]
    s = _sampler(len(rows), vocab, max_tokens=64, seed=4)
    logits = torch.randn(len(rows), vocab, generator=g) * 2
    # the oracle's view of the same steps
    x = logits.numpy().copy()
    depth = {}
    for i, r in enumerate(rows):
        d = depth.get(id(r), 0)
        depth[id(r)] = d + 1
        if r.params.penalized():
            from collections import Counter
            counts = Counter(r.out)
            counts.update(r.drafts[:d])
            ids = sorted(set(r.prompt) | counts.keys())
            x[i] = A.penalties(x[i], np.array(ids), np.array([counts[t] for t in ids], np.int32),
                               r.params.presence_penalty, r.params.frequency_penalty,
                               r.params.repetition_penalty)
        banned = banned_ngram_tokens(list(r.prompt) + list(r.out) + list(r.drafts[:d]),
                                     r.params.no_repeat_ngram_size)
        x[i, banned] = -np.inf
    ks = np.array([r.params.kernel_top_k() for r in rows], np.int32)
    tp = np.array([r.params.top_p for r in rows], np.float32)
    tt = np.array([r.params.kernel_temperature() for r in rows], np.float32)
    width = min(int(ks.max()), vocab)
    out = torch.empty(len(rows) * vocab, device="cuda")
    idx = torch.empty(len(rows) * vocab, dtype=torch.int64, device="cuda")
    d_logits = logits.cuda()
    values, ids = s.probabilities(d_logits, rows, out, idx)
    want_v, want_i = A.probabilities(x, ks, tp, tt, width)
    assert np.array_equal(d_logits.cpu().numpy(), x)
    assert np.array_equal(ids.cpu().numpy(), want_i)
    assert np.array_equal(values.cpu().numpy().view(np.uint32), want_v.view(np.uint32))
    # and the sample itself (a fresh copy of the logits: prepare runs again)
    d_logits = logits.cuda()
    got = s.sample(d_logits, rows).cpu().numpy()
    u = s.uniforms[:len(rows)].cpu().numpy()
    want = A.sample(x, ks, tp, tt, u, width)
    assert np.array_equal(got, want)


def test_resolve_slots_closed_form(gpu):
    """slot = table[seq, pos // page] * page + pos % page (snowllm/engine/spec_decode.py:183,
    snowllm/ops/cache.py:40-53); rows outside the table, negative positions or sequences and
    padding entries give -1."""
    from snowllm_amd.layers import resolve_slots
    g = torch.Generator().manual_seed(8)
    B, width, page = 5, 12, 16
    table = torch.randperm(200, generator=g)[:B * width].int().view(B, width)
    table[3, 9:] = -1   # a shorter request, padded
    M = 400
    seq = torch.randint(0, B, (M,), generator=g, dtype=torch.int32)
    pos = torch.randint(0, width * page + 40, (M,), generator=g, dtype=torch.int32)
    pos[:7] = torch.tensor([-1, -16, 0, 15, 16, width * page - 1, width * page], dtype=torch.int32)
    seq[10:13] = torch.tensor([-1, -7, 2], dtype=torch.int32)
    got = resolve_slots(table.cuda(), seq.cuda(), pos.cuda(), page).cpu()
    want = []
    for s, p in zip(seq.tolist(), pos.tolist()):
        if s < 0 or p < 0 or p // page >= width or table[s, p // page] < 0:
            want.append(-1)
        else:
            want.append(int(table[s, p // page]) * page + p % page)
    assert got.tolist() == want
    assert (got == -1).sum() > 10


def test_dispatch_beyond_fused_shapes_takes_lists(gpu):
    """32 requests of block 9 (288 rows > the fused kernels' 256): the sampling batch falls back
    to probabilities + reject and the greedy batch to argmax + spec_accept, bit-exact."""
    from snowllm_amd.dflash_sampling import DFlashAcceptance, SamplingParams, VerifyRequest
    vocab, width, count = 4096, 9, 32
    length = width - 1
    acc = DFlashAcceptance(max_seqs=count, block=width, vocab=vocab, seed=9)
    g = torch.Generator().manual_seed(14)
    cand = torch.stack([torch.stack([torch.randperm(vocab, generator=g)[:16]
                                     for _ in range(length)]) for _ in range(count)])
    q = torch.rand(count, length, 16, generator=g) + 0.05
    q = q / q.sum(-1, keepdim=True)
    acc.candidates.copy_(cand)
    acc.q.copy_(q)
    for temp in (1.0, 0.0):
        logits = torch.randn(count * width, vocab, generator=g) * 2
        top = torch.from_numpy(A.argmax(logits.numpy())).view(count, width)
        drafts = top[:, :length].clone()
        drafts[::3, 2] = torch.randint(0, vocab, (drafts[::3].shape[0],), generator=g)
        batch = [VerifyRequest(slot=i, params=SamplingParams(temp), drafts=tuple(drafts[i].tolist()))
                 for i in range(count)]
        acc.remember(batch, [r.drafts for r in batch])
        _say(f"dispatch 288 rows temperature {temp}")
        tokens, accepted = acc.verify(logits.cuda(), batch, drafts.cuda())
        torch.cuda.synchronize()
        if temp == 0.0:
            assert acc.path == "greedy"
            assert torch.equal(tokens.cpu(), top)
            assert np.array_equal(accepted.cpu().numpy(), A.spec_accept(top.numpy(), drafts.numpy()))
            continue
        assert acc.path == "lists"
        ident = np.tile(np.arange(vocab), (count * width, 1))
        u = acc.verify_uniform[:count * width].view(count, width).cpu().numpy()
        want_out, want_acc = A.reject(A.softmax(logits.numpy()), ident, drafts.numpy(),
                                      cand.numpy(), q.numpy(), np.arange(count, dtype=np.int32),
                                      np.ones(count, np.int32), u)
        assert np.array_equal(tokens.cpu().numpy(), want_out)
        assert np.array_equal(accepted.cpu().numpy(), want_acc)


def test_dispatch_nucleus_over_whole_vocabulary(gpu):
    """A plain top-p request (top_k unset, top_p 0.9) at V = 151,936 next to a wide top-k one:
    the lists branch, bit-exact against the oracle (no -2 tokens)."""
    from snowllm_amd.dflash_sampling import DFlashAcceptance, SamplingParams, VerifyRequest
    width, length = 9, 8
    acc = DFlashAcceptance(max_seqs=2, block=width, vocab=V, seed=2)
    g = torch.Generator().manual_seed(31)
    cand = torch.stack([torch.stack([torch.randperm(V, generator=g)[:16] for _ in range(length)])
                        for _ in range(2)])
    q = torch.rand(2, length, 16, generator=g) + 0.05
    q = q / q.sum(-1, keepdim=True)
    acc.candidates.copy_(cand)
    acc.q.copy_(q)
    logits = torch.randn(2 * width, V, generator=g) * 2
    drafts = cand[:, :, 0].clone()
    batch = [VerifyRequest(slot=0, params=SamplingParams(1.0, top_p=0.9), drafts=tuple(drafts[0].tolist())),
             VerifyRequest(slot=1, params=SamplingParams(0.8, top_k=3000, top_p=0.95),
                           drafts=tuple(drafts[1].tolist()))]
    acc.remember(batch, [r.drafts for r in batch])
    _say("dispatch nucleus over the whole vocabulary")
    tokens, accepted = acc.verify(logits.cuda(), batch, drafts.cuda())
    torch.cuda.synchronize()
    assert acc.path == "lists"
    rows = [r for r in batch for _ in range(width)]
    ks = np.array([r.params.kernel_top_k() for r in rows], np.int32)
    tp = np.array([r.params.top_p for r in rows], np.float32)
    tt = np.array([r.params.kernel_temperature() for r in rows], np.float32)
    p, ids = A.probabilities(logits.numpy(), ks, tp, tt, min(int(ks.max()), V))
    u = acc.verify_uniform[:2 * width].view(2, width).cpu().numpy()
    want_out, want_acc = A.reject(p, ids, drafts.numpy(), cand.numpy(), q.numpy(),
                                  np.arange(2, dtype=np.int32), np.ones(2, np.int32), u)
    assert np.array_equal(tokens.cpu().numpy(), want_out)
    assert np.array_equal(accepted.cpu().numpy(), want_acc)
    assert (tokens.cpu() >= -1).all()
