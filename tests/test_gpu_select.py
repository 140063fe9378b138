"""GPU parity of the DFlash 2 selector (snowllm_draft_select / snowllm_draft_sample) against the
C oracle: path, candidate ids and probabilities bit for bit, on the scenarios of the
reference's own tests (tests/test_dflash_sampling.py:44-75, tests/test_dflash_selector_topk.py:
42-61), at the BASELINE config-4 vocabulary, and across graph replays."""
import numpy as np
import pytest
import torch

from oracle import accept as A

pytestmark = pytest.mark.gpu

K = 16


def _run(hidden, logits, pred, succ, anchor, temp, uniform, slots, ids, q, path):
    from snowllm_amd import dflash as d
    n = logits.shape[0]
    scratch = torch.empty(d.select_scratch_bytes(n), dtype=torch.uint8, device="cuda")
    d.select_path(hidden, logits, pred, succ, anchor, path, scratch, temperature=temp,
                  uniform=uniform, slots=slots, candidate_ids=ids, probabilities=q)


def _oracle(hidden, logits, pred, succ, anchor, temp, uniform, slots, n_slots):
    return A.select(hidden.cpu(), logits.cpu().numpy(), pred.cpu(), succ.cpu(),
                    anchor.cpu().numpy(), None if temp is None else temp.cpu().numpy(),
                    None if uniform is None else uniform.cpu().numpy(),
                    None if slots is None else slots.cpu().numpy(), n_slots)


def test_mixed_greedy_and_sampling_walk(gpu):
    """tests/test_dflash_sampling.py:44-75: three requests, T = 0 / 1 / 0.65, stable slots."""
    print("selector mixed walk b=3 ell=7 V=67", flush=True)
    torch.manual_seed(0)
    batch, length, vocab, rank = 3, 7, 67, 256
    hidden = (torch.randn(batch * length, rank) * .2).bfloat16().cuda()
    logits = torch.randn(batch * length, vocab, device="cuda")
    pred = (torch.randn(vocab, rank) * .2).bfloat16().cuda()
    succ = (torch.randn(vocab, rank) * .2).bfloat16().cuda()
    anchor = torch.tensor([5, 21, 51], device="cuda")
    temp = torch.tensor([0., 1., .65], device="cuda")
    uniform = torch.rand(batch, length, device="cuda")
    slots = torch.tensor([4, 0, 2], dtype=torch.int32, device="cuda")
    path = torch.empty(batch, length, dtype=torch.int64, device="cuda")
    ids = torch.full((5, length, K), -99, dtype=torch.int64, device="cuda")
    q = torch.full_like(ids, -99, dtype=torch.float32)
    from snowllm_amd import dflash as d
    scratch = torch.empty(d.select_scratch_bytes(batch * length), dtype=torch.uint8, device="cuda")

    def run():
        d.select_path(hidden, logits, pred, succ, anchor, path, scratch, temperature=temp,
                      uniform=uniform, slots=slots, candidate_ids=ids, probabilities=q)

    def check():
        want_path, want_ids, want_q = _oracle(hidden, logits, pred, succ, anchor, temp, uniform,
                                              slots, 5)
        s = slots.long().cpu().numpy()
        assert np.array_equal(path.cpu().numpy(), want_path)
        assert np.array_equal(ids.cpu().numpy()[s], want_ids[s])
        assert np.array_equal(q.cpu().numpy()[s], want_q[s])
        assert bool((q[1] == -99).all() and (q[3] == -99).all() and (ids[1] == -99).all())

    run()
    torch.cuda.synchronize()
    check()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for u in (.97, .03):
        uniform.fill_(u)
        graph.replay()
        torch.cuda.synchronize()
        check()


@pytest.mark.parametrize("vocab,rows", [(67, 3), (151936, 8), (248320, 3), (248320, 12),
                                        (248320, 16), (248320, 17)])
def test_stable_top16_with_zero_codebooks(gpu, vocab, rows):
    """tests/test_dflash_selector_topk.py:42-61: candidate order, probabilities and path for
    random / tied / NaN rows; scratch, path and unused slots stay untouched."""
    from snowllm_amd import dflash as d
    torch.manual_seed(1743)
    pred = torch.zeros(vocab, 256, dtype=torch.bfloat16, device="cuda")
    hidden = torch.zeros(rows, 256, dtype=torch.bfloat16, device="cuda")
    logits = torch.empty(rows, vocab, device="cuda")
    anchor = torch.zeros(1, dtype=torch.int64, device="cuda")
    temp = torch.zeros(1, device="cuda")
    uniform = torch.full((1, rows), .371, device="cuda")
    slots = torch.tensor([1], dtype=torch.int32, device="cuda")
    path_alloc = torch.full((rows + 128,), -73, dtype=torch.int64, device="cuda")
    path = path_alloc[:rows].view(1, rows)
    ids_alloc = torch.full((3 * rows * K + 128,), -99, dtype=torch.int64, device="cuda")
    ids = ids_alloc[:3 * rows * K].view(3, rows, K)
    q_alloc = torch.full((3 * rows * K + 128,), -99., device="cuda")
    q = q_alloc[:3 * rows * K].view(3, rows, K)
    need = d.select_scratch_bytes(rows)
    scratch = torch.full((need + 256,), 123, dtype=torch.uint8, device="cuda")
    for pattern in ["random", "ties", "nan-mix"]:
        logits.normal_()
        if pattern == "ties":
            logits.zero_()
            logits[:, ::2] = -0.
        elif pattern == "nan-mix":
            logits[:, ::257] = float("nan")
        for temperature in [0., .7]:
            print(f"selector V={vocab} rows={rows} {pattern} T={temperature}", flush=True)
            temp.fill_(temperature)
            d.select_path(hidden, logits, pred, pred, anchor, path, scratch[:need],
                          temperature=temp, uniform=uniform, slots=slots, candidate_ids=ids,
                          probabilities=q)
            torch.cuda.synchronize()
            want_path, want_ids, want_q = _oracle(hidden, logits, pred, pred, anchor, temp,
                                                  uniform, slots, 3)
            assert np.array_equal(ids[1].cpu().numpy(), want_ids[1])
            assert np.array_equal(q[1].cpu().numpy(), want_q[1])
            assert np.array_equal(path.cpu().numpy(), want_path)
            clean = logits.cpu().nan_to_num(nan=-float("inf"))
            assert torch.equal(ids[1].cpu(), clean.argsort(dim=-1, descending=True, stable=True)[:, :K])
            assert bool((scratch[need:] == 123).all() and (path_alloc[rows:] == -73).all()
                        and (ids_alloc[3 * rows * K:] == -99).all()
                        and (q_alloc[3 * rows * K:] == -99).all()
                        and (ids[0] == -99).all() and (ids[2] == -99).all()
                        and (q[0] == -99).all() and (q[2] == -99).all())


def test_greedy_select_equals_temperature_zero(gpu):
    """snowllm_draft_select (no temperature) walks the same path as draft_sample at T = 0."""
    from snowllm_amd import dflash as d
    print("selector greedy entry b=2 ell=8 V=151936", flush=True)
    torch.manual_seed(5)
    b, ell, vocab = 2, 8, 151936
    hidden = (torch.randn(b * ell, 256) * .3).bfloat16().cuda()
    logits = torch.randn(b * ell, vocab, device="cuda") * 2
    pred = (torch.randn(vocab, 256) * .3).bfloat16().cuda()
    succ = (torch.randn(vocab, 256) * .3).bfloat16().cuda()
    anchor = torch.tensor([7, 90000], device="cuda")
    scratch = torch.empty(d.select_scratch_bytes(b * ell), dtype=torch.uint8, device="cuda")
    p1 = torch.empty(b, ell, dtype=torch.int64, device="cuda")
    d.select_path(hidden, logits, pred, succ, anchor, p1, scratch)
    p2 = torch.empty_like(p1)
    ids = torch.empty(b, ell, K, dtype=torch.int64, device="cuda")
    q = torch.empty(b, ell, K, device="cuda")
    d.select_path(hidden, logits, pred, succ, anchor, p2, scratch,
                  temperature=torch.zeros(b, device="cuda"),
                  uniform=torch.rand(b, ell, device="cuda"),
                  slots=torch.arange(b, dtype=torch.int32, device="cuda"), candidate_ids=ids,
                  probabilities=q)
    torch.cuda.synchronize()
    want, _, _ = _oracle(hidden, logits, pred, succ, anchor, None, None, None, None)
    assert np.array_equal(p1.cpu().numpy(), want) and torch.equal(p1, p2)


@pytest.mark.parametrize("rank", [64, 128, 512])
def test_other_codebook_ranks(gpu, rank):
    """The extension entry at codebook ranks other than 256 follows the same canonical sum."""
    print(f"selector rank {rank}", flush=True)
    torch.manual_seed(rank)
    b, ell, vocab = 2, 5, 5000
    hidden = (torch.randn(b * ell, rank) * .3).bfloat16().cuda()
    logits = torch.randn(b * ell, vocab, device="cuda")
    pred = (torch.randn(vocab, rank) * .3).bfloat16().cuda()
    succ = (torch.randn(vocab, rank) * .3).bfloat16().cuda()
    anchor = torch.tensor([1, 4999], device="cuda")
    temp = torch.tensor([0., .8], device="cuda")
    uniform = torch.rand(b, ell, device="cuda")
    slots = torch.tensor([1, 0], dtype=torch.int32, device="cuda")
    path = torch.empty(b, ell, dtype=torch.int64, device="cuda")
    ids = torch.empty(2, ell, K, dtype=torch.int64, device="cuda")
    q = torch.empty(2, ell, K, device="cuda")
    _run(hidden, logits, pred, succ, anchor, temp, uniform, slots, ids, q, path)
    torch.cuda.synchronize()
    want_path, want_ids, want_q = _oracle(hidden, logits, pred, succ, anchor, temp, uniform,
                                          slots, 2)
    assert np.array_equal(path.cpu().numpy(), want_path)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.array_equal(q.cpu().numpy(), want_q)
