"""Draft-side proposal heads on the GPU: the DSpark Markov walk (snowllm_dspark_markov) against
oracle/dspark.py -- picks bit for bit, confidence within 1e-5 as the reference's own check
(tests/test_lfm2_dspark_reference.py:158-163) -- and the DFlash 2 selector's hidden projection
(SELECTOR_HIDDEN, models/qwen3_5/dflash_draft.py:187-204) within the matmul tolerance, feeding
the selector walk bit-exactly against the C oracle."""
import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import dspark as D
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _markov_case(V, rank, b, block, seed, stride_pad=0):
    g = torch.Generator().manual_seed(seed)
    W1 = (torch.randn(V, rank, generator=g) * .25).bfloat16()
    W2 = (torch.randn(V, rank, generator=g) * .25 * (256 / rank) ** .5).bfloat16()
    base = torch.randn(b * block, V + stride_pad, generator=g)
    anchor = torch.randint(0, V, (b,), generator=g)
    H = 512
    hidden = torch.randn(b * block, H, generator=g).bfloat16()
    conf_w = torch.randn(H + rank, generator=g) * .05
    conf_b = torch.tensor([.3])
    return W1, W2, base, anchor, hidden, conf_w, conf_b


CASES = [
    # V, rank, b, block, stride pad, fp32 bias
    (151936, 256, 1, 8, 0, False),    # the 35B-A3B vocabulary, Markov rank 256, block 8
    (1000, 64, 3, 5, 24, False),      # a partial last tile, padded logit rows
    (4096, 128, 16, 4, 0, False),     # the largest batch
    (2048, 512, 2, 16, 0, True),      # the largest rank, fp32 bias
]


@pytest.mark.parametrize("V,rank,b,block,pad,fp32", CASES)
def test_markov_equals_oracle(gpu, V, rank, b, block, pad, fp32):
    from snowllm_amd.draft_heads import MarkovHead
    _say(f"dspark markov V={V} rank={rank} b={b} block={block} pad={pad} fp32={fp32}")
    W1, W2, base, anchor, hidden, conf_w, conf_b = _markov_case(V, rank, b, block, V + rank, pad)
    if b == 16:
        anchor[3], anchor[7] = -1, V + 9        # outside the table: a zero latent
        base[5, :] = float("nan")               # a row of NaN: index 0
        base[6, 10:20] = 50.0                   # a plateau the bias decides
    head = MarkovHead(W1.cuda(), W2.cuda(), conf_w.cuda(), conf_b.cuda())
    path = torch.full((b, block), -7, dtype=torch.int64, device="cuda")
    conf = torch.full((b, block), -1.0, device="cuda")
    logits = base.cuda()[:, :V] if pad else base.cuda()
    head.propose(hidden.cuda(), logits, anchor.cuda(), path, conf, fp32_bias=fp32)
    torch.cuda.synchronize()
    want_path, want_conf = D.markov(base[:, :V].numpy(), _bits(W1), _bits(W2), anchor.numpy(),
                                    block, pre_head=_bits(hidden), conf_w=conf_w.numpy(),
                                    conf_b=float(conf_b), fp32_bias=fp32)
    assert np.array_equal(path.cpu().numpy(), want_path)
    assert np.abs(conf.cpu().double().numpy() - want_conf).max() < 1e-5
    if b == 16:
        assert path[1, 1].item() == 0 and 10 <= path[1, 2].item() < 20


def test_markov_without_confidence_and_graph_replay(gpu):
    """No confidence output; the arrival counter carries across captured replays."""
    from snowllm_amd.draft_heads import MarkovHead
    V, rank, b, block = 4096, 256, 2, 8
    W1, W2, base, anchor, hidden, conf_w, conf_b = _markov_case(V, rank, b, block, 3)
    head = MarkovHead(W1.cuda(), W2.cuda())
    logits = torch.empty(b * block, V, device="cuda")
    anchors = anchor.cuda()
    path = torch.empty(b, block, dtype=torch.int64, device="cuda")
    logits.copy_(base)
    head.propose(None, logits, anchors, path)          # eager once (allocates the workspace)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        head.propose(None, logits, anchors, path)
    g = torch.Generator().manual_seed(11)
    for i in range(4):
        _say(f"markov graph replay {i}")
        fresh = torch.randn(b * block, V, generator=g)
        logits.copy_(fresh)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want, _ = D.markov(fresh.numpy(), _bits(W1), _bits(W2), anchor.numpy(), block)
        assert np.array_equal(path.cpu().numpy(), want)


@pytest.mark.parametrize("fmt,n", [(0, 8), (0, 24), (4, 8), (8, 40)])
def test_selector_hidden_projection(gpu, fmt, n):
    """hp = hidden W^T against fp32 (W bf16, or dequantised Q4_K / Q8_0), then the selector
    walk on the projected rows equals the C oracle's walk on them."""
    from snowllm_amd import dflash
    from snowllm_amd.draft_heads import SelectorHead
    from snowllm_amd.verify import gguf_random
    H, V, R = 2048, 4096, 256
    _say(f"selector hidden projection fmt={fmt} rows={n}")
    g = torch.Generator().manual_seed(n + fmt)
    hidden = (torch.randn(n, H, generator=g)).bfloat16()
    pred = (torch.randn(V, R, generator=g) * .2).bfloat16()
    succ = (torch.randn(V, R, generator=g) * .2).bfloat16()
    if fmt:
        raw = gguf_random(fmt, R, H, seed=n, centered=fmt == 4)
        w_ref = torch.from_numpy((Q.dequant_q4_k if fmt == 4 else Q.dequant_q8_0)(
            raw.cpu().numpy(), R, H))
        head = SelectorHead(H, raw, pred.cuda(), succ.cuda(), fmt=fmt)
    else:
        w = (torch.randn(R, H, generator=g) * H ** -.5).bfloat16()
        w_ref = w.float()
        head = SelectorHead(H, w.cuda(), pred.cuda(), succ.cuda())
    assert dflash.proj_shape(dflash.Proj.SELECTOR_HIDDEN) == (R, H)
    hp = head.project(hidden.cuda())
    torch.cuda.synchronize()
    ref = hidden.float() @ w_ref.T
    got = hp.float().cpu()
    rel = float((got - ref).norm() / ref.norm())
    _say(f"  hp rel L2 {rel:.2e} vs fp32")
    assert rel < 3e-3                                   # bf16 output rounding: ~1.1e-3
    assert float((got - ref.bfloat16().float()).norm() / ref.norm()) < 1e-3
    # the walk on the projected rows: n / 8 requests of 8 rows, greedy
    b = n // 8
    logits = torch.randn(n, V, generator=g).cuda()
    anchor = torch.arange(b, device="cuda") * 7 + 3
    path = torch.empty(b, 8, dtype=torch.int64, device="cuda")
    hp2 = head.propose(hidden.cuda(), logits, anchor, path)
    torch.cuda.synchronize()
    assert torch.equal(hp2, hp)
    want, _, _ = A.select(hp.cpu(), logits.cpu().numpy(), pred, succ, anchor.cpu().numpy())
    assert np.array_equal(path.cpu().numpy(), want)


def test_other_draft_projections_are_refused(gpu):
    from snowllm_amd import dflash
    from snowllm_amd.errors import SnowLLMError
    dflash.select(type("S", (), {"hidden": 2048})())
    for which in (dflash.Proj.FC, dflash.Proj.QKV, dflash.Proj.DOWN):
        with pytest.raises(SnowLLMError):
            dflash.proj_shape(which)
