"""Batched and ragged verify steps (snowllm/engine/spec_decode.py:143-209, 263-309): several
requests, each with its own context, pages and (DSpark) prefix length, verified in one step of
up to 256 rows. Every request's rows are checked against the CPU layer reference
(oracle/model.py) under teacher forcing, its logits against the head reference, and the
batched acceptance bit-exact against the C oracle."""
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import model as RM
from tests.kvcache import cache_rows

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _say(msg):
    print(msg, flush=True)


def tiny(kind, block=9):
    from snowllm_amd.verify import VerifyConfig
    base = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rot_half=32,
                rope_theta=1e4, vocab=2048, context=300, block=block)
    if kind == "moe":
        return VerifyConfig("tiny_moe", experts=16, expert_ffn=256, topk=4, **base)
    return VerifyConfig("tiny_dense", ffn=512, **dict(base, kv_heads=1, rot_half=64))


def check_layers(m, contexts, lengths, layers, tol):
    """Teacher-forced layer parity for every request of the staged batch."""
    cfg, T = m.cfg, m.cfg.block
    inv = m.inv_freq.cpu()
    cos, sin = RM.rope_tables(m.positions.cpu(), inv)
    for layer in layers:
        m.forward(upto_layer=layer)
        torch.cuda.synchronize()
        x_in = m.x.float().cpu()
        res_in = None if layer == 0 else m.layer_residual.float().cpu()
        kpool, vpool = m.k_pools[layer].cpu(), m.v_pools[layer].cpu()
        m.forward(upto_layer=layer + 1)
        torch.cuda.synchronize()
        attn_g, x_g = m.attn.float().cpu(), m.x.float().cpu()
        res_g = m.layer_residual.float().cpu()
        ids_g = m.route_ids.cpu().long() if cfg.moe else None
        h2_g = m.h2.float().cpu() if cfg.moe else None
        for b, (ctx, n) in enumerate(zip(contexts, lengths)):
            rows = slice(b * T, b * T + n)
            pages = m.table[b].long().cpu()
            kctx = cache_rows(kpool, pages, cfg.kv_heads, cfg.head_dim, 16, key=True)[:ctx]
            vctx = cache_rows(vpool, pages, cfg.kv_heads, cfg.head_dim, 16, key=False)[:ctx]
            ref = RM.LayerRef(cfg, m.layers[layer])
            x2, r2, attn, routing = RM.layer_forward(
                ref, x_in[rows], None if res_in is None else res_in[rows], cos[rows], sin[rows],
                kctx, vctx, [(2 << t) - 1 for t in range(n)])
            e = (rel(attn_g[rows], attn), rel(res_g[rows], r2), rel(x_g[rows], x2))
            flips = 0
            if routing is not None:
                flips = int((ids_g[rows].sort(-1).values != routing.sort(-1).values)
                            .any(-1).sum())
            _say(f"  layer {layer} request {b} (ctx {ctx}, {n} rows): attn {e[0]:.2e} "
                 f"residual {e[1]:.2e} ffn {e[2]:.2e} routing differs on {flips} rows")
            assert e[0] < tol[0] and e[1] < tol[1], (layer, b, e)
            if routing is not None and flips:
                # the oracle's own attention moved a near-tie of the router: the experts are
                # checked on the GPU's normalised rows instead (teacher forcing the MoE)
                h2 = h2_g[rows]
                logits = (h2.double() @ ref.router.double().T).float()
                x2, routing = RM.moe_ffn(ref, h2, logits)
                e = (e[0], e[1], rel(x_g[rows], x2))
                _say(f"    MoE on the GPU's rows: ffn {e[2]:.2e}")
            assert e[2] < tol[2], (layer, b, e)
            if routing is not None:
                assert torch.equal(ids_g[rows].sort(-1).values, routing.sort(-1).values)


def check_logits(m, lengths, tol):
    T = m.cfg.block
    logits = m.forward().clone()
    torch.cuda.synchronize()
    want = RM.head_reference(m.x.float().cpu(), m.layer_residual.float().cpu(),
                             m.final_norm.cpu(), m.lm_head_raw.cpu(), m.cfg.eps)
    for b, n in enumerate(lengths):
        rows = slice(b * T, b * T + n)
        e = rel(logits.cpu()[rows], want[rows])
        assert e < tol, (b, e)
    return logits


@pytest.mark.parametrize("kind", ["moe", "dense"])
def test_batch_of_four_blocks(gpu, kind):
    """Four requests of block 9 (36 rows: three 16-row chunks for the MoE and the 16-bit
    GEMVs) at different contexts: layers, logits and the batched rejection acceptance."""
    from snowllm_amd import layers as L
    from snowllm_amd.verify import Acceptance, VerifyModel
    cfg = tiny(kind)
    B, T = 4, cfg.block
    _say(f"batch {B} x {T} {cfg.name}")
    m = VerifyModel(cfg, seed=7, keep_raw=True, batch=B)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, cfg.vocab, (B, T), generator=g)
    contexts = [300, 17, 250, 160]
    m.set_batch(ids, contexts)
    check_layers(m, contexts, [T] * B, range(cfg.layers), (2e-3, 3e-3, 1.1e-2))
    logits = check_logits(m, [T] * B, 5e-7)
    assert L.moe_sync_error() == 0
    # batched acceptance over the whole vocabulary
    k = T - 1
    acc = Acceptance(cfg.vocab, list(range(T)), batch=B)
    gd = torch.Generator(device="cuda").manual_seed(9)
    draft_logits = torch.randn(B * k, cfg.vocab, device="cuda", generator=gd) * 2
    top = logits.view(B, T, -1)[:, :k].argmax(-1)
    sampled = torch.multinomial(draft_logits.softmax(-1), 1, generator=gd).view(B, k)
    drafts = torch.where(torch.arange(k, device="cuda") % 3 == 0, sampled, top)
    u = torch.rand(B, T, device="cuda", generator=gd)
    acc.set_draft(draft_logits, drafts, u)
    out, accepted = acc(logits)
    torch.cuda.synchronize()
    p = A.softmax(logits.cpu().numpy())
    q = A.softmax(draft_logits.cpu().numpy()).reshape(B, k, -1)
    ident = np.tile(np.arange(cfg.vocab), (B * T, 1))
    qid = np.tile(np.arange(cfg.vocab), (B, k, 1))
    want_out, want_acc = A.reject(p, ident, drafts.cpu().numpy(), qid, q,
                                  np.arange(B, dtype=np.int32), np.ones(B, np.int32),
                                  u.cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), want_out)
    assert np.array_equal(accepted.cpu().numpy(), want_acc)
    # the captured batched step replays to the eager logits
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        m.forward()
    for _ in range(2):
        m.logits.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.logits, logits)


def test_ragged_dspark_batch(gpu):
    """DSpark prefix lengths 3 / 9 / 16 in one step (snowllm/engine/spec_decode.py:168-209):
    padded to 16 rows per request, padding rows write no cache and are invisible to the real
    ones; each request's real rows match the reference, and the per-row samples + prefix
    acceptance match the oracle."""
    from snowllm_amd.sampler import Sampler, SamplingParams
    from snowllm_amd.verify import VerifyModel
    from types import SimpleNamespace
    cfg = tiny("moe", block=16)
    B, T = 3, 16
    lengths = [3, 9, 16]
    contexts = [120, 299, 64]
    m = VerifyModel(cfg, seed=8, keep_raw=True, batch=B)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab, (B, T), generator=g)
    m.set_batch(ids, contexts, lengths)
    _say(f"ragged batch {lengths}")
    # padding rows write nothing: snapshot the pools past each request's real rows
    check_layers(m, contexts, lengths, range(cfg.layers), (2e-3, 3e-3, 1.1e-2))
    logits = check_logits(m, lengths, 5e-7)
    # each request's block positions beyond its real rows keep the values they had
    m2 = VerifyModel(cfg, seed=8, batch=B)
    for layer in range(cfg.layers):
        for b, (ctx, n) in enumerate(zip(contexts, lengths)):
            pages = m.table[b].long().cpu()
            got = cache_rows(m.k_pools[layer].cpu(), pages, cfg.kv_heads, cfg.head_dim, 16,
                             key=True)[ctx + n:ctx + T]
            orig = cache_rows(m2.k_pools[layer].cpu(), pages, cfg.kv_heads, cfg.head_dim, 16,
                              key=True)[ctx + n:ctx + T]
            assert torch.equal(got, orig), (layer, b)
    del m2
    # per-row greedy samples + the ragged prefix acceptance (spec_decode.py:196-207)
    rows = [SimpleNamespace(params=SamplingParams(temperature=0.0)) for _ in range(B * T)]
    s = Sampler()
    s.reserve(B * T, cfg.vocab, max_tokens=64)
    tokens = s.sample(logits.clone(), rows).view(B, T)
    drafts = ids[:, 1:].clone()
    for b, n in enumerate(lengths):
        drafts[b, n - 1:] = -1          # no drafts past the request's prefix
    drafts[0, :2] = tokens[0, :2].cpu()  # request 0 accepts its whole prefix
    from snowllm_amd import ops
    acc = ops.spec_accept(tokens, drafts.cuda())
    torch.cuda.synchronize()
    want_tok = A.argmax(logits.cpu().numpy()).reshape(B, T)
    assert np.array_equal(tokens.cpu().numpy(), want_tok)
    want_acc = A.spec_accept(want_tok, drafts.numpy())
    assert np.array_equal(acc.cpu().numpy(), want_acc)
    assert all(int(a) <= n for a, n in zip(acc.cpu(), lengths)) and int(acc[0]) == 3


def test_batch_rows_limit(gpu):
    from snowllm_amd.errors import SnowLLMError
    from snowllm_amd.verify import VerifyModel
    with pytest.raises(SnowLLMError):
        VerifyModel(tiny("moe"), batch=29)   # 29 * 9 = 261 > 256 rows


@pytest.mark.parametrize("shape", ["batch4", "ragged"])
def test_fullsize_config4_batches(gpu, shape):
    """BASELINE config 4 (40 layers, 8K context, V = 151,936) with four requests of block 9,
    and with a ragged DSpark batch of prefix lengths 3 / 9 / 16: the first and last layer of
    every request under teacher forcing and its logits, against the CPU reference."""
    from snowllm_amd import layers as L
    from snowllm_amd.verify import CONFIG4, VerifyModel
    if shape == "batch4":
        cfg, B, lengths, contexts = CONFIG4, 4, [9] * 4, [8192, 8000, 5000, 8191]
    else:
        cfg, B, lengths, contexts = replace(CONFIG4, block=16), 3, [3, 9, 16], [8192, 8100, 7000]
    _say(f"config 4 {shape}: {B} requests, rows {lengths}")
    m = VerifyModel(cfg, seed=1, keep_raw={0, cfg.layers - 1}, batch=B)
    ids = torch.randint(0, cfg.vocab, (B, cfg.block), generator=torch.Generator().manual_seed(17))
    m.set_batch(ids, contexts, lengths)
    # tolerances of the single-block full-size test (tests/test_gpu_fullsize.py)
    check_layers(m, contexts, lengths, [0, cfg.layers - 1], (2e-3, 4e-3, 1.3e-2))
    check_logits(m, lengths, 5e-7)
    assert L.moe_sync_error() == 0
    del m
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("wt", [1, 2])
def test_dense_gemv_wide_rows_equal_row_tiles(gpu, wt):
    """The 16-bit GEMV over up to 256 rows (weights loaded once per four row tiles) gives each
    row the bits of the 16-row launches, and stays within the fp64 product's tolerance."""
    from snowllm_amd import layers as L, ops
    N, K = 2000, 2048
    g = torch.Generator(device="cuda").manual_seed(5 + wt)
    dt = torch.float16 if wt == 1 else torch.bfloat16
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(dt)
    ws_w = L.dense_shuffle(w)
    for M in (17, 36, 64, 100, 256):
        _say(f"dense_gemv wt={wt} M={M}")
        x = torch.randn(M, K, device="cuda", generator=g).bfloat16()
        out = torch.empty(M, N, device="cuda")
        if wt == 1:
            act = torch.empty(ops.gemm_kquant_a_ws_bytes(M, K), dtype=torch.uint8, device="cuda")
            ops.gemm_kquant_prepare_a(x, act)
        else:
            act = x
        L.dense_gemv(wt, ws_w, act, out, M, N, K)
        tiles = torch.empty_like(out)
        tb = ops.gemm_kquant_a_ws_bytes(16, K)
        for r0 in range(0, M, 16):
            n = min(16, M - r0)
            a = act[(r0 // 16) * tb:] if wt == 1 else x[r0:r0 + n]
            L.dense_gemv(wt, ws_w, a, tiles[r0:r0 + n], n, N, K)
        torch.cuda.synchronize()
        assert torch.equal(out, tiles), M
        want = x.double().cpu() @ w.double().cpu().T
        assert rel(out.cpu(), want) < (1e-3 if wt == 1 else 1e-5)
