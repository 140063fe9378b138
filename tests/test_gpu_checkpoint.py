"""A verify model read from a GGUF checkpoint (snowllm_amd.checkpoint, after the reference's
snowllm/checkpoint/gguf/source.py and models/qwen3_5/qwen3_5_weights.py) against the model
whose GGUF blocks were written: the expert, router and projection repacks from the on-disk
layout give the same bytes as the repack of the generated matrices, the forward gives the same
logits bit for bit, and the Q4_K embedding and k-quant head match the oracle's dequantisation."""
import numpy as np
import pytest
import torch

from oracle import model as RM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def tiny(kind, **kw):
    from snowllm_amd.verify import VerifyConfig
    base = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rot_half=32,
                rope_theta=1e4, vocab=2048, context=300, block=9)
    base.update(kw)
    if kind == "moe":
        return VerifyConfig("tiny_moe", experts=16, expert_ffn=256, topk=4, **base)
    return VerifyConfig("tiny_dense", ffn=512, **base)


@pytest.fixture
def default_geometry():
    from snowllm_amd import ops
    yield
    ops.select_geometry(0)


def rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


CASES = [
    # kind, config overrides, parts of the checkpoint
    ("moe", {}, 1),
    ("moe", {"attn_fmt": 8}, 3),
    ("dense", {"attn_fmt": 8}, 1),
    # the other k-quants of a Q4_K_M / UD-Q4_K_XL file
    ("moe", {"attn_fmt": 6}, 1),
    ("dense", {"attn_fmt": 5, "ffn_fmt": 6}, 2),
    # experts: Q4_K with Q6_K down (Q4_K_M), Q5_K with Q6_K down (Q5_K_M), all Q6_K
    ("moe", {"down_fmt": 6}, 1),
    ("moe", {"attn_fmt": 5, "ffn_fmt": 5, "down_fmt": 6}, 2),
    ("moe", {"attn_fmt": 6, "ffn_fmt": 6}, 1),
    # attn_v wider than attn_q / attn_k: the split projection
    ("moe", {"v_fmt": 6, "down_fmt": 6}, 1),
    ("dense", {"attn_fmt": 8, "v_fmt": 5}, 1),
]


@pytest.mark.parametrize("kind,over,parts", CASES)
def test_gguf_model_matches_its_source(gpu, tmp_path, default_geometry, kind, over, parts):
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    from snowllm_amd.checkpoint import load_gguf, model_tensors, save_gguf
    from snowllm_amd.verify import VerifyModel
    cfg = tiny(kind, **over)
    _say(f"checkpoint {cfg.name} {over} parts={parts}: source model")
    m = VerifyModel(cfg, seed=3, keep_raw=True)
    path = save_gguf(tmp_path / "m.gguf", cfg, model_tensors(m), parts=parts)
    _say("  load")
    lm = load_gguf(path, context=cfg.context, block=cfg.block, seed=3)
    assert (lm.cfg.layers, lm.cfg.hidden, lm.cfg.experts, lm.cfg.ffn, lm.cfg.attn_fmt,
            lm.cfg.ffn_fmt) == (cfg.layers, cfg.hidden, cfg.experts, cfg.ffn, cfg.attn_fmt,
                                cfg.ffn_fmt)
    for i, (a, b) in enumerate(zip(m.layers, lm.layers)):
        names = ["qkv", "o", "gu", "dn"] + (["sh_gu", "sh_dn"] if cfg.moe else [])
        assert (a.v is None) == (b.v is None) and a.v_fmt == b.v_fmt, i
        names += ["v"] if a.v is not None else []
        for n in names:
            wa, wb = getattr(a, n), getattr(b, n)
            # the last 4 quant bytes are read slack, never written
            assert torch.equal(wa[0][:-4], wb[0][:-4]) and torch.equal(wa[1], wb[1]), (i, n)
        for n in ("in_norm", "post_norm", "q_norm", "k_norm"):
            assert torch.equal(getattr(a, n), getattr(b, n)), (i, n)
        if cfg.moe:
            assert torch.equal(a.router, b.router), i
    assert torch.equal(lm.final_norm, m.final_norm)
    assert torch.equal(lm.embed, m.embed.bfloat16())
    # the checkpoint's head is bf16 (the reference reads 16-bit matrices as bf16): give the
    # source model the same head, then the two forwards must agree bit for bit
    m.lm_head = ops.lm_head_shuffle_weight(m.lm_head_raw.bfloat16())
    m.head_wt = L.WT_BF16
    n = cfg.vocab * cfg.hidden * 2   # the repacked bytes; the allocation has slack behind them
    assert torch.equal(lm.lm_head[:n], m.lm_head[:n])
    ids = torch.randint(0, cfg.vocab, (cfg.block,), generator=torch.Generator().manual_seed(5))
    for model in (m, lm):
        model.set_block(ids)
    _say("  forward both")
    want = m.forward().clone()
    got = lm.forward().clone()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # and the bf16 head against the oracle on the loaded model's own final hidden state
    ref = RM.head_reference(lm.x.float().cpu(), lm.layer_residual.float().cpu(),
                            lm.final_norm.cpu(), m.lm_head_raw.bfloat16().cpu(), cfg.eps)
    e = rel(got.cpu(), ref)
    _say(f"  bf16 head logits rel L2 {e:.2e}")
    assert e < 1e-6


def test_q4k_embedding_and_kquant_head(gpu, tmp_path, default_geometry):
    from snowllm_amd.checkpoint import load_gguf, model_tensors, save_gguf
    from snowllm_amd.verify import HEAD_KQUANT, VerifyModel, gguf_random
    cfg = tiny("moe")
    _say("checkpoint with a Q4_K embedding and a Q8_0 head")
    m = VerifyModel(cfg, seed=4, keep_raw=True)
    V, H = cfg.vocab, cfg.hidden
    emb = gguf_random(4, V, H, seed=21, centered=True).cpu()
    head = gguf_random(8, V, H, seed=22).cpu()
    tensors = [t for t in model_tensors(m) if t[0] not in ("token_embd.weight", "output.weight")]
    tensors += [("token_embd.weight", (V, H), "Q4_K", emb), ("output.weight", (V, H), "Q8_0", head)]
    lm = load_gguf(save_gguf(tmp_path / "q.gguf", cfg, tensors), context=cfg.context,
                   block=cfg.block, seed=4)
    assert lm.embed_q4k and lm.head_wt == HEAD_KQUANT and lm.head_fmt == 8
    ids = torch.tensor([0, 1, V - 1, 17, 17, 1000, 3, 2047, 512])
    lm.set_block(ids)
    lm.forward(upto_layer=0)
    torch.cuda.synchronize()
    table = torch.from_numpy(Q.dequant_q4_k(emb.numpy(), V, H))
    assert torch.equal(lm.x.cpu(), table[ids].bfloat16())
    logits = lm.forward().clone()
    torch.cuda.synchronize()
    ref = RM.head_reference(lm.x.float().cpu(), lm.layer_residual.float().cpu(),
                            lm.final_norm.cpu(), torch.from_numpy(Q.dequant_q8_0(head.numpy(), V, H)),
                            cfg.eps)
    e = rel(logits.cpu(), ref)
    _say(f"  Q8_0 head logits rel L2 {e:.2e}")
    assert e < 1e-5


def test_tied_head(gpu, tmp_path, default_geometry):
    """No output.weight: the head is the embedding, read as bf16 (qwen3_5_weights.py:415-421)."""
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    from snowllm_amd.checkpoint import load_gguf, model_tensors, save_gguf
    from snowllm_amd.verify import VerifyModel
    cfg = tiny("dense")
    _say("checkpoint with a tied head")
    m = VerifyModel(cfg, seed=6, keep_raw=True)
    lm = load_gguf(save_gguf(tmp_path / "t.gguf", cfg, model_tensors(m, tied=True)),
                   context=cfg.context, block=cfg.block, seed=6)
    assert lm.head_wt == L.WT_BF16
    n = cfg.vocab * cfg.hidden * 2
    assert torch.equal(lm.lm_head[:n], ops.lm_head_shuffle_weight(m.embed.bfloat16())[:n])


def test_gather_embedding_q4_k_equals_dequant(gpu):
    """snowllm_gather_embedding_q4_k bit for bit against the oracle's Q4_K dequantisation
    rounded to bf16; ids outside the table read row 0."""
    from snowllm_amd import ops
    from snowllm_amd.verify import gguf_random
    for V, H, seed in ((300, 256, 1), (1000, 2048, 2), (151936, 2048, 3)):
        _say(f"gather_embedding_q4_k V={V} H={H}")
        raw = gguf_random(4, V, H, seed=seed).cpu().numpy()
        ids = torch.tensor([0, V - 1, 5, -1, V, 2 * V, 7, V // 2], dtype=torch.int64)
        out = torch.empty(len(ids), H, dtype=torch.bfloat16, device="cuda")
        w = torch.from_numpy(np.ascontiguousarray(raw)).cuda().view(V, H // 256 * 144)
        ops.gather_embedding_q4_k(ids.cuda(), w, out)
        torch.cuda.synchronize()
        rows = ids.clone()
        rows[(rows < 0) | (rows >= V)] = 0
        blk = raw.reshape(V, -1)[rows.numpy()].reshape(-1)
        want = torch.from_numpy(Q.dequant_q4_k(blk, len(ids), H)).bfloat16()
        assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("head_q", ["Q6_K", "Q5_K"])
def test_q6k_q5k_head(gpu, tmp_path, default_geometry, head_q):
    """A Q6_K (Q4_K_M's usual output.weight) or Q5_K head read from the checkpoint: the logits
    against the oracle's decode of the same blocks."""
    from snowllm_amd.checkpoint import load_gguf, model_tensors, save_gguf
    from snowllm_amd.verify import HEAD_KQUANT, VerifyModel, gguf_random
    fmt = {"Q5_K": 5, "Q6_K": 6}[head_q]
    cfg = tiny("dense")
    _say(f"checkpoint with a {head_q} head")
    m = VerifyModel(cfg, seed=5, keep_raw=True)
    V, H = cfg.vocab, cfg.hidden
    head = gguf_random(fmt, V, H, seed=23).cpu()
    tensors = [t for t in model_tensors(m) if t[0] != "output.weight"]
    tensors += [("output.weight", (V, H), head_q, head)]
    lm = load_gguf(save_gguf(tmp_path / "h.gguf", cfg, tensors), context=cfg.context,
                   block=cfg.block, seed=5)
    assert lm.head_wt == HEAD_KQUANT and lm.head_fmt == fmt
    lm.set_block(torch.arange(cfg.block) * 11)
    logits = lm.forward().clone()
    torch.cuda.synchronize()
    ref = RM.head_reference(lm.x.float().cpu(), lm.layer_residual.float().cpu(),
                            lm.final_norm.cpu(), torch.from_numpy(Q.dequant(head.numpy(), fmt, V, H)),
                            cfg.eps)
    e = rel(logits.cpu(), ref)
    _say(f"  {head_q} head logits rel L2 {e:.2e}")
    assert e < 1e-3
