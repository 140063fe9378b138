"""Pins of the CPU layer reference's composition (oracle/model.py: swiglu_ffn, qk_norm_rope,
moe_ffn, layer_forward, head_reference, inv_freq). CPU only.

The independent restatement is the local transformers library's Qwen3-Next decoder layer
(transformers/models/qwen3_next/modeling_qwen3_next.py: Qwen3NextDecoderLayer with full
attention and the sparse MoE block or the dense MLP, Qwen3NextRMSNorm, the partial rotary
embedding). It is the model family of the reference's Qwen3.5 layer
(snowllm/models/qwen3_5/qwen3_5.py:32-78, layers.py:75-228), written by other authors, in fp32
without the bf16 tensor boundaries of the oracle. Its attention gates the output with
sigmoid(gate rows of q_proj); those rows are set to zero here (gate 0.5) and o_proj doubled,
which is exact, so the layer is the ungated attention of the reference's configs.

Each comparison has a planted-mistake control: the same comparison run against an oracle with
one plausible slip (gate/up halves swapped, RoPE before the QK norm, the rotation's sign
flipped, the shared expert ungated) must fail, so the tolerance separates a right oracle from a wrong one.
"""
import math
from types import SimpleNamespace

import pytest
import torch

from oracle import model as RM
from oracle import quant as Q

tf_next = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
from transformers.cache_utils import DynamicCache  # noqa: E402
from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig  # noqa: E402

# oracle (bf16 tensor boundaries) vs transformers (fp32): observed <= 1.1e-2 (the MoE output,
# where bf16 rounding of the normed rows moves the router weights); planted slips >= 0.23
TOL = 2e-2
SLIP = 5e-2


def rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _cfg(kind):
    c = SimpleNamespace(hidden=256, heads=4, kv_heads=2, head_dim=64, rot_half=16,
                        rope_theta=1e4, eps=1e-6, attn_fmt=4, ffn_fmt=4, experts=0,
                        expert_ffn=0, topk=0, ffn=0)
    if kind == "moe":
        c.experts, c.expert_ffn, c.topk = 8, 256, 2
    else:
        c.ffn = 512
    c.moe = c.experts > 0
    c.qkv_n = (c.heads + 2 * c.kv_heads) * c.head_dim
    return c


def _weights(c, seed):
    g = torch.Generator().manual_seed(seed)
    H = c.hidden

    def gamma(n):   # far from 1 so that the order of norm and rotation matters
        return (1.0 + 0.5 * torch.randn(n, generator=g)).bfloat16()

    def q4k(n, k, s):
        return (None, None, torch.from_numpy(Q.make_q4_k_centered(n, k, seed * 31 + s, 2e-3)))

    lw = SimpleNamespace(in_norm=gamma(H), post_norm=gamma(H), q_norm=gamma(c.head_dim),
                         k_norm=gamma(c.head_dim), qkv=q4k(c.qkv_n, H, 0),
                         o=q4k(H, c.heads * c.head_dim, 1), raw={})
    if c.moe:
        E, F = c.experts, c.expert_ffn
        lw.raw["router"] = (torch.randn(E + 1, H, generator=g) * 2 / math.sqrt(H)).bfloat16()
        lw.gu, lw.dn = q4k(E * 2 * F, H, 2), q4k(E * H, F, 3)
        lw.sh_gu, lw.sh_dn = q4k(2 * F, H, 4), q4k(H, F, 5)
    else:
        lw.gu, lw.dn = q4k(2 * c.ffn, H, 2), q4k(H, c.ffn, 3)
    return lw


def _inputs(c, seed, T=5, ctx=24):
    g = torch.Generator().manual_seed(seed)
    x = RM.bf(torch.randn(T, c.hidden, generator=g))
    res = RM.bf(torch.randn(T, c.hidden, generator=g) * 2)
    k_ctx = RM.bf(torch.randn(ctx, c.kv_heads, c.head_dim, generator=g))
    v_ctx = RM.bf(torch.randn(ctx, c.kv_heads, c.head_dim, generator=g))
    return x, res, k_ctx, v_ctx


def _tf_layer(c, ref):
    """transformers' Qwen3-Next decoder layer carrying the oracle's dequantized weights."""
    rotary = 2 * c.rot_half / c.head_dim
    kw = dict(vocab_size=128, hidden_size=c.hidden, num_hidden_layers=1,
              num_attention_heads=c.heads, num_key_value_heads=c.kv_heads,
              head_dim=c.head_dim, rms_norm_eps=c.eps, layer_types=["full_attention"],
              rope_parameters={"rope_type": "default", "rope_theta": c.rope_theta,
                               "partial_rotary_factor": rotary})
    if c.moe:
        kw.update(num_experts=c.experts, num_experts_per_tok=c.topk, norm_topk_prob=True,
                  moe_intermediate_size=c.expert_ffn,
                  shared_expert_intermediate_size=c.expert_ffn, mlp_only_layers=[],
                  decoder_sparse_step=1, intermediate_size=c.expert_ffn)
    else:
        kw.update(num_experts=0, intermediate_size=c.ffn, mlp_only_layers=[0])
    cfg = Qwen3NextConfig(**kw)
    cfg._attn_implementation = "eager"
    cfg._experts_implementation = "eager"
    layer = tf_next.Qwen3NextDecoderLayer(cfg, 0).eval()
    H, D, Hq, Hkv = c.hidden, c.head_dim, c.heads, c.kv_heads
    with torch.no_grad():
        layer.input_layernorm.weight.copy_(ref.in_norm - 1)   # Qwen3NextRMSNorm scales by 1 + w
        layer.post_attention_layernorm.weight.copy_(ref.post_norm - 1)
        at = layer.self_attn
        at.q_norm.weight.copy_(ref.q_norm - 1)
        at.k_norm.weight.copy_(ref.k_norm - 1)
        wq = ref.qkv[:Hq * D].view(Hq, D, H)
        qp = torch.zeros(Hq, 2, D, H)
        qp[:, 0] = wq                                           # gate rows stay zero
        at.q_proj.weight.copy_(qp.view(2 * Hq * D, H))
        at.k_proj.weight.copy_(ref.qkv[Hq * D:(Hq + Hkv) * D])
        at.v_proj.weight.copy_(ref.qkv[(Hq + Hkv) * D:])
        at.o_proj.weight.copy_(2 * ref.o)                       # undo sigmoid(0) = 0.5
        if c.moe:
            E, F = c.experts, c.expert_ffn
            mlp = layer.mlp
            mlp.gate.weight.copy_(ref.router[:E])
            mlp.shared_expert_gate.weight.copy_(ref.router[E:E + 1])
            for e in range(E):
                gu, dn = ref.expert(e)
                mlp.experts.gate_up_proj[e].copy_(gu)
                mlp.experts.down_proj[e].copy_(dn)
            mlp.shared_expert.gate_proj.weight.copy_(ref.sh_gu[:F])
            mlp.shared_expert.up_proj.weight.copy_(ref.sh_gu[F:])
            mlp.shared_expert.down_proj.weight.copy_(ref.sh_dn)
        else:
            layer.mlp.gate_proj.weight.copy_(ref.gu[:c.ffn])
            layer.mlp.up_proj.weight.copy_(ref.gu[c.ffn:])
            layer.mlp.down_proj.weight.copy_(ref.dn)
    return layer, tf_next.Qwen3NextRotaryEmbedding(cfg)


def _tf_forward(c, ref, r1, k_ctx, v_ctx, positions, masks):
    """Layer output, residual after attention and attention output of the transformers
    layer; the context keys/values sit in its cache (already rotated, as the paged cache
    holds them)."""
    layer, rot = _tf_layer(c, ref)
    T, ctx = r1.shape[0], k_ctx.shape[0]
    taps = {}
    layer.post_attention_layernorm.register_forward_pre_hook(
        lambda m, a: taps.__setitem__("r2", a[0].detach().clone()))
    layer.self_attn.o_proj.register_forward_pre_hook(
        lambda m, a: taps.__setitem__("attn", 2 * a[0].detach().clone()))
    cache = DynamicCache()
    cache.update(k_ctx.float().permute(1, 0, 2)[None], v_ctx.float().permute(1, 0, 2)[None], 0)
    vis = RM.visibility(ctx, masks)
    mask = torch.zeros(1, 1, T, ctx + T).masked_fill(~vis[None, None], float("-inf"))
    cos, sin = rot(r1[None], positions[None])
    with torch.no_grad():
        out = layer(r1[None], position_embeddings=(cos, sin), attention_mask=mask,
                    past_key_values=cache)
    out = out[0] if isinstance(out, tuple) else out
    return out[0], taps["r2"][0], taps["attn"][0].view(T, c.heads, c.head_dim), (cos[0], sin[0])


def _run(kind, seed=1, masks=None):
    c = _cfg(kind)
    ref = RM.LayerRef(c, _weights(c, seed))
    x, res, k_ctx, v_ctx = _inputs(c, seed + 100)
    T, ctx = x.shape[0], k_ctx.shape[0]
    masks = masks or [(2 << t) - 1 for t in range(T)]
    depth = [bin(m).count("1") - 1 for m in masks]
    positions = torch.tensor([ctx + d for d in depth])
    r1 = RM.bf(x + res)
    tf_out, tf_r2, tf_attn, (tcos, tsin) = _tf_forward(c, ref, r1, k_ctx, v_ctx, positions, masks)
    cos, sin = RM.rope_tables(positions, RM.inv_freq(c.rope_theta, c.rot_half))
    # the rotary tables: the oracle's half tables are transformers' (cat(f, f)) first half
    assert torch.allclose(tcos[:, :c.rot_half], cos, atol=2e-6)
    assert torch.allclose(tcos[:, c.rot_half:], cos, atol=2e-6)
    assert torch.allclose(tsin[:, :c.rot_half], sin, atol=2e-6)

    def oracle():
        return RM.layer_forward(ref, x, res, cos, sin, k_ctx, v_ctx, masks)

    return c, ref, oracle, (tf_out, tf_r2, tf_attn)


def _errors(oracle_out, tf):
    x2, r2, attn, _ = oracle_out
    tf_out, tf_r2, tf_attn = tf
    return rel(attn, tf_attn), rel(r2, tf_r2), rel(x2 + r2, tf_out)


def test_inv_freq_matches_transformers_default_rope():
    for theta, D, half in ((1e6, 128, 64), (1e7, 256, 32), (1e4, 64, 16)):
        cfg = Qwen3NextConfig(head_dim=D, rope_parameters={
            "rope_type": "default", "rope_theta": theta, "partial_rotary_factor": 2 * half / D})
        want, _ = tf_next.Qwen3NextRotaryEmbedding.compute_default_rope_parameters(cfg)
        assert torch.equal(RM.inv_freq(theta, half), want.float()), (theta, D, half)


@pytest.mark.parametrize("kind", ["moe", "dense"])
def test_layer_forward_matches_transformers_qwen3_next(kind):
    c, ref, oracle, tf = _run(kind)
    out = oracle()
    e_attn, e_r2, e_out = _errors(out, tf)
    print(f"{kind}: attn {e_attn:.2e} r2 {e_r2:.2e} layer out {e_out:.2e}")
    assert e_attn < TOL and e_r2 < TOL and e_out < TOL
    if c.moe:   # routing of the oracle = transformers' top-k on the same logits
        assert out[3].shape == (5, c.topk)


def test_layer_forward_tree_mask_matches_transformers():
    parents = [-1, 0, 1, 0, 3]
    masks = []
    for i, p in enumerate(parents):
        masks.append((1 << i) | (masks[p] if p >= 0 else 0))
    _, _, oracle, tf = _run("moe", seed=2, masks=masks)
    e = _errors(oracle(), tf)
    assert max(e) < TOL, e


def test_planted_slips_fail_the_comparison(monkeypatch):
    """Each plausible slip in the oracle, planted on the CPU, moves the comparison far past
    the tolerance (so the passing comparisons above pin the right composition)."""
    good_swiglu, good_rope = RM.swiglu_ffn, RM.rope
    _, _, oracle, tf = _run("dense")

    def swapped(x, gu, dn, F):          # up rows taken as the gate
        return good_swiglu(x, torch.cat([gu[F:], gu[:F]]), dn, F)

    def rope_first(t, gamma, cos, sin, half, eps):   # rotate, then normalise
        r = good_rope(t, cos, sin, half)
        return RM.bf(r * torch.rsqrt(r.square().mean(-1, keepdim=True) + eps) * gamma)

    def sign_flip(x, cos, sin, half):   # rotation the other way
        return good_rope(x, cos, -sin, half)

    for name, fn in (("swiglu_ffn", swapped), ("qk_norm_rope", rope_first), ("rope", sign_flip)):
        with monkeypatch.context() as m:
            m.setattr(RM, name, fn)
            e = _errors(oracle(), tf)
        print(name, e)
        assert max(e) > SLIP, (name, e)
    # the MoE's shared expert taken ungated
    _, ref, oracle, tf = _run("moe")
    good_route = RM.route
    with monkeypatch.context() as m:
        m.setattr(RM, "route", lambda lg, E, K: (*good_route(lg, E, K)[:2], torch.ones(lg.shape[0])))
        e = _errors(oracle(), tf)
    assert e[2] > SLIP, e


def test_zero_attention_and_experts_leave_the_residual_stream():
    """With O = 0 the attention update adds nothing (r2 = r1); with every expert and the
    shared expert zero the FFN output is zero, so the next layer sees r2 unchanged."""
    c = _cfg("moe")
    ref = RM.LayerRef(c, _weights(c, 4))
    x, res, k_ctx, v_ctx = _inputs(c, 5)
    ref.o = torch.zeros_like(ref.o)
    ref.sh_gu, ref.sh_dn = torch.zeros_like(ref.sh_gu), torch.zeros_like(ref.sh_dn)
    zero = (torch.zeros(2 * c.expert_ffn, c.hidden), torch.zeros(c.hidden, c.expert_ffn))
    ref._experts = {e: zero for e in range(c.experts)}
    T = x.shape[0]
    cos, sin = RM.rope_tables(torch.arange(24, 24 + T), RM.inv_freq(c.rope_theta, c.rot_half))
    x2, r2, _, _ = RM.layer_forward(ref, x, res, cos, sin, k_ctx, v_ctx,
                                    [(2 << t) - 1 for t in range(T)])
    assert torch.equal(r2, RM.bf(x + res))
    assert torch.equal(x2, torch.zeros_like(x2))


def test_one_expert_at_weight_one_is_a_dense_swiglu():
    """top-1 routing renormalises the chosen expert's weight to exactly 1; a shared-gate
    logit of -inf makes sigmoid 0, so the MoE equals that expert's dense SwiGLU."""
    c = _cfg("moe")
    c.topk = 1
    ref = RM.LayerRef(c, _weights(c, 6))
    g = torch.Generator().manual_seed(7)
    h2 = RM.bf(torch.randn(3, c.hidden, generator=g))
    logits = torch.randn(3, c.experts + 1, generator=g)
    logits[:, c.experts] = float("-inf")
    out, ids = RM.moe_ffn(ref, h2, logits)
    for t in range(3):
        e = int(logits[t, :c.experts].argmax())
        assert int(ids[t, 0]) == e
        gu, dn = ref.expert(e)
        assert torch.equal(out[t], RM.swiglu_ffn(h2[t:t + 1], gu, dn, c.expert_ffn)[0])


def test_swiglu_known_values_gate_rows_first():
    """x = e_0 picks column 0 of the packed [gate; up] matrix: g, u known, down = identity,
    so the output is bf16(silu(g) * u) with silu taken of the gate rows."""
    F = 8
    g = torch.tensor([-3.0, -1.0, -0.5, 0.0, 0.25, 1.0, 2.0, 4.0])
    u = torch.tensor([1.0, -2.0, 0.5, 3.0, -1.0, 0.75, -0.25, 2.0])
    gu = torch.zeros(2 * F, F)
    gu[:F, 0], gu[F:, 0] = g, u
    x = torch.zeros(1, F)
    x[0, 0] = 1.0
    out = RM.swiglu_ffn(x, gu, torch.eye(F), F)[0]
    want = (torch.nn.functional.silu(g.double()) * u.double()).float().bfloat16().float()
    assert torch.equal(out, want)
    assert not torch.equal(out, (torch.nn.functional.silu(u.double()) * g.double()).float()
                           .bfloat16().float())


def test_head_reference_matches_explicit_formula_and_transformers_norm():
    g = torch.Generator().manual_seed(8)
    T, H, V = 4, 256, 96
    x = RM.bf(torch.randn(T, H, generator=g))
    res = RM.bf(torch.randn(T, H, generator=g))
    gamma = (1 + 0.3 * torch.randn(H, generator=g)).bfloat16()
    head = (0.05 * torch.randn(V, H, generator=g)).half()
    got = RM.head_reference(x, res, gamma, head, 1e-6)
    norm = tf_next.Qwen3NextRMSNorm(H, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(gamma.float() - 1)
        want = norm(x + res) @ head.float().T
    assert rel(got, want) < 1e-2
    # explicit: bf16 residual sum, RMS norm with gamma, bf16 rounding, fp64 product
    r = (x + res).bfloat16().double()
    h = (r / (r.square().mean(-1, keepdim=True) + 1e-6).sqrt() * gamma.double()).float().bfloat16()
    assert rel(got, (h.double() @ head.double().T).float()) < 1e-6
