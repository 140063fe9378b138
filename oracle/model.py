"""CPU reference of one verify-step layer -- TEST INFRASTRUCTURE ONLY.

torch fp32 arithmetic with bf16 rounding at the tensor boundaries of the reference's Qwen3.5
layer (snowllm/models/qwen3_5/qwen3_5.py:32-78, layers.py:75-228):
  residual update, RMSNorm (x * rsqrt(mean(x^2) + eps) * gamma; gamma stored as 1 + w,
  snowllm/models/qwen3_5/qwen3_5_weights.py:39-40), QKV projection, per-head QK RMSNorm and
  rotate-half RoPE rounded once (tests/test_lfm2_dspark_reference.py:16-27), masked softmax
  attention (tests/test_lfm2_long_attention.py:36-44), O projection, and either a SwiGLU MLP
  or the Qwen-Next MoE (softmax over routed experts in fp32, top-k, renormalised, plus the
  sigmoid-gated shared expert: transformers models/qwen3_next/modeling_qwen3_next.py).
Weights are dequantized with oracle.quant from the raw GGUF bytes the GPU model was built from.
"""
import numpy as np
import torch

from oracle import quant as Q


def bf(x):
    return x.to(torch.bfloat16).float()


def rmsnorm(x, gamma, eps):
    return bf(x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps) * gamma.float())


def rope(x, cos, sin, half):
    """x [T, heads, D] fp32; rotates dims [0, 2*half) in (i, i + half) pairs."""
    out = x.clone()
    a, b = x[..., :half], x[..., half:2 * half]
    c, s = cos[:, None, :], sin[:, None, :]
    out[..., :half] = a * c - b * s
    out[..., half:2 * half] = b * c + a * s
    return out


def dequant_raw(raw, fmt, n, k):
    return torch.from_numpy(Q.dequant(raw.cpu().numpy(), fmt, n, k))


def linear(x, w):
    """bf16 output of x [T, K] @ w[N, K]^T computed in float64."""
    return bf((x.double() @ w.double().T).float())


def cache_rows(pool, pages, heads, dim, page, *, key):
    """Paged pool -> dense rows [len, heads, dim] (tests/test_lfm2_dspark_reference.py:30-36:
    K [blocks, Hkv, d/16, page, 16], V [blocks, Hkv, page/4, d, 4])."""
    x = pool.view(torch.bfloat16)
    if key:
        x = x.view(-1, heads, dim // 16, page, 16)[pages].permute(0, 3, 1, 2, 4)
    else:
        x = x.view(-1, heads, page // 4, dim, 4)[pages].permute(0, 2, 4, 1, 3)
    return x.reshape(-1, heads, dim)


class LayerRef:
    """Dequantized weights of one layer (CPU). Routed experts are dequantized when first
    used (the reference's CPU path only touches the experts a block routes to)."""

    def __init__(self, cfg, lw):
        c = cfg
        H = c.hidden
        self.cfg = c
        self.in_norm = lw.in_norm.cpu().float()
        self.post_norm = lw.post_norm.cpu().float()
        self.q_norm = lw.q_norm.cpu().float()
        self.k_norm = lw.k_norm.cpu().float()
        # a layer's own formats where they differ from the config's (0 or absent: the config's)
        own = lambda obj, name: getattr(obj, name, 0) or 0  # noqa: E731
        v = getattr(lw, "v", None)
        if v is None:
            self.qkv = dequant_raw(lw.qkv[2], own(lw, "qkv_fmt") or c.attn_fmt, c.qkv_n, H)
        else:   # q|k rows, then the V rows in their own format
            nqk = (c.heads + c.kv_heads) * c.head_dim
            self.qkv = torch.cat([dequant_raw(lw.qkv[2], own(lw, "qkv_fmt") or c.attn_fmt, nqk, H),
                                  dequant_raw(v[2], lw.v_fmt, c.qkv_n - nqk, H)])
        self.o = dequant_raw(lw.o[2], own(lw, "o_fmt") or c.attn_fmt, H, c.heads * c.head_dim)
        self.gu_fmt = own(lw, "gu_fmt") or c.ffn_fmt
        self.dn_fmt = own(lw, "dn_fmt") or own(c, "down_fmt") or c.ffn_fmt
        if c.moe:
            F = c.expert_ffn
            self.router = lw.raw["router"].cpu().float()
            self._gu_raw = lw.gu[2].cpu()
            self._dn_raw = lw.dn[2].cpu()
            self._experts = {}
            self.sh_gu = dequant_raw(lw.sh_gu[2], self.gu_fmt, 2 * F, H)
            self.sh_dn = dequant_raw(lw.sh_dn[2], self.dn_fmt, H, F)
        else:
            self.gu = dequant_raw(lw.gu[2], self.gu_fmt, 2 * c.ffn, H)
            self.dn = dequant_raw(lw.dn[2], self.dn_fmt, H, c.ffn)

    def expert(self, e):
        """(gate_up [2F, H], down [H, F]) of routed expert e."""
        if e not in self._experts:
            c = self.cfg
            H, F = c.hidden, c.expert_ffn
            gb = self._gu_raw.numel() // c.experts
            db = self._dn_raw.numel() // c.experts
            gu = dequant_raw(self._gu_raw[e * gb:(e + 1) * gb], self.gu_fmt, 2 * F, H)
            dn = dequant_raw(self._dn_raw[e * db:(e + 1) * db], self.dn_fmt, H, F)
            self._experts[e] = (gu, dn)
        return self._experts[e]


def inv_freq(theta, rot_half):
    """RoPE inverse frequencies theta^(-j / rot_half), j < rot_half: rotary dims 2*rot_half
    in (i, i + rot_half) pairs (snowllm/ops/rope.py:11-24 takes them as a tensor)."""
    return 1.0 / (theta ** (torch.arange(rot_half, dtype=torch.float32) / rot_half))


def swiglu_ffn(x, gu, dn, F):
    """SwiGLU over packed gate/up rows (gate rows first: snowllm/models/qwen3_5/
    qwen3_5_weights.py:216,233 concatenates gate_proj then up_proj): down(silu(g) * u)."""
    g = linear(x, gu[:F])
    u = linear(x, gu[F:])
    act = bf(g / (1 + torch.exp(-g)) * u)
    return linear(act, dn)


def visibility(ctx, masks):
    """[T, ctx + T] bool: row t sees the context and block row j iff bit j of masks[t]."""
    T = len(masks)
    vis = torch.zeros(T, ctx + T, dtype=torch.bool)
    vis[:, :ctx] = True
    for t in range(T):
        for j in range(T):
            if (masks[t] >> j) & 1:
                vis[t, ctx + j] = True
    return vis


def masked_attention(q, keys, vals, vis, scale):
    """GQA softmax attention in float64: q [T, Hq, D], keys/vals [L, Hkv, D], vis [T, L]."""
    T, Hq, D = q.shape
    Hkv = keys.shape[1]
    G = Hq // Hkv
    attn = torch.empty(T, Hq, D)
    for hk in range(Hkv):
        qs = q[:, hk * G:(hk + 1) * G].double()
        s = torch.einsum("tgd,ld->tgl", qs, keys[:, hk].double()) * scale
        s = s.masked_fill(~vis[:, None, :], float("-inf"))
        attn[:, hk * G:(hk + 1) * G] = torch.einsum("tgl,ld->tgd", s.softmax(-1), vals[:, hk].double()).float()
    return attn


def route(logits, E, K):
    """Qwen-Next routing: softmax over the E routed logits, top-K, renormalised; sigmoid of
    column E is the shared expert's gate."""
    probs = torch.softmax(logits[:, :E], -1)
    w, ids = torch.topk(probs, K, dim=-1)
    return ids, w / w.sum(-1, keepdim=True), torch.sigmoid(logits[:, E])


def qk_norm_rope(t, gamma, cos, sin, half, eps):
    """Per-head RMSNorm, then RoPE, rounded once to bf16 (snowllm/ops/attention_full.py:
    736-784 normalises before it rotates; tests/test_lfm2_dspark_reference.py:16-27)."""
    n = t * torch.rsqrt(t.square().mean(-1, keepdim=True) + eps) * gamma
    return bf(rope(n, cos, sin, half))


def moe_ffn(ref, h2, logits):
    """Qwen-Next MoE of the normed rows h2 [T, H] given router logits [T, E + 1]: each row's
    top-K experts weighted by the renormalised softmax, plus the shared expert weighted by
    sigmoid(logit E); every expert output is a bf16 tensor, the weighted sum is rounded once.
    Returns (output [T, H], routed ids [T, K])."""
    c = ref.cfg
    E, F, K = c.experts, c.expert_ffn, c.topk
    T = h2.shape[0]
    ids, w, gate = route(logits, E, K)
    out = torch.zeros(T, c.hidden)
    for t in range(T):
        acc = torch.zeros(c.hidden)
        for kk in range(K):
            gu, dn = ref.expert(int(ids[t, kk]))
            y = swiglu_ffn(h2[t:t + 1], gu, dn, F)[0]
            acc += y * w[t, kk]
        sh = swiglu_ffn(h2[t:t + 1], ref.sh_gu, ref.sh_dn, F)[0]
        acc += sh * gate[t]
        out[t] = acc
    return bf(out), ids


def layer_forward(ref, x, res, cos, sin, k_ctx, v_ctx, masks):
    """One layer. x: block input [T, H] (bf16 values), res: residual stream or None,
    k_ctx/v_ctx: context keys/values [ctx, Hkv, D]; masks: per-row visibility bits over the
    block. Returns (FFN output x', the residual stream after the attention update r2 = o + r1,
    attention output, routed ids or None). The next layer's input is x' with residual r2."""
    c = ref.cfg
    T = x.shape[0]
    D, Hq, Hkv = c.head_dim, c.heads, c.kv_heads
    r1 = x if res is None else bf(x + res)
    h = rmsnorm(r1, ref.in_norm, c.eps)
    proj = linear(h, ref.qkv)
    q = proj[:, :Hq * D].view(T, Hq, D)
    k = proj[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = proj[:, (Hq + Hkv) * D:].view(T, Hkv, D)

    q = qk_norm_rope(q, ref.q_norm, cos, sin, c.rot_half, c.eps)
    k = qk_norm_rope(k, ref.k_norm, cos, sin, c.rot_half, c.eps)
    keys = torch.cat([k_ctx.float(), k])
    vals = torch.cat([v_ctx.float(), v])
    attn = bf(masked_attention(q, keys, vals, visibility(k_ctx.shape[0], masks), D ** -0.5))
    o = linear(attn.view(T, -1), ref.o)
    r2 = bf(o + r1)
    h2 = rmsnorm(r2, ref.post_norm, c.eps)
    routing = None
    if c.moe:
        logits = (h2.double() @ ref.router.double().T).float()
        x2, routing = moe_ffn(ref, h2, logits)
    else:
        x2 = swiglu_ffn(h2, ref.gu, ref.dn, c.ffn)
    return x2, r2, attn, routing


def rope_tables(positions, inv_freq):
    """cos/sin of pos * inv_freq with the angle rounded to fp32 (as the tables are built)."""
    ang = positions.float()[:, None] * inv_freq.float()[None, :]
    return torch.cos(ang.double()).float(), torch.sin(ang.double()).float()


def head_reference(x, res, final_norm, lm_head, eps):
    """Final norm + fp16 LM head -> f32 logits [T, V]."""
    r = bf(x + res)
    h = rmsnorm(r, final_norm.float(), eps)
    return (h.double() @ lm_head.double().T).float()
