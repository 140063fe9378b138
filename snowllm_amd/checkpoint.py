"""The verify model's weights from a GGUF checkpoint.

Follows the reference's GGUF path for the parts this build computes:
  - shapes from the "{arch}.*" metadata (snowllm/checkpoint/gguf/names.py:37-100);
  - the tensor names of a decoder layer and the top level (names.py:166-205);
  - reads (snowllm/checkpoint/gguf/source.py:219-346): norm weights as float32 minus one, to
    bf16, and the model adds the one back in float32 (models/qwen3_5/qwen3_5_weights.py:39-40),
    so a norm is bf16(1 + bf16(w - 1)); 16-bit and float matrices are read as bf16;
  - k-quant projections as raw GGUF blocks: q|k|v concatenated into one [q + 2 kv, H] weight
    (qwen3_5_weights.py:80-110, source.py:294-307), the experts' stacks through
    moe_kquant_shuffle_gate_up / _down (qwen3_5_weights.py:307-335, ops/moe.py:136-162), the
    shared expert as a one-expert stack (qwen3_5_weights.py:296-304), the router as
    [ffn_gate_inp; ffn_gate_inp_shexp] bf16 (qwen3_5_weights.py:333-335);
  - the embedding as bf16 or Q4_K blocks and the head as bf16 or Q4_K / Q5_K / Q6_K / Q8_0
    blocks, tied to the embedding when the file has no output.weight
    (qwen3_5_weights.py:405-421).

Scope: every layer must be full GQA attention with QK-norm and no output gate, followed by a
SwiGLU MLP or a routed MoE with a shared expert whose width equals the experts'; attention and
dense matrices in Q4_K, Q5_K, Q6_K or Q8_0 (the formats the reference's GEMM takes, snowllm/
checkpoint/gguf/source.py:263-272), with q/k in one format and v in the same or another
(qwen3_5_weights.py:95-109), gate/up in one and down in any;
the experts' gate/up in Q4_K, Q5_K or Q6_K and their down in the same format or a wider one
(Q4_K_M files store some layers' ffn_down_exps as Q6_K), the shared expert in the routed
experts' formats. Formats may change from layer to layer.
Anything else raises SnowLLMError naming the tensor; nothing falls back to another path.
"""
import torch

from . import layers as Lops
from . import ops
from ._capi import SnowLLMError
from .gguf import GGUF, KQUANT_FORMAT
from .verify import (HEAD_KQUANT, LayerWeights, VerifyConfig, VerifyModel, geometry_fields)

_FLOAT = ("F32", "F16", "BF16")


def _int(g: GGUF, key, default=None):
    v = g.get(key, default)
    return None if v is None else int(v)


def config_from_gguf(g: GGUF, *, context: int, block: int, tree_parents=(),
                     name: str = None) -> VerifyConfig:
    """The VerifyConfig of a checkpoint (names.py:37-100), checked against what this build
    computes."""
    if g.arch not in ARCHITECTURES:
        raise SnowLLMError(f"{g.path.name} is a {g.arch!r} checkpoint; this build's verify step "
                           f"reads {' and '.join(map(repr, ARCHITECTURES))} checkpoints")
    if (g.arch == "qwen35moe") != bool(_int(g, "{arch}.expert_count", 0)):
        raise SnowLLMError(f"{g.path.name}: a {g.arch!r} checkpoint "
                           f"{'without' if g.arch == 'qwen35moe' else 'with'} experts")
    nextn = _int(g, "{arch}.nextn_predict_layers", 0) or 0
    layers = int(g.need("{arch}.block_count")) - nextn
    interval = _int(g, "{arch}.full_attention_interval", 1)
    if interval != 1:
        raise SnowLLMError(f"{g.path.name}: full attention every {interval} layers; the other "
                           f"layers are linear attention, which this build does not compute")
    hidden = int(g.need("{arch}.embedding_length"))
    heads = int(g.need("{arch}.attention.head_count"))
    kv_heads = int(g.need("{arch}.attention.head_count_kv"))
    head_dim = _int(g, "{arch}.attention.key_length", hidden // heads)
    if _int(g, "{arch}.attention.value_length", head_dim) != head_dim:
        raise SnowLLMError(f"{g.path.name}: key and value head sizes differ")
    rope_dim = _int(g, "{arch}.rope.dimension_count", head_dim)
    theta = float(g.get("{arch}.rope.freq_base", 10000.0))
    eps = float(g.need("{arch}.attention.layer_norm_rms_epsilon"))
    vocab = g["token_embd.weight"].shape[0]
    experts = _int(g, "{arch}.expert_count", 0) or 0
    fields = dict(layers=layers, hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                  rot_half=rope_dim // 2, rope_theta=theta, vocab=vocab, context=context,
                  block=block, tree_parents=tuple(tree_parents), eps=eps)
    if experts:
        F = int(g.need("{arch}.expert_feed_forward_length"))
        shared = _int(g, "{arch}.expert_shared_feed_forward_length", F)
        if shared != F:
            raise SnowLLMError(f"{g.path.name}: shared expert width {shared} differs from the "
                               f"experts' {F}; this build runs both in one launch of width F")
        fmt = _expert_fmt(g, "blk.0.ffn_gate_exps.weight")
        fields.update(experts=experts, expert_ffn=F,
                      topk=int(g.need("{arch}.expert_used_count")), ffn_fmt=fmt)
    else:
        fields.update(ffn=int(g.need("{arch}.feed_forward_length")),
                      ffn_fmt=_kfmt(g, "blk.0.ffn_gate.weight"))
    fields["attn_fmt"] = _kfmt(g, "blk.0.attn_q.weight")
    return VerifyConfig(name or f"gguf:{g.path.name}", **fields)


# the reference's architecture names (snowllm/checkpoint/gguf/names.py:16-17): MoE, dense
ARCHITECTURES = ("qwen35moe", "qwen35")
# expert formats the MoE kernels compute: gate/up in one of these, down in the same or a wider
EXPERT_FORMATS = (KQUANT_FORMAT["Q4_K"], KQUANT_FORMAT["Q5_K"], KQUANT_FORMAT["Q6_K"])


def _expert_fmt(g: GGUF, name: str) -> int:
    fmt = _kfmt(g, name)
    if fmt not in EXPERT_FORMATS:
        raise SnowLLMError(f"{g.path.name}: {name} is {g[name].quant.name}; this build's MoE "
                           f"kernels compute Q4_K, Q5_K and Q6_K experts")
    return fmt


def _kfmt(g: GGUF, name: str) -> int:
    q = g[name].quant.name
    if q not in KQUANT_FORMAT:
        raise SnowLLMError(f"{g.path.name}: {name} is {q}; this build computes Q4_K, Q5_K, "
                           f"Q6_K and Q8_0 matrices")
    return KQUANT_FORMAT[q]


def _shape(g: GGUF, name: str, *shape):
    got = g[name].shape
    if tuple(got) != tuple(shape):
        raise SnowLLMError(f"{g.path.name}: {name} is {tuple(got)}, the config needs {shape}")


def _blocks(g: GGUF, names, fmt=None):
    """Raw GGUF blocks of one or more tensors in one format, concatenated, on the GPU."""
    fmts = {_kfmt(g, n) for n in names}
    if len(fmts) != 1 or (fmt is not None and fmts != {fmt}):
        raise SnowLLMError(f"{g.path.name}: {', '.join(names)} must share one k-quant format "
                           f"(have {sorted(g[n].quant.name for n in names)})")
    parts = [g.payload(n) for n in names]
    host = parts[0] if len(parts) == 1 else torch.cat(parts)
    return host.to("cuda"), fmts.pop()


def _bf16(g: GGUF, name: str) -> torch.Tensor:
    """A float tensor read as bf16 on the GPU (source.py:329-336)."""
    if g[name].quant.name not in _FLOAT:
        raise SnowLLMError(f"{g.path.name}: {name} is {g[name].quant.name}; expected F32/F16/BF16")
    return g.tensor(name).to("cuda").to(torch.bfloat16).contiguous()


def norm_weight(w: torch.Tensor) -> torch.Tensor:
    """A stored norm weight as the model applies it: bf16(1 + float(bf16(w - 1)))
    (source.py:338-340 reads w - 1 into bf16, qwen3_5_weights.py:39-40 adds the one back)."""
    w = w.float().reshape(-1)
    return (1.0 + (w - 1.0).to(torch.bfloat16).float()).to(torch.bfloat16).contiguous()


def _gamma(g: GGUF, name: str) -> torch.Tensor:
    if g[name].quant.name not in _FLOAT:
        raise SnowLLMError(f"{g.path.name}: {name} is {g[name].quant.name}; expected F32/F16/BF16")
    return norm_weight(g.tensor(name)).to("cuda")


def _layer(g: GGUF, cfg: VerifyConfig, i: int) -> LayerWeights:
    p = f"blk.{i}."
    H, d = cfg.hidden, cfg.head_dim
    for banned in ("ssm_a", "ssm_out.weight", "attn_qkv.weight", "attn_gate.weight"):
        if p + banned in g:
            raise SnowLLMError(f"{g.path.name}: {p + banned} belongs to a linear-attention layer, "
                               f"which this build does not compute")
    q_rows = cfg.heads * d
    if g[p + "attn_q.weight"].shape[0] == 2 * q_rows:
        raise SnowLLMError(f"{g.path.name}: {p}attn_q.weight carries an output gate per head; "
                           f"gated attention output is not computed by this build")
    _shape(g, p + "attn_q.weight", q_rows, H)
    _shape(g, p + "attn_k.weight", cfg.kv_heads * d, H)
    _shape(g, p + "attn_v.weight", cfg.kv_heads * d, H)
    _shape(g, p + "attn_output.weight", H, q_rows)
    for n in ("attn_q_norm.weight", "attn_k_norm.weight"):
        if p + n not in g:
            raise SnowLLMError(f"{g.path.name}: no {p + n}; this build applies QK-norm")
    if cfg.moe:   # checked before any tensor is read
        gu_fmt = _expert_fmt(g, p + "ffn_gate_exps.weight")
        dn_fmt = _expert_fmt(g, p + "ffn_down_exps.weight")
        if dn_fmt < gu_fmt:
            raise SnowLLMError(f"{g.path.name}: {p}ffn_down_exps.weight is narrower than the "
                               f"experts' gate/up; the MoE kernels take down in the gate/up "
                               f"format or a wider one")
    names = [p + n for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight")]
    v = v_fmt = None
    if len({_kfmt(g, n) for n in names}) == 1:
        raw, qkv_fmt = _blocks(g, names)
        qkv = ops.gemm_kquant_shuffle_b(qkv_fmt, raw, cfg.qkv_n, H)
    else:
        # q|k in one format and v in its own (qwen3_5_weights.py:95-109): two GEMVs into the
        # columns of one projection output
        nqk = (cfg.heads + cfg.kv_heads) * d
        raw, qkv_fmt = _blocks(g, names[:2])
        qkv = ops.gemm_kquant_shuffle_b(qkv_fmt, raw, nqk, H)
        raw, v_fmt = _blocks(g, names[2:])
        v = (*ops.gemm_kquant_shuffle_b(v_fmt, raw, cfg.qkv_n - nqk, H), None)
    raw, o_fmt = _blocks(g, [p + "attn_output.weight"])
    o = ops.gemm_kquant_shuffle_b(o_fmt, raw, H, q_rows)
    lw = LayerWeights(in_norm=_gamma(g, p + "attn_norm.weight"),
                      post_norm=_gamma(g, p + "post_attention_norm.weight"),
                      q_norm=_gamma(g, p + "attn_q_norm.weight"),
                      k_norm=_gamma(g, p + "attn_k_norm.weight"),
                      qkv=(*qkv, None), o=(*o, None), qkv_fmt=qkv_fmt, o_fmt=o_fmt, v=v,
                      v_fmt=v_fmt or 0)
    if cfg.moe:
        E, F = cfg.experts, cfg.expert_ffn
        if p + "ffn_gate_inp_shexp.weight" not in g:
            raise SnowLLMError(f"{g.path.name}: {p}ffn_gate_inp_shexp.weight is missing; this "
                               f"build's MoE has a gated shared expert")
        _shape(g, p + "ffn_gate_inp.weight", E, H)
        router = torch.cat([_bf16(g, p + "ffn_gate_inp.weight"),
                            _bf16(g, p + "ffn_gate_inp_shexp.weight").reshape(1, H)])
        lw.router = ops.moe_shuffle_router(router)
        for n, shape in (("ffn_gate_exps", (E, F, H)), ("ffn_up_exps", (E, F, H)),
                         ("ffn_down_exps", (E, H, F)), ("ffn_gate_shexp", (F, H)),
                         ("ffn_up_shexp", (F, H)), ("ffn_down_shexp", (H, F))):
            _shape(g, p + n + ".weight", *shape)
        gate, _ = _blocks(g, [p + "ffn_gate_exps.weight"], gu_fmt)
        up, _ = _blocks(g, [p + "ffn_up_exps.weight"], gu_fmt)
        gu = ops.moe_kquant_shuffle_gate_up(gate, up, gu_fmt, E)
        del gate, up
        down, _ = _blocks(g, [p + "ffn_down_exps.weight"], dn_fmt)
        dn = ops.moe_kquant_shuffle_down(down, dn_fmt, E)
        del down
        # one launch computes the routed and shared experts: the same formats for both
        sg, _ = _blocks(g, [p + "ffn_gate_shexp.weight"], gu_fmt)
        su, _ = _blocks(g, [p + "ffn_up_shexp.weight"], gu_fmt)
        sd, _ = _blocks(g, [p + "ffn_down_shexp.weight"], dn_fmt)
        sh_gu = ops.moe_kquant_shuffle_gate_up(sg, su, gu_fmt, 1)
        sh_dn = ops.moe_kquant_shuffle_down(sd, dn_fmt, 1)
        lw.gu_fmt, lw.dn_fmt = gu_fmt, dn_fmt
        lw.gu, lw.dn = (gu.p0, gu.p1, None), (dn.p0, dn.p1, None)
        lw.sh_gu, lw.sh_dn = (sh_gu.p0, sh_gu.p1, None), (sh_dn.p0, sh_dn.p1, None)
    else:
        F = cfg.ffn
        _shape(g, p + "ffn_gate.weight", F, H)
        _shape(g, p + "ffn_up.weight", F, H)
        _shape(g, p + "ffn_down.weight", H, F)
        raw, gu_fmt = _blocks(g, [p + "ffn_gate.weight", p + "ffn_up.weight"])
        lw.gu = (*ops.gemm_kquant_shuffle_b(gu_fmt, raw, 2 * F, H), None)
        lw.gu_fmt = gu_fmt
        raw, dn_fmt = _blocks(g, [p + "ffn_down.weight"])
        lw.dn = (*ops.gemm_kquant_shuffle_b(dn_fmt, raw, H, F), None)
        lw.dn_fmt = dn_fmt
    return lw


_QNAME = {v: k for k, v in KQUANT_FORMAT.items()}


def gguf_metadata(cfg: VerifyConfig) -> dict:
    """The "{arch}.*" metadata of a config, under the reference's architecture names
    (names.py:14-16: qwen35moe, qwen35), all layers full attention."""
    arch = "qwen35moe" if cfg.moe else "qwen35"
    kv = {"general.architecture": arch, f"{arch}.block_count": cfg.layers,
          f"{arch}.embedding_length": cfg.hidden, f"{arch}.attention.head_count": cfg.heads,
          f"{arch}.attention.head_count_kv": cfg.kv_heads,
          f"{arch}.attention.key_length": cfg.head_dim,
          f"{arch}.attention.value_length": cfg.head_dim,
          f"{arch}.rope.dimension_count": 2 * cfg.rot_half,
          f"{arch}.rope.freq_base": float(cfg.rope_theta),
          f"{arch}.attention.layer_norm_rms_epsilon": float(cfg.eps),
          f"{arch}.full_attention_interval": 1, f"{arch}.context_length": 262144}
    if cfg.moe:
        kv.update({f"{arch}.expert_count": cfg.experts, f"{arch}.expert_used_count": cfg.topk,
                   f"{arch}.expert_feed_forward_length": cfg.expert_ffn,
                   f"{arch}.expert_shared_feed_forward_length": cfg.expert_ffn})
    else:
        kv[f"{arch}.feed_forward_length"] = cfg.ffn
    return kv


def model_tensors(model: VerifyModel, *, tied: bool = False):
    """(name, shape, quant name, payload) of a random-weight VerifyModel built with
    keep_raw=True, in the GGUF names: its GGUF blocks as generated, norms and router F32, the
    embedding and head F16 (no head when tied)."""
    cfg = model.cfg
    H, d = cfg.hidden, cfg.head_dim
    out = []

    def f32(t):
        return t.detach().float().cpu().contiguous()

    def rows(raw, fmt, k):
        q = _QNAME[fmt]
        from .gguf import QUANTS
        return raw.detach().cpu().view(-1, QUANTS[q].nbytes(k)), q

    for i, lw in enumerate(model.layers):
        if any(t is None for t in (lw.qkv[2], lw.o[2], lw.gu[2], lw.dn[2])):
            raise SnowLLMError("model_tensors needs a model built with keep_raw=True")
        p = f"blk.{i}."
        qkv, qa = rows(lw.qkv[2], lw.qkv_fmt or cfg.attn_fmt, H)
        nq, nk = cfg.heads * d, cfg.kv_heads * d
        out += [(p + "attn_q.weight", (nq, H), qa, qkv[:nq]),
                (p + "attn_k.weight", (nk, H), qa, qkv[nq:nq + nk])]
        if lw.v is None:
            out.append((p + "attn_v.weight", (nk, H), qa, qkv[nq + nk:]))
        else:
            if lw.v[2] is None:
                raise SnowLLMError("model_tensors needs a model built with keep_raw=True")
            vr, va = rows(lw.v[2], lw.v_fmt, H)
            out.append((p + "attn_v.weight", (nk, H), va, vr))
        o, oa = rows(lw.o[2], lw.o_fmt or cfg.attn_fmt, nq)
        out.append((p + "attn_output.weight", (H, nq), oa, o))
        for n, t in (("attn_norm", lw.in_norm), ("post_attention_norm", lw.post_norm),
                     ("attn_q_norm", lw.q_norm), ("attn_k_norm", lw.k_norm)):
            out.append((p + n + ".weight", tuple(t.shape), "F32", f32(t)))
        gu_fmt = lw.gu_fmt or cfg.ffn_fmt
        dn_fmt = lw.dn_fmt or cfg.down_fmt or cfg.ffn_fmt
        if cfg.moe:
            E, F = cfg.experts, cfg.expert_ffn
            router = f32(lw.raw["router"])
            out += [(p + "ffn_gate_inp.weight", (E, H), "F32", router[:E]),
                    (p + "ffn_gate_inp_shexp.weight", (H,), "F32", router[E])]
            gu, fa = rows(lw.gu[2], gu_fmt, H)
            gu = gu.view(E, 2, F, -1)
            dn, da = rows(lw.dn[2], dn_fmt, F)
            sgu, _ = rows(lw.sh_gu[2], gu_fmt, H)
            sdn, _ = rows(lw.sh_dn[2], dn_fmt, F)
            out += [(p + "ffn_gate_exps.weight", (E, F, H), fa, gu[:, 0].contiguous()),
                    (p + "ffn_up_exps.weight", (E, F, H), fa, gu[:, 1].contiguous()),
                    (p + "ffn_down_exps.weight", (E, H, F), da, dn),
                    (p + "ffn_gate_shexp.weight", (F, H), fa, sgu[:F]),
                    (p + "ffn_up_shexp.weight", (F, H), fa, sgu[F:]),
                    (p + "ffn_down_shexp.weight", (H, F), da, sdn)]
        else:
            F = cfg.ffn
            gu, fa = rows(lw.gu[2], gu_fmt, H)
            dn, da = rows(lw.dn[2], dn_fmt, F)
            out += [(p + "ffn_gate.weight", (F, H), fa, gu[:F]),
                    (p + "ffn_up.weight", (F, H), fa, gu[F:]),
                    (p + "ffn_down.weight", (H, F), da, dn)]
    out.append(("token_embd.weight", (cfg.vocab, H), "F16", model.embed.detach().cpu()))
    if not tied:
        if model.lm_head_raw is None:
            raise SnowLLMError("model_tensors needs a model built with keep_raw=True")
        out.append(("output.weight", (cfg.vocab, H), "F16", model.lm_head_raw.detach().cpu()))
    out.append(("output_norm.weight", (H,), "F32", f32(model.final_norm)))
    return out


def save_gguf(path, cfg: VerifyConfig, tensors, *, parts: int = 1):
    """Write tensors (as model_tensors gives them) as a GGUF checkpoint of `parts` files named
    NAME-0000i-of-0000n.gguf when parts > 1; returns the path to open."""
    from .gguf import write_gguf
    import pathlib
    kv = gguf_metadata(cfg)
    path = pathlib.Path(path)
    if parts == 1:
        return write_gguf(path, kv, tensors)
    stem = path.name[:-5] if path.name.endswith(".gguf") else path.name
    chunks = [tensors[i::parts] for i in range(parts)]
    first = None
    for i, chunk in enumerate(chunks):
        meta = dict(kv) if i == 0 else {"general.architecture": kv["general.architecture"]}
        meta.update({"split.no": i, "split.count": parts, "split.tensors.count": len(tensors)})
        p = write_gguf(path.parent / f"{stem}-{i + 1:05d}-of-{parts:05d}.gguf", meta, chunk)
        first = first or p
    return first


def load_gguf(path, *, context: int, block: int, tree_parents=(), kv_std: float = 1.0,
              seed: int = 0, name: str = None) -> VerifyModel:
    """A VerifyModel whose weights come from the GGUF checkpoint at `path` (one file or the
    first part of a split one). The KV cache is random (kv_std, seed) and holds `context` prior
    tokens; `block` rows are verified per step. Installs the checkpoint's geometry (the repack
    entry points read their shapes from it) and leaves it active."""
    g = GGUF(path)
    try:
        cfg = config_from_gguf(g, context=context, block=block, tree_parents=tree_parents,
                               name=name)
        ops.define_geometry(**geometry_fields(cfg))

        def install(model: VerifyModel):
            H, V = cfg.hidden, cfg.vocab
            model.layers = []
            for i in range(cfg.layers):
                model.layers.append(_layer(g, cfg, i))
                torch.cuda.synchronize()   # the layer's staged blocks are freed before the next
            emb = g["token_embd.weight"]
            if emb.quant.name == "Q4_K":
                model.embed = g.payload("token_embd.weight").to("cuda").view(V, H // 256 * 144)
                model.embed_q4k = True
            else:
                model.embed = _bf16(g, "token_embd.weight")
            _shape(g, "token_embd.weight", V, H)
            head = "output.weight" if "output.weight" in g else "token_embd.weight"
            _shape(g, head, V, H)
            if g[head].quant.name in KQUANT_FORMAT:
                w = ops.lm_head_kquant_shuffle_weight(g.payload(head).to("cuda"),
                                                      KQUANT_FORMAT[g[head].quant.name])
                model.lm_head, model.head_wt, model.head_fmt = (w.p0, w.p1), HEAD_KQUANT, w.fmt
            else:
                model.lm_head = ops.lm_head_shuffle_weight(_bf16(g, head))
                model.head_wt = Lops.WT_BF16
            model.final_norm = _gamma(g, "output_norm.weight")

        model = VerifyModel(cfg, seed=seed, kv_std=kv_std, weights=install)
        torch.cuda.synchronize()
        return model
    finally:
        g.close()
