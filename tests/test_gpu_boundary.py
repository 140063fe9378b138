"""The reference-signature entry points (geometry-driven, _Weight descriptors, the paged-attention
step descriptor) against this build's explicit-shape path: one decoder layer run in the
reference's own dataflow (snowllm/models/qwen3_5/qwen3_5.py:32-43, layers.py:86-117, 166-188)
must give the same bits as VerifyModel's layer, and each operator matches its explicit form."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def tiny(kind):
    from snowllm_amd.verify import VerifyConfig
    base = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rot_half=32,
                rope_theta=1e4, vocab=2048, context=300, block=9)
    if kind == "moe":
        return VerifyConfig("tiny_moe", experts=16, expert_ffn=256, topk=4, **base)
    return VerifyConfig("tiny_dense", ffn=512, **base)


@pytest.fixture
def geometry_of():
    """Install the geometry of a VerifyConfig for the reference-signature entry points; the
    default geometry comes back afterwards."""
    from snowllm_amd import ops

    def install(cfg):
        from snowllm_amd.verify import geometry_fields
        ops.define_geometry(**geometry_fields(cfg))
    yield install
    ops.select_geometry(0)


# v_fmt 6: q|k Q4_K and v Q6_K, the split projection (qwen3_5_weights.py:95-109)
@pytest.mark.parametrize("v_fmt", [0, 6])
def test_reference_dataflow_layer_matches_verify_model(gpu, geometry_of, v_fmt):
    from dataclasses import replace
    from snowllm_amd import ops
    from snowllm_amd.verify import VerifyModel
    cfg = replace(tiny("moe"), v_fmt=v_fmt)
    geometry_of(cfg)
    print(f"reference-signature layer, tiny moe, v format {v_fmt or cfg.attn_fmt}", flush=True)
    m = VerifyModel(cfg, seed=8)
    T, H, d = cfg.block, cfg.hidden, cfg.head_dim
    m.set_block(torch.arange(T) * 11)
    m.forward(upto_layer=0)
    torch.cuda.synchronize()
    x0 = m.x.clone()  # the embeddings: the residual stream entering layer 0
    lw = m.layers[0]
    k_pool, v_pool = m.k_pools[0].clone(), m.v_pools[0].clone()
    # -- the reference's layer 0, entry point by entry point --------------------------------
    residual = x0.clone()
    bf = torch.bfloat16
    proj = torch.empty(T, cfg.qkv_n, dtype=bf, device="cuda")
    scratch = torch.empty(ops.qkv_proj_scratch_bytes(T), dtype=torch.uint8, device="cuda")
    w_qkv = ops.KQuantProjWeight(lw.qkv[0], lw.qkv[1], cfg.attn_fmt)
    w_v = ops.KQuantProjWeight(lw.v[0], lw.v[1], lw.v_fmt) if v_fmt else None
    ops.inference_qkv(residual, w_qkv, None, w_v, None, scratch, proj, 0, None, lw.in_norm,
                      cfg.eps)
    cos = torch.empty(T, 64, device="cuda")
    sin = torch.empty_like(cos)
    ops.rope_cos_sin(m.positions, m.inv_freq, cos, sin)
    q = torch.empty(T, cfg.heads, d, dtype=bf, device="cuda")
    v = proj[:, (cfg.heads + cfg.kv_heads) * d:]
    ops.qk_norm_rope_cache(proj, lw.q_norm, lw.k_norm, cos, sin, q, v, k_pool, v_pool, m.slots,
                           cfg.eps, 16)
    attn = torch.empty(*ops.attn_output_shape(T, False, False), dtype=bf, device="cuda")
    ascratch = torch.empty(ops.paged_attention_scratch_bytes(1, T, False), dtype=torch.uint8,
                           device="cuda")
    ops.paged_attention(q, (k_pool, v_pool), attn, None, m.table, m.lens, None, 0, None, None,
                        0, T, 16, d ** -0.5, False, ascratch,
                        ops.attn_output_gating(proj, False, False))
    blk = torch.empty(T, H, dtype=bf, device="cuda")
    _, need = ops.attn_output_plan(T, False, False)
    w_o = ops.KQuantProjWeight(lw.o[0], lw.o[1], cfg.attn_fmt)
    ops.attn_output_project(attn, proj, w_o, None,
                            torch.empty(max(need, 1), dtype=torch.uint8, device="cuda"), blk,
                            False, False)
    hidden = torch.empty(T, H, dtype=bf, device="cuda")
    mws = torch.empty(ops.moe_workspace_bytes(T), dtype=torch.uint8, device="cuda")
    gate = ops.KQuantExpertWeight(lw.gu[0], lw.gu[1], None, cfg.ffn_fmt)
    down = ops.KQuantExpertWeight(lw.dn[0], lw.dn[1], None, cfg.ffn_fmt)
    sh_gate = ops.KQuantProjWeight(lw.sh_gu[0], lw.sh_gu[1], cfg.ffn_fmt)
    sh_down = ops.KQuantProjWeight(lw.sh_dn[0], lw.sh_dn[1], cfg.ffn_fmt)
    ops.inference_moe_norm(blk, residual, lw.post_norm, cfg.eps, hidden, lw.router, gate, down,
                           sh_gate, sh_down, blk, mws)
    torch.cuda.synchronize()
    # -- VerifyModel's layer 0 ------------------------------------------------------------
    m.forward(upto_layer=1)
    torch.cuda.synchronize()
    assert torch.equal(proj, m.proj) and torch.equal(q, m.q)
    assert torch.equal(k_pool, m.k_pools[0]) and torch.equal(v_pool, m.v_pools[0])
    assert torch.equal(attn, m.attn)
    assert torch.equal(hidden, m.h2)
    assert torch.equal(residual, m.layer_residual)
    assert torch.equal(blk, m.x)


@pytest.mark.parametrize("down_fmt", [0, 6])   # 6: Q6_K down under Q4_K gate/up (Q4_K_M)
def test_moe_without_norm_and_head(gpu, geometry_of, down_fmt):
    from dataclasses import replace
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    from snowllm_amd.verify import VerifyModel
    cfg = replace(tiny("moe"), down_fmt=down_fmt)
    dn_f = down_fmt or cfg.ffn_fmt
    geometry_of(cfg)
    print(f"reference-signature MoE / head, tiny moe, down format {dn_f}", flush=True)
    m = VerifyModel(cfg, seed=9)
    T, H = cfg.block, cfg.hidden
    m.set_block(torch.arange(T) * 3)
    m.forward()
    torch.cuda.synchronize()
    lw = m.layers[1]
    y = m.h2.clone()  # a normalised hidden of the last layer
    out = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
    mws = torch.empty(ops.inference_moe_workspace_bytes(T), dtype=torch.uint8, device="cuda")
    gate = ops.KQuantExpertWeight(lw.gu[0], lw.gu[1], None, cfg.ffn_fmt)
    down = ops.KQuantExpertWeight(lw.dn[0], lw.dn[1], None, dn_f)
    sh_gate = ops.KQuantProjWeight(lw.sh_gu[0], lw.sh_gu[1], cfg.ffn_fmt)
    sh_down = ops.KQuantProjWeight(lw.sh_dn[0], lw.sh_dn[1], dn_f)
    ops.inference_moe(y, lw.router, gate, down, sh_gate, sh_down, out, mws)
    # explicit path on the same rows
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(T, H), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_prepare_a(y, ws)
    L.dense_gemv(L.WT_BF16, lw.router, y, m.router_logits, T, cfg.experts + 1, H)
    L.moe_route_plan(m.router_logits, cfg.experts, cfg.topk, m.route_w, m.route_ids, m.shared_w,
                     m.plan)
    want = torch.empty_like(out)
    L.moe_experts(cfg.ffn_fmt | dn_f << 8, lw.gu, lw.dn, lw.sh_gu, lw.sh_dn, m.plan, ws, m.route_w,
                  m.shared_w, m.moe_act, m.pairs, m.shared_out, want, T, cfg.topk, cfg.experts, H,
                  cfg.expert_ffn)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    # LM head on normalised rows: bf16 head (kind 0) and a Q8_0 head (kind 3), through the
    # descriptor and the direct entry points, against the explicit GEMVs
    from snowllm_amd.verify import gguf_random
    hs = torch.empty(ops.lm_head_scratch_bytes(T), dtype=torch.uint8, device="cuda")
    head = (0.02 * torch.randn(cfg.vocab, H, device="cuda")).bfloat16()
    hw = ops.lm_head_shuffle_weight(head)
    want_l = torch.empty(T, cfg.vocab, device="cuda")
    L.dense_gemv(L.WT_BF16, hw, y, want_l, T, cfg.vocab, H)
    kraw = gguf_random(8, cfg.vocab, H, seed=5)
    kw = ops.lm_head_kquant_shuffle_weight(kraw, 8)
    want_k = torch.empty_like(want_l)
    ops.gemm_kquant_a(8, y, kw.p0, kw.p1, want_k, T, cfg.vocab, H, ws)
    for w, want, direct in ((hw, want_l, ops.lm_head), (kw, want_k, ops.lm_head_kquant)):
        logits = torch.full_like(want_l, float("nan"))
        ops.inference_head(y, w, logits, hs)
        logits2 = torch.full_like(want_l, float("nan"))
        direct(y, w, logits2, hs)
        torch.cuda.synchronize()
        assert torch.equal(logits, want) and torch.equal(logits2, want)


def test_moe_of_a_batch(gpu, geometry_of):
    """snowllm_inference_moe over 36 rows (a batched verify step; one expert routed every row,
    so it takes three slots) equals the explicit route/plan + experts launches bit for bit,
    and the oracle's dequantised experts within tolerance."""
    import numpy as np
    from oracle import quant as Q
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    from snowllm_amd.verify import VerifyModel
    cfg = tiny("moe")
    geometry_of(cfg)
    print("reference-signature MoE over 36 rows", flush=True)
    m = VerifyModel(cfg, seed=12, keep_raw=True)
    E, K, H, F = cfg.experts, cfg.topk, cfg.hidden, cfg.expert_ffn
    M = 36
    g = torch.Generator(device="cuda").manual_seed(3)
    y = torch.randn(M, H, device="cuda", generator=g).bfloat16()
    lw = m.layers[0]
    # a router whose expert 2 wins every row: its slots hold 16, 16 and 4 rows
    router = lw.raw["router"].clone()
    router[2] = y.float().mean(0).bfloat16() * 50
    rw = L.dense_shuffle(router)
    out = torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
    mws = torch.empty(ops.inference_moe_workspace_bytes(M), dtype=torch.uint8, device="cuda")
    gate = ops.KQuantExpertWeight(lw.gu[0], lw.gu[1], None, cfg.ffn_fmt)
    down = ops.KQuantExpertWeight(lw.dn[0], lw.dn[1], None, cfg.ffn_fmt)
    sh_gate = ops.KQuantProjWeight(lw.sh_gu[0], lw.sh_gu[1], cfg.ffn_fmt)
    sh_down = ops.KQuantProjWeight(lw.sh_dn[0], lw.sh_dn[1], cfg.ffn_fmt)
    ops.inference_moe(y, rw, gate, down, sh_gate, sh_down, out, mws)
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(M, H), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_prepare_a(y, ws)
    logits = torch.empty(M, E + 1, device="cuda")
    L.dense_gemv(L.WT_BF16, rw, y, logits, M, E + 1, H)
    w = torch.empty(M, K, device="cuda")
    ids = torch.empty(M, K, dtype=torch.int32, device="cuda")
    sw = torch.empty(M, device="cuda")
    plan = torch.empty(L.MOE_PLAN_BYTES, dtype=torch.uint8, device="cuda")
    L.moe_route_plan(logits, E, K, w, ids, sw, plan)
    act = torch.empty(L.moe_max_slots(M, K, E), 16, F, dtype=torch.bfloat16, device="cuda")
    pairs = torch.empty(M * K, H, device="cuda")
    shared = torch.empty(M, H, device="cuda")
    want = torch.empty_like(out)
    L.moe_experts(cfg.ffn_fmt, lw.gu, lw.dn, lw.sh_gu, lw.sh_dn, plan, ws, w, sw, act, pairs,
                  shared, want, M, K, E, H, F)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    p = L.parse_plan(plan)
    assert list(p["slot_expert"]).count(2) == 3 and list(p["slot_expert"]).count(E) == 3
    # against the dequantised experts (fp64), rows as the kernels see them (bf16 products)
    def bf(x):
        return x.to(torch.bfloat16).double()
    gub, dnb = lw.gu[2].cpu().numpy(), lw.dn[2].cpu().numpy()
    gbytes, dbytes = gub.size // E, dnb.size // E
    xc = y.cpu().double()
    ref = torch.zeros(M, H, dtype=torch.float64)
    cache = {}

    def ffn(xr, gw, dw):
        gg, uu = bf(xr @ gw[:F].T), bf(xr @ gw[F:].T)
        return bf(bf(gg / (1 + torch.exp(-gg)) * uu) @ dw.T)
    ids_c, w_c, sw_c = ids.cpu().long(), w.cpu().double(), sw.cpu().double()
    for r in range(M):
        for k in range(K):
            e = int(ids_c[r, k])
            if e not in cache:
                cache[e] = (torch.from_numpy(Q.dequant(gub[e * gbytes:(e + 1) * gbytes], 4, 2 * F, H)).double(),
                            torch.from_numpy(Q.dequant(dnb[e * dbytes:(e + 1) * dbytes], 4, H, F)).double())
            ref[r] += w_c[r, k] * ffn(xc[r:r + 1], *cache[e])[0]
    sg = torch.from_numpy(Q.dequant(lw.sh_gu[2].cpu().numpy(), 4, 2 * F, H)).double()
    sd = torch.from_numpy(Q.dequant(lw.sh_dn[2].cpu().numpy(), 4, H, F)).double()
    ref += sw_c[:, None] * ffn(xc, sg, sd)
    err = ((out.cpu().double() - ref).norm() / ref.norm()).item()
    print(f"  36-row MoE rel L2 {err:.2e}", flush=True)
    assert err < 5e-3
    assert np.isfinite(out.float().cpu().numpy()).all()


def test_dense_mlp(gpu, geometry_of):
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    from snowllm_amd.verify import VerifyModel
    cfg = tiny("dense")
    geometry_of(cfg)
    print("reference-signature MLP, tiny dense", flush=True)
    m = VerifyModel(cfg, seed=10)
    T, H, F = cfg.block, cfg.hidden, cfg.ffn
    lw = m.layers[0]
    x = (torch.randn(T, H, device="cuda") * .5).bfloat16()
    out = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
    scratch = torch.empty(ops.mlp_workspace_bytes(T), dtype=torch.uint8, device="cuda")
    ops.inference_mlp(x, ops.KQuantProjWeight(lw.gu[0], lw.gu[1], cfg.ffn_fmt),
                      ops.KQuantProjWeight(lw.dn[0], lw.dn[1], cfg.ffn_fmt), out, scratch, True)
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(T, H), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_prepare_a(x, ws)
    act = torch.empty(T, F, dtype=torch.bfloat16, device="cuda")
    L.gate_up_swiglu(cfg.ffn_fmt, lw.gu[0], lw.gu[1], ws, act, T, F, H)
    want = torch.empty_like(out)
    ws2 = torch.empty(ops.gemm_kquant_a_ws_bytes(T, F), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_a(cfg.ffn_fmt, act, lw.dn[0], lw.dn[1], want, T, H, F, ws2)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_unsupported_features_are_refused(gpu, geometry_of):
    """Features outside the verify path return hipErrorNotSupported, not a wrong answer."""
    from snowllm_amd import ops
    from snowllm_amd._capi import SnowLLMError
    cfg = tiny("moe")
    geometry_of(cfg)
    with pytest.raises(SnowLLMError):
        ops.attn_output_plan(9, False, True)  # int8 KV
    assert ops.attn_output_gating(torch.empty(9, 8, dtype=torch.bfloat16, device="cuda"),
                                  False, False)[0] == 0
    assert ops.paged_attention_varlen(True, 9, False) and not ops.paged_attention_varlen(False, 9, False)


def test_split_kv_decode_entry_equals_explicit_attention(gpu, geometry_of):
    """snowllm_paged_attn_decode (the reference's split-KV decode signature, with its plan call
    and a q read at a row pitch from row q_row0) gives the explicit-shape attention's bits."""
    from snowllm_amd import ops
    from snowllm_amd.verify import VerifyConfig
    cfg = VerifyConfig("decode_geo", layers=1, hidden=2048, heads=16, kv_heads=2, head_dim=256,
                       rot_half=32, rope_theta=1e7, vocab=2048, context=3000, block=9,
                       experts=16, expert_ffn=512, topk=4)
    geometry_of(cfg)
    print("split-KV decode entry, 3 sequences", flush=True)
    g = torch.Generator(device="cuda").manual_seed(31)
    T, Hq, Hkv, D = 9, 16, 2, 256
    lengths = [3000 + T, 777 + T, 40 + T]
    B = len(lengths)
    width = max((L + 15) // 16 for L in lengths)
    blocks = B * width + 5
    kp = torch.randn(blocks, Hkv, D // 16, 16, 16, device="cuda", generator=g).bfloat16()
    vp = torch.randn(blocks, Hkv, 4, D, 4, device="cuda", generator=g).bfloat16()
    table = torch.randperm(blocks, device="cuda", generator=g)[:B * width].int().view(B, width)
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    pitch, row0 = Hq * D + 512, 2
    buf = torch.randn(row0 + B * T, pitch, device="cuda", generator=g).bfloat16()
    q = buf[row0:, :Hq * D].contiguous().view(B * T, Hq, D)
    want = torch.empty_like(q)
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(B, T, Hq, Hkv, D),
                          dtype=torch.uint8, device="cuda")
    ops.paged_attention_explicit(q, kp, vp, want, table, lens, D ** -0.5, scratch)
    slots = ops.paged_decode_num_slots(B)
    plan = torch.empty(ops.paged_decode_plan_elems(B, slots), dtype=torch.int32, device="cuda")
    ws = torch.empty(ops.paged_decode_workspace_size(slots, T), dtype=torch.uint8, device="cuda")
    ops.paged_attn_decode_plan(lens, plan, slots, 16)
    got = torch.empty_like(q)
    ops.paged_attn_decode(buf, lens, kp, vp, got, table, plan, ws, B, slots, D ** -0.5, 16,
                          q_tokens=T, q_pitch=pitch, q_row0=row0)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert T <= ops.PAGED_DECODE_MAX_Q_TOKENS
    assert ops.paged_attention_prepare(lens, T, slots, 16, False) is None
