"""MoE routing, plan and experts on the GPU at the 35B-A3B shape (hidden
2048, 256 routed experts of FFN 512 + a shared expert, top-8, block of 9 rows).

Routing follows transformers' qwen3_next semantics (softmax over the routed logits, top-k,
renormalised, sigmoid shared-expert gate); the experts are checked against fp64 matmuls of the
dequantized GGUF blocks of the experts the block touches (oracle/quant.py)."""
import numpy as np
import pytest
import torch

from oracle import quant as Q

pytestmark = pytest.mark.gpu

H, F, E, K = 2048, 512, 256, 8


def _route_reference(logits, topk):
    probs = torch.softmax(logits[:, :E].double(), -1)
    w, ids = torch.topk(probs, topk, dim=-1)
    return ids, w / w.sum(-1, keepdim=True), torch.sigmoid(logits[:, E].double())


def _expected_plan(ids_np, M, shared=True):
    """The plan's slots by brute force: experts in ascending id, each expert's rows in
    ascending order, 16 per slot; then the shared expert's rows, 16 per slot."""
    K = ids_np.shape[1]
    slots = []
    for e in np.unique(ids_np):
        rows = [r for r in range(M) if e in ids_np[r]]
        for j in range(0, len(rows), 16):
            part = rows[j:j + 16]
            slots.append((int(e), part, [r * K + list(ids_np[r]).index(e) for r in part]))
    n_routed = len(slots)
    if shared:
        for j in range(0, M, 16):
            part = list(range(j, min(M, j + 16)))
            slots.append((E, part, [-1] * len(part)))
    return slots, n_routed


def _check_plan(p, ids_np, M, shared=True):
    slots, n_routed = _expected_plan(ids_np, M, shared)
    assert p["n_routed"] == n_routed and p["n_slots"] == len(slots)
    for s, (e, rows, pairs) in enumerate(slots):
        n = len(rows)
        assert p["slot_expert"][s] == e and p["slot_rows"][s] == n, s
        assert list(p["row_of"][s][:n]) == rows, s
        assert list(p["pair_of"][s][:n]) == pairs, s


# up to 16 rows: one slot per expert; 36 and 64 rows (batched verify): an expert routed more
# than 16 rows takes one slot per 16 ("hot": every row routed to expert 5)
@pytest.mark.parametrize("M,hot", [(1, False), (9, False), (16, False), (36, False), (36, True),
                                   (64, True)])
def test_route_plan(gpu, M, hot):
    from snowllm_amd import layers as L
    print(f"route+plan M={M} hot={hot}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M)
    logits = torch.randn(M, E + 1, device="cuda", generator=g)
    if hot:
        logits[:, 5] += 50.0
    w = torch.empty(M, K, device="cuda")
    ids = torch.empty(M, K, dtype=torch.int32, device="cuda")
    sw = torch.empty(M, device="cuda")
    plan = torch.empty(L.MOE_PLAN_BYTES, dtype=torch.uint8, device="cuda")
    L.moe_route_plan(logits, E, K, w, ids, sw, plan)
    torch.cuda.synchronize()
    rid, rw, rsw = _route_reference(logits.cpu(), K)
    assert torch.equal(ids.cpu().long(), rid)
    assert torch.allclose(w.cpu().double(), rw, rtol=1e-5, atol=1e-7)
    assert torch.allclose(sw.cpu().double(), rsw, rtol=1e-5, atol=1e-7)
    p = L.parse_plan(plan)
    ids_np = ids.cpu().numpy()
    _check_plan(p, ids_np, M)
    assert p["n_slots"] <= L.moe_max_slots(M, K, E)
    if hot:
        assert list(p["slot_expert"]).count(5) == (M + 15) // 16
    # the separate route + plan entry points agree with the fused one
    w2, ids2 = torch.empty_like(w), torch.empty_like(ids)
    plan2 = torch.zeros_like(plan)
    L.moe_route(logits, E, K, w2, ids2, None)
    L.moe_plan(ids2, E, plan2, shared=True)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(w2, w)
    _check_plan(L.parse_plan(plan2), ids_np, M)


# one / two superblocks per down wave; expert formats (gate/up, down): Q4_K_M keeps some
# layers' down in Q6_K, Q5_K_M / Q6_K files store the experts in those formats
@pytest.mark.parametrize("E,F,gu_f,dn_f", [(E, F, 4, 4), (64, 1024, 4, 4), (E, F, 4, 6),
                                           (E, F, 6, 6), (64, 1024, 5, 6), (E, F, 5, 5)])
def test_gate_up_down_equals_separate_launches(gpu, E, F, gu_f, dn_f):
    """Gate/up and down in one launch (down items wait for their slot's gate/up items) give the
    bits of the two launches; consecutive launches of different sizes reuse the flags."""
    from snowllm_amd import layers as L, ops
    from snowllm_amd.verify import packed_random
    gu = packed_random(gu_f, E * 2 * F, H, 51, stack=E)
    dn = packed_random(dn_f, E * H, F, 52, stack=E)
    sgu = packed_random(gu_f, 2 * F, H, 53)
    sdn = packed_random(dn_f, H, F, 54)
    # (rows, shared, routing): "spread" puts every row on its own experts (the most slots),
    # "hot" every row on expert 3 (one slot per 16 rows of it)
    cases = ((9, True, ""), (16, True, "spread"), (1, True, ""), (9, False, "spread"),
             (9, True, "spread"), (36, True, "hot"), (64, True, "spread"), (40, False, "hot"),
             (4, True, "spread"))
    for M, shared, route in cases if (gu_f, dn_f) == (4, 4) else cases[:3] + cases[5:6]:
        print(f"gate_up_down E={E} F={F} fmt={gu_f}/{dn_f} M={M} shared={shared} "
              f"routing={route}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(70 + M)
        x = torch.randn(M, H, device="cuda", generator=g).bfloat16()
        logits = torch.randn(M, E + 1, device="cuda", generator=g) * 2
        if route == "spread":
            for r in range(M):
                logits[r, (K * r) % E:(K * r) % E + K] += 40.0
        elif route == "hot":
            logits[:, 3] += 40.0
        w = torch.empty(M, K, device="cuda")
        ids = torch.empty(M, K, dtype=torch.int32, device="cuda")
        sw = torch.empty(M, device="cuda") if shared else None
        plan = torch.empty(L.MOE_PLAN_BYTES, dtype=torch.uint8, device="cuda")
        L.moe_route_plan(logits, E, K, w, ids, sw, plan)
        ws = torch.empty(ops.gemm_kquant_a_ws_bytes(M, H), dtype=torch.uint8, device="cuda")
        ops.gemm_kquant_prepare_a(x, ws)
        ns = L.moe_max_slots(M, K, E, shared)
        sg, sd = (sgu, sdn) if shared else ((None, None), (None, None))
        outs = []
        # the separate launches, the one-launch form twice, and both again with the largest
        # slot bound: a launch of 64 or more slots runs each gate/up pair on one wave standing
        # for two, which must give the bits of the two-wave form the smaller bounds take
        for fused, bound in ((False, ns), (True, ns), (True, ns), (True, L.MOE_MAX_SLOTS),
                             (False, L.MOE_MAX_SLOTS)):
            act = torch.zeros(bound, 16, F, dtype=torch.bfloat16, device="cuda")
            pairs = torch.zeros(M * K, H, device="cuda")
            sh_out = torch.zeros(M, H, device="cuda")
            if fused:
                L.moe_gate_up_down(gu_f | dn_f << 8, gu, dn, sg, sd, plan, ws, w, sw, act, pairs,
                                   sh_out, M, bound, E, H, F)
            else:
                L.moe_gate_up(gu_f, gu, sg, plan, ws, act, M, bound, E, H, F)
                L.moe_down(dn_f, dn, sd, plan, act, w, sw, pairs, sh_out, bound, E, H, F)
            torch.cuda.synchronize()
            outs.append((act, pairs, sh_out))
        p = L.parse_plan(plan)
        for o in outs[1:]:
            for sl in range(p["n_slots"]):
                r = p["slot_rows"][sl]
                assert torch.equal(o[0][sl, :r], outs[0][0][sl, :r])
            assert torch.equal(o[1], outs[0][1])
            assert torch.equal(o[2], outs[0][2])
    assert L.moe_sync_error() == 0


def _bf(x):
    return x.to(torch.bfloat16).double()


@pytest.mark.parametrize("M,gu_f,dn_f", [(9, 4, 4), (3, 4, 4), (9, 5, 5), (9, 6, 6), (9, 4, 6),
                                          (3, 5, 6), (36, 4, 4), (40, 4, 6)])
def test_experts_match_dequantized_reference(gpu, M, gu_f, dn_f):
    from snowllm_amd import layers as L, ops
    from snowllm_amd.verify import packed_random
    print(f"moe experts M={M} H={H} F={F} E={E} top{K} fmt={gu_f}/{dn_f}", flush=True)
    gu = packed_random(gu_f, E * 2 * F, H, 11, keep_raw=True, stack=E)
    dn = packed_random(dn_f, E * H, F, 12, keep_raw=True, stack=E)
    sgu = packed_random(gu_f, 2 * F, H, 13, keep_raw=True)
    sdn = packed_random(dn_f, H, F, 14, keep_raw=True)
    g = torch.Generator(device="cuda").manual_seed(20 + M)
    x = torch.randn(M, H, device="cuda", generator=g).bfloat16()
    logits = torch.randn(M, E + 1, device="cuda", generator=g) * 2
    if M > 16:   # more than 16 rows of one expert: several slots of it, and of the shared one
        logits[:, 7] += 40.0
    w = torch.empty(M, K, device="cuda")
    ids = torch.empty(M, K, dtype=torch.int32, device="cuda")
    sw = torch.empty(M, device="cuda")
    plan = torch.empty(L.MOE_PLAN_BYTES, dtype=torch.uint8, device="cuda")
    L.moe_route_plan(logits, E, K, w, ids, sw, plan)
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(M, H), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_prepare_a(x, ws)
    act = torch.empty(L.moe_max_slots(M, K, E), 16, F, dtype=torch.bfloat16, device="cuda")
    pairs = torch.empty(M * K, H, device="cuda")
    shared = torch.empty(M, H, device="cuda")
    out = torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
    L.moe_experts(gu_f | dn_f << 8, gu, dn, sgu, sdn, plan, ws, w, sw, act, pairs, shared, out,
                  M, K, E, H, F)
    torch.cuda.synchronize()
    # CPU reference over the touched experts
    xc = x.cpu().double()
    ids_c, w_c, sw_c = ids.cpu().long(), w.cpu().double(), sw.cpu().double()
    gub, dnb = gu[2].cpu().numpy(), dn[2].cpu().numpy()
    gbytes, dbytes = gub.size // E, dnb.size // E

    def ffn(xr, gw, dw):
        gg = _bf(xr @ gw[:F].T)
        uu = _bf(xr @ gw[F:].T)
        a = _bf(gg / (1 + torch.exp(-gg)) * uu)
        return _bf(a @ dw.T)

    cache = {}
    want = torch.zeros(M, H, dtype=torch.float64)
    for r in range(M):
        for k in range(K):
            e = int(ids_c[r, k])
            if e not in cache:
                cache[e] = (torch.from_numpy(Q.dequant(gub[e * gbytes:(e + 1) * gbytes], gu_f, 2 * F, H)).double(),
                            torch.from_numpy(Q.dequant(dnb[e * dbytes:(e + 1) * dbytes], dn_f, H, F)).double())
            want[r] += w_c[r, k] * ffn(xc[r:r + 1], *cache[e])[0]
    sg = torch.from_numpy(Q.dequant(sgu[2].cpu().numpy(), gu_f, 2 * F, H)).double()
    sd = torch.from_numpy(Q.dequant(sdn[2].cpu().numpy(), dn_f, H, F)).double()
    want += sw_c[:, None] * ffn(xc, sg, sd)
    err = ((out.cpu().double() - want).norm() / want.norm()).item()
    print(f"  experts rel L2 {err:.2e} ({len(cache)} experts touched)", flush=True)
    assert err < 5e-3


@pytest.mark.parametrize("M,shared", [(9, True), (16, False), (3, True)])
def test_norm_prep_moe_equals_combine_then_norm(gpu, M, shared):
    """The norm fused with the experts' combine gives the same bits as combine + norm."""
    from snowllm_amd import layers as L
    from snowllm_amd import ops
    print(f"norm_prep_moe M={M} shared={shared}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(40 + M)
    pairs = torch.randn(M * K, H, device="cuda", generator=g) * .1
    sh = torch.randn(M, H, device="cuda", generator=g) * .1 if shared else None
    res_in = torch.randn(M, H, device="cuda", generator=g).bfloat16()
    gamma = (torch.rand(H, device="cuda", generator=g) + .5).bfloat16()
    wsb = ops.gemm_kquant_a_ws_bytes(M, H)
    outs = []
    for fused in (False, True):
        x = torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
        res_out = torch.empty_like(x)
        y = torch.empty_like(x)
        ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
        if fused:
            L.norm_prep_moe(pairs, sh, K, gamma, ws, 1e-6, x_out=x, res_in=res_in,
                            res_out=res_out, y_out=y)
        else:
            L.moe_combine(pairs, sh, x, M, K, H)
            L.norm_prep(x, gamma, ws, 1e-6, res_in=res_in, res_out=res_out, y_out=y)
        torch.cuda.synchronize()
        outs.append((x, res_out, y, ws))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("M,Hd,shared", [(9, 2048, True), (1, 2048, True), (15, 2048, False),
                                         (11, 512, True), (5, 4096, True)])
def test_norm_router_plan_equals_separate_launches(gpu, M, Hd, shared):
    """Post-attention norm + router GEMV + routing/plan in one launch (every workgroup
    normalises the rows itself; the last one to finish routes and plans) gives the bits of
    norm_prep, dense_gemv and moe_route_plan, on two launches in a row."""
    from snowllm_amd import layers as L
    print(f"norm+router+plan M={M} H={Hd} shared={shared}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + Hd)
    N = E + (1 if shared else 0)
    x = torch.randn(M, Hd, device="cuda", generator=g).bfloat16()
    res = (torch.randn(M, Hd, device="cuda", generator=g) * 4).bfloat16()
    gamma = (1 + 0.1 * torch.randn(Hd, device="cuda", generator=g)).bfloat16()
    router = (torch.randn(N, Hd, device="cuda", generator=g) / Hd ** 0.5).bfloat16()
    rw = L.dense_shuffle(router)
    from snowllm_amd import ops
    nws = ops.gemm_kquant_a_ws_bytes(M, Hd)

    def bufs():
        return dict(res_out=torch.zeros(M, Hd, dtype=torch.bfloat16, device="cuda"),
                    y=torch.zeros(M, Hd, dtype=torch.bfloat16, device="cuda"),
                    ws=torch.zeros(nws, dtype=torch.uint8, device="cuda"),
                    logits=torch.zeros(M, N, device="cuda"),
                    w=torch.zeros(M, K, device="cuda"),
                    ids=torch.zeros(M, K, dtype=torch.int32, device="cuda"),
                    sw=torch.zeros(M, device="cuda") if shared else None,
                    plan=torch.zeros(L.MOE_PLAN_BYTES, dtype=torch.uint8, device="cuda"))

    a = bufs()
    L.norm_prep(x, gamma, a["ws"], 1e-6, res_in=res, res_out=a["res_out"], y_out=a["y"])
    L.dense_gemv(L.WT_BF16, rw, a["y"], a["logits"], M, N, Hd)
    L.moe_route_plan(a["logits"], E, K, a["w"], a["ids"], a["sw"], a["plan"])
    outs = []
    for _ in range(2):
        b = bufs()
        L.norm_router_plan(x, gamma, b["ws"], 1e-6, rw, b["logits"], K, b["w"], b["ids"], b["sw"],
                           b["plan"], res_in=res, res_out=b["res_out"], y_out=b["y"])
        outs.append(b)
    torch.cuda.synchronize()
    for b in outs:
        for key in ("res_out", "y", "ws", "logits", "w", "ids") + (("sw",) if shared else ()):
            assert torch.equal(a[key], b[key]), key
        # the plan, but for its epoch (the last word: every plan gets a new one)
        assert torch.equal(a["plan"][:-4], b["plan"][:-4])
    assert L.parse_plan(outs[1]["plan"])["n_slots"] == L.parse_plan(a["plan"])["n_slots"]
