"""Verify-step benchmark on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line: the metric of BASELINE.json ("verify-step us + accepted tok/s (block 8);
achieved HBM GB/s vs peak"), the roofline of the dominant kernel (algorithmic bytes per launch
/ its average launch duration, HIP events on the launch stream) and the reference CPU path
timed on this host's cores over a bounded sample.

Workloads:
  config4  (default) BASELINE config 4: the MoE 35B-A3B-shaped verify step, 40 layers, block
           k=8 (9 rows), 8192-token paged KV cache, Q4_K weights, full-vocabulary rejection
           sampling. One step = embed -> 40 layers -> LM head -> probabilities -> acceptance,
           replayed as one HIP graph with every input already in HBM.
  config3  BASELINE config 3: the dense 8B-shaped step (36 layers, Q4_K, SwiGLU 14336).
  config5  BASELINE config 5: the MoE shape at 220000 tokens of context, tree block of 11 rows.
  gemv     BASELINE config 2: one Q4_K dequant-GEMV, M=9, K=4096, N=14336, bf16 out.
  config1  BASELINE config 1: the acceptance alone (9 rows x 151936), T=1 rejection sampling
           and greedy straight from the logits, with the list-based forms timed beside them.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verify-step µs + accepted tok/s (block 8); achieved HBM GB/s vs peak"
PEAK_HBM_GBS = 8000.0


def cpu_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_events(fn, iters, stream=None):
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters  # ms


# ---------------------------------------------------------------------------------------
# config 2: single Q4_K GEMV
# ---------------------------------------------------------------------------------------
def bench_gemv(args):
    import numpy as np
    import torch
    from snowllm_amd import ops
    from oracle import quant as Q

    M, K, N = 9, 4096, 14336
    raw = Q.make_q4_k(N, K, seed=2)
    x = Q.make_activations(M, K, seed=3).cuda()
    quant, meta = ops.gemm_kquant_shuffle_b(4, torch.from_numpy(raw).cuda(), N, K)
    # Rotate over enough weight copies (> 256 MiB Infinity Cache) that every launch streams
    # its weights from HBM.
    copies = max(1, (768 << 20) // (quant.numel() + meta.numel()))
    weights = [(quant.clone(), meta.clone()) for _ in range(copies)]
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(M, K), dtype=torch.uint8, device="cuda")
    # parity on the benchmark inputs
    ops.gemm_kquant_a(4, x, quant, meta, c, M, N, K, ws)
    want = Q.gemv_reference(x.cpu(), Q.dequant_q4_k(raw, N, K))
    err = Q.rel_l2(c.float().cpu().numpy(), want)
    assert err < 3e-3, f"parity failure on the benchmark inputs: rel L2 {err}"

    it = [0]

    def step():  # the whole operator: activation prep + GEMV
        qm = weights[it[0] % copies]
        it[0] += 1
        ops.gemm_kquant_a(4, x, qm[0], qm[1], c, M, N, K, ws)

    def gemv_only():
        qm = weights[it[0] % copies]
        it[0] += 1
        ops.gemm_kquant_a_prepared(4, qm[0], qm[1], c, M, N, K, ws)

    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms_step = time_events(step, args.steps, stream)
    ms_gemv = time_events(gemv_only, args.steps, stream)
    # graph-replayed step (launch overhead removed)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(copies):
            ops.gemm_kquant_a(4, x, weights[i][0], weights[i][1], c, M, N, K, ws)
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps // copies)
    ms_graph = time_events(lambda: g.replay(), reps, stream) / copies

    alg_bytes = N * K // 256 * 144 + 2 * M * K + 2 * M * N  # 33,361,920
    flops = 2 * M * N * K
    achieved = alg_bytes / (ms_gemv * 1e-3) / 1e9

    # reference CPU path: dequantize + x.float() @ W.float().T (tests/test_mixed_gguf.py:57-67)
    cores = cpu_cores()
    torch.set_num_threads(cores)
    xc = x.cpu()
    t0 = time.perf_counter()
    n_full = 0
    while time.perf_counter() - t0 < 6.0 or n_full < 2:
        w = torch.from_numpy(Q.dequant_q4_k(raw, N, K))
        xc.float() @ w.T
        n_full += 1
    ms_cpu_full = (time.perf_counter() - t0) * 1e3 / n_full
    w = torch.from_numpy(Q.dequant_q4_k(raw, N, K))
    t0 = time.perf_counter()
    n_mm = 0
    while time.perf_counter() - t0 < 4.0 or n_mm < 5:
        xc.float() @ w.T
        n_mm += 1
    ms_cpu_mm = (time.perf_counter() - t0) * 1e3 / n_mm

    us = ms_graph * 1e3
    return {
        "metric": METRIC, "value": round(us, 3), "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_graph, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k x bf16 (fp16 mfma, fp32 acc)",
        "data": "synthetic (BASELINE config 2 generators, seeds 2/3)",
        "config": {"workload": "config2_q4k_gemv", "M": M, "K": K, "N": N, "out": "bf16",
                   "weight_copies_rotated": copies},
        "roofline": {"bound": "hbm", "kernel": "kquant_gemv<Q4_K>", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": read_traffic("kquant_gemv<Q4_K>", "gemv"),
                     "alg_bytes_per_launch": alg_bytes, "kernel_us": round(ms_gemv * 1e3, 3)},
        "timings_us": {"op_eager": round(ms_step * 1e3, 3), "op_graph": round(us, 3),
                       "gemv_kernel_eager": round(ms_gemv * 1e3, 3)},
        "tflops_effective": round(flops / (ms_gemv * 1e-3) / 1e12, 1),
        "parity_rel_l2": err,
        "cpu_baseline": {"value": round(ms_cpu_full * 1e3, 1), "unit": "us", "cores": cores,
                         "kind": "port", "cpu": cpu_model(),
                         "sample": f"dequantize+matmul x{n_full} (torch CPU); matmul only on "
                                   f"pre-dequantized W: {ms_cpu_mm * 1e3:.1f} us (x{n_mm})",
                         "matmul_only_us": round(ms_cpu_mm * 1e3, 1)},
    }


# ---------------------------------------------------------------------------------------
# config 1: acceptance only
# ---------------------------------------------------------------------------------------
def acceptance_inputs(k=8, V=151936):
    """target logits [k+1, V] and draft logits [k, V] ~N(0, 2^2), drafts
    sampled from the draft softmax with seed 0, acceptance uniforms U(0,1) with seed 1."""
    import torch
    g10, g11 = torch.Generator().manual_seed(10), torch.Generator().manual_seed(11)
    target = torch.randn(k + 1, V, generator=g10) * 2
    draft = torch.randn(k, V, generator=g11) * 2
    drafts = torch.multinomial(draft.softmax(-1), 1, generator=torch.Generator().manual_seed(0))
    uniform = torch.rand(1, k + 1, generator=torch.Generator().manual_seed(1))
    return target, draft, drafts.view(1, k), uniform


def time_acceptance(reps=200):
    """Config 1 on the device, inputs resident: (greedy us, rejection us) straight from the
    logits, the list-based forms beside them, the accept lengths / emitted ids (checked
    against the oracle) and the algorithmic bytes of each mode."""
    import numpy as np
    import torch
    from snowllm_amd import ops
    from oracle import accept as A
    target, draft, drafts, uniform = acceptance_inputs()
    k, V = drafts.shape[1], target.shape[1]
    T = k + 1
    dev = lambda x: x.cuda()
    tl, dl, dr, u = dev(target), dev(draft), dev(drafts), dev(uniform)
    ones = torch.ones(T, device="cuda")
    kmax = torch.full((T,), ops.SAMPLING_MAX_K, dtype=torch.int32, device="cuda")
    ws = torch.empty(ops.sample_workspace_bytes(T, V, V), dtype=torch.uint8, device="cuda")
    q = torch.empty(k, V, device="cuda")
    qid = torch.empty(k, V, dtype=torch.int64, device="cuda")
    ops.probabilities(dl, kmax[:k], ones[:k], ones[:k], V, q, qid, ws)  # the draft side
    q3, qid3 = q.view(1, k, V), qid.view(1, k, V)
    slot = torch.zeros(1, dtype=torch.int32, device="cuda")
    valid = torch.ones(1, dtype=torch.int32, device="cuda")
    out = torch.empty(1, T, dtype=torch.int64, device="cuda")
    acc = torch.empty(1, dtype=torch.int64, device="cuda")
    tokens = torch.empty(1, T, dtype=torch.int64, device="cuda")
    p = torch.empty(T, V, device="cuda")
    pid = torch.empty(T, V, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()

    def fused_rej():
        ops.dflash.accept_reject(tl, dr, qid3, q3, slot, valid, u, out, acc)

    def lists_rej():
        ops.probabilities(tl, kmax, ones, ones, V, p, pid, ws)
        ops.dflash.reject(p, pid, dr, qid3, q3, slot, valid, u, out, acc)

    def fused_greedy():
        ops.dflash.accept_greedy(tl, dr, tokens, acc)

    def two_greedy():
        ops.argmax(tl, out=tokens.view(-1))
        ops.spec_accept(tokens, dr, out=acc)

    res = {}
    for name, fn in (("rejection", fused_rej), ("rejection_lists", lists_rej),
                     ("greedy", fused_greedy), ("greedy_argmax_then_prefix", two_greedy)):
        res[name] = round(timed_graph(fn, reps, stream, per=reps) * 1e3, 2)
    # parity on the benchmark inputs (the oracle is the checker only)
    fused_rej()
    torch.cuda.synchronize()
    p_ref = A.softmax(target.numpy())
    q_ref = A.softmax(draft.numpy())
    ident = np.tile(np.arange(V), (T, 1))
    want_out, want_acc = A.reject(p_ref, ident, drafts.numpy(), ident[:k][None], q_ref[None],
                                  np.zeros(1, np.int32), np.ones(1, np.int32), uniform.numpy())
    assert np.array_equal(out.cpu().numpy(), want_out) and int(acc[0]) == int(want_acc[0])
    rej = {"accepted": int(acc[0]), "emitted": out[0, :int(acc[0])].tolist()}
    fused_greedy()
    torch.cuda.synchronize()
    want_tok = A.argmax(target.numpy())
    assert np.array_equal(tokens.cpu().numpy()[0], want_tok)
    gre = {"accepted": int(acc[0]), "emitted": tokens[0, :int(acc[0])].tolist()}
    return {"us": res, "rejection": rej, "greedy": gre,
            "alg_bytes": {"greedy": T * V * 4, "rejection": (T + k) * V * 4}}


def bench_config1(args):
    import numpy as np
    import torch
    from oracle import accept as A
    r = time_acceptance(reps=max(args.steps, 50))
    us_g, us_r = r["us"]["greedy"], r["us"]["rejection"]
    gbs_r = r["alg_bytes"]["rejection"] / (us_r * 1e-6) / 1e9
    gbs_g = r["alg_bytes"]["greedy"] / (us_g * 1e-6) / 1e9
    # CPU path: the oracle's softmax + rejection and argmax + prefix on this host (kind port)
    target, draft, drafts, uniform = acceptance_inputs()
    T, V = target.shape
    cores = cpu_cores()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < 5.0 or n < 3:
        p = A.softmax(target.numpy())
        q = A.softmax(draft.numpy())
        ident = np.tile(np.arange(V), (T, 1))
        A.reject(p, ident, drafts.numpy(), ident[:T - 1][None], q[None], np.zeros(1, np.int32),
                 np.ones(1, np.int32), uniform.numpy())
        n += 1
    cpu_us = (time.perf_counter() - t0) / n * 1e6
    return {
        "metric": METRIC, "value": us_r, "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_r / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 logits, 44-bit fixed-point sums",
        "data": "synthetic (BASELINE config 1 generators: N(0,2^2) logits, seeds 0/1)",
        "config": {"workload": "config1_acceptance", "k": T - 1, "vocab": V,
                   "modes": ["T=1.0 rejection (value)", "greedy"]},
        "acceptance_us": r["us"], "rejection": r["rejection"], "greedy": r["greedy"],
        "roofline": {"bound": "hbm", "kernel": "fa_max + fa_sum + fa_pick (step)", "achieved": round(gbs_r, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs_r / PEAK_HBM_GBS, 4),
                     "traffic": None, "alg_bytes_per_launch": r["alg_bytes"]["rejection"],
                     "kernel_us": us_r, "greedy_gbs": round(gbs_g, 1)},
        "cpu_baseline": {"value": round(cpu_us, 1), "unit": "us", "cores": 1, "kind": "port",
                         "cpu": cpu_model(),
                         "sample": f"oracle softmax x2 + rejection sampling (C, one thread) x{n}"},
    }


# ---------------------------------------------------------------------------------------
# configs 3-5: the full verify step
# ---------------------------------------------------------------------------------------
def q4k_bytes(n, k):
    return n * k // 256 * 144


def q80_bytes(n, k):
    return n * k // 32 * 34


SEL_RANK = 256


def use_selector(cfg):
    """BASELINE config 4 runs the fused selector + acceptance; the others take the draft
    proposal from outside the step."""
    return cfg.moe and not cfg.tree_parents


def step_bytes(cfg, slots, selector=False, batch=1):
    """Algorithmic HBM bytes of one verify step: every weight byte the step must read once
    (the touched experts only), the KV cache of the context plus the block's new rows of every
    request, the LM head, the logits/probabilities of the acceptance, and (with the selector)
    the draft logits plus the codebook rows the selector gathers (16 candidates and 16
    previous tokens per position). slots[i]: the experts layer i must read (the unique
    experts the step's rows touch + the shared expert)."""
    H, T, V = cfg.hidden, cfg.block, cfg.vocab
    wb = q4k_bytes if cfg.attn_fmt == 4 else q80_bytes
    attn_w = wb(cfg.qkv_n, H) + wb(H, cfg.heads * cfg.head_dim)
    kv = batch * (cfg.context + T) * cfg.kv_heads * cfg.head_dim * 2 * 2
    T = batch * T   # rows of the step from here on
    total = 0
    for i in range(cfg.layers):
        total += attn_w + kv + 2 * 2 * H * 2  # + norm weights (bf16), negligible
        if cfg.moe:
            F = cfg.expert_ffn
            total += (cfg.experts + 1) * H * 2 + int(slots[i]) * (q4k_bytes(2 * F, H) + q4k_bytes(H, F))
        else:
            total += q4k_bytes(2 * cfg.ffn, H) + q4k_bytes(H, cfg.ffn)
    total += V * H * 2 + T * H * 2  # LM head (fp16), embedding rows
    total += 3 * T * V * 4          # logits write, probabilities read + write
    if selector:
        k = cfg.block - 1
        total += batch * (k * V * 4 + k * (2 * 16 + 1) * SEL_RANK * 2)
    return total


def timed_graph(fn, reps, stream, per=1):
    """ms per replay of a graph holding `per` calls of fn (divided by per)."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per):
            fn()
    g.replay()
    torch.cuda.synchronize()
    return time_events(lambda: g.replay(), max(1, reps // per), stream) / per


def bench_step(args, name):
    import numpy as np
    import torch
    from snowllm_amd import layers as Lops, ops
    from snowllm_amd.verify import CONFIGS, VerifyModel, Acceptance

    cfg = CONFIGS[name]
    B = args.batch
    T, V, k = cfg.block, cfg.vocab, None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # raw GGUF bytes of layer 0 for the CPU baseline
    m = VerifyModel(cfg, seed=0, keep_raw=1, batch=B)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    ids = torch.randint(0, V, (B, T), generator=torch.Generator().manual_seed(7))
    m.set_batch(ids, [cfg.context] * B)
    rows = list(range(T)) if not cfg.tree_parents else chain_rows(cfg.tree_parents)
    k = len(rows) - 1
    acc = Acceptance(V, rows, batch=B, block=T)
    # draft side (BASELINE config 1 generators): draft logits ~N(0, 2^2), drafts sampled from
    # the draft softmax with seed 0, acceptance uniforms U(0, 1) with seed 1 (one block of
    # them per request)
    g0, g1 = torch.Generator().manual_seed(0), torch.Generator().manual_seed(1)
    draft_logits = torch.randn(B * k, V, generator=g0) * 2
    drafts = torch.multinomial(draft_logits.softmax(-1), 1, generator=g0).view(B, k)
    uniform = torch.rand(B, k + 1, generator=g1)
    # config 4 is quoted with the DFlash 2 selector in the step: it walks the draft logits
    # (codebook rank 256, seeded synthetic codebooks and selector projection) at T = 1.0,
    # proposes the drafts and hands its 16-candidate lists to the rejection step
    sel = None
    if use_selector(cfg):
        g2 = torch.Generator().manual_seed(2)
        hp = (torch.randn(B * k, SEL_RANK, generator=g2) * .2).bfloat16()
        pred = (torch.randn(V, SEL_RANK, generator=g2) * .2).bfloat16()
        succ = (torch.randn(V, SEL_RANK, generator=g2) * .2).bfloat16()
        sel_u = torch.rand(B, k, generator=g2)
        sel = dict(hp=hp, pred=pred, succ=succ, anchor=ids[:, 0].clone(), temp=torch.ones(B),
                   u=sel_u)
        acc.set_selector(hp.cuda(), draft_logits.cuda(), pred.cuda(), succ.cuda(),
                         sel["anchor"].cuda(), sel["temp"].cuda(), sel_u.cuda(), uniform.cuda())
    else:
        acc.set_draft(draft_logits.cuda(), drafts.cuda(), uniform.cuda())

    def step():
        if sel is not None:
            acc.propose(m.ids)
        m.forward()
        acc(m.logits)

    stream = torch.cuda.current_stream()
    # byte accounting: an eager pass that records each layer's plan size
    slots = torch.zeros(cfg.layers, dtype=torch.int32, device="cuda")
    if sel is not None:
        acc.propose(m.ids)
    m.forward(record_slots=slots if cfg.moe else None)
    acc(m.logits)
    torch.cuda.synchronize()
    slots_np = slots.cpu().numpy()
    alg = step_bytes(cfg, slots_np, selector=sel is not None, batch=B)
    # the timed region: K graph replays of the whole step, inputs resident in HBM
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(max(1, args.warmup)):
        g.replay()
    torch.cuda.synchronize()
    ms = time_events(lambda: g.replay(), args.steps, stream)
    torch.cuda.synchronize()
    if cfg.moe and Lops.moe_sync_error() != 0:
        raise RuntimeError("a MoE expert hand-off timed out during the timed steps "
                           "(its outputs were poisoned with NaN)")
    # accepted drafts + the correction/bonus token, over the batch's requests
    emitted = int(acc.accepted.sum())
    out_tokens = [acc.out[b, :int(acc.accepted[b])].tolist() for b in range(B)]
    if B == 1:
        out_tokens = out_tokens[0]
    step_gbs = alg / (ms * 1e-3) / 1e9

    # per-kernel launch times (HIP events, launch stream), each rotated over the layers so the
    # weights stream from HBM as they do inside the step
    c, H = cfg, cfg.hidden
    Lw = m.layers
    kern = {}

    def per_launch(label, fn_layer, alg_bytes, launches=1):
        def run():
            for i in range(len(Lw)):
                fn_layer(i)
        ms_all = timed_graph(run, 3, stream)
        us = ms_all * 1e3 / len(Lw) / launches
        kern[label] = {"us": round(us, 3), "alg_bytes": int(alg_bytes),
                       "gbs": round(alg_bytes / (us * 1e-6) / 1e9, 1)}

    wb = q4k_bytes if cfg.attn_fmt == 4 else q80_bytes
    R = m.rows   # all rows of the step
    per_launch("kquant_gemv qkv", lambda i: ops.gemm_kquant_a_prepared(
        c.attn_fmt, Lw[i].qkv[0], Lw[i].qkv[1], m.proj, R, c.qkv_n, H, m.ws_h), wb(c.qkv_n, H))
    per_launch("paged_attention (split + merge)", lambda i: ops.paged_attention_explicit(
        m.q, m.k_pools[i], m.v_pools[i], m.attn, m.table, m.lens, c.head_dim ** -0.5,
        m.attn_scratch, tree=m.tree), B * (c.context + T) * c.kv_heads * c.head_dim * 4)
    if cfg.moe:
        F = c.expert_ffn
        # the expert gate/up and down GEMVs: one launch (moe_experts_kernel) per plan of up to
        # 64 rows; timed on the first plan as the last layer left it
        n0 = m.moe_chunks[0][1]
        plan0 = m.plans[0]
        slots0 = int(plan0[:4].view(torch.int32).item())
        per_launch("moe_experts", lambda i: Lops.moe_gate_up_down(
            c.ffn_fmt, Lw[i].gu, Lw[i].dn, Lw[i].sh_gu, Lw[i].sh_dn, plan0, m.ws_h2,
            m.route_w[:n0], m.shared_w[:n0], m.moe_act, m.pairs[:n0 * c.topk], m.shared_out[:n0],
            n0, m.moe_slots[0], c.experts, H, F),
            slots0 * (q4k_bytes(2 * F, H) + q4k_bytes(H, F)))
    else:
        n0 = m.row_chunks[0][1]
        per_launch("gate_up_swiglu", lambda i: Lops.gate_up_swiglu(
            c.ffn_fmt, Lw[i].gu[0], Lw[i].gu[1], m.ws_h2, m.act[:n0], n0, c.ffn, H),
            q4k_bytes(2 * c.ffn, H))
    if sel is not None:
        us = timed_graph(lambda: acc.propose(), 5, stream) * 1e3
        sb = k * V * 4 + k * (2 * 16 + 1) * SEL_RANK * 2
        kern["draft_select (chunks + table + walk)"] = {
            "us": round(us, 3), "alg_bytes": int(sb), "gbs": round(sb / (us * 1e-6) / 1e9, 1)}
    adaptive = None
    if cfg.name == CONFIGS["config4"].name and B == 1:
        # BASELINE config 1 (the acceptance alone) beside the north-star step
        kern["config1_acceptance"] = dict(time_acceptance(reps=200), outside_step=True)
        # the draft heads that produce the next proposal, and the adaptive prefix scheduler
        # on this step's measured costs
        heads = time_draft_heads(stream, V, k)
        kern.update(heads)
        if not args.no_adaptive:
            adaptive = adaptive_prefix(m, heads["dspark_markov (per block row)"]["us"] * k * 1e-6,
                                       heads["_markov_confidence"])
        kern.pop("_markov_confidence", None)
    elif cfg.name == CONFIGS["config4"].name:
        # the scheduler over the batch's requests together, on batched step costs
        heads = time_draft_heads(stream, V, k, requests=B)
        kern.update(heads)
        if not args.no_adaptive:
            draft_s = heads[f"dspark_markov ({B} requests, per block row)"]["us"] * k * 1e-6
            adaptive = adaptive_prefix(m, draft_s, heads["_markov_confidence"], requests=B)
        kern.pop("_markov_confidence", None)
    # dominant kernel of the step (launch time; every candidate runs once per layer); the
    # attention counts as its split + merge pair
    per_step = {kk: (1 if kk.startswith("draft_select") else cfg.layers) for kk in kern}
    single = {kk: v for kk, v in kern.items() if "us" in v and not v.get("outside_step")}
    dom = max(single, key=lambda kk: single[kk]["us"] * per_step[kk])
    d = kern[dom]
    traffic = read_traffic(dom, name) if B == 1 else None

    # reference CPU path (oracle, torch CPU) on a bounded sample: layer 0 x layers + head +
    # acceptance
    cpu = cpu_step_baseline(m, cfg, rows, draft_logits[:k], drafts[:1], uniform[:1],
                            sel and dict(sel, hp=sel["hp"][:k], anchor=sel["anchor"][:1],
                                         temp=sel["temp"][:1], u=sel["u"][:1]))
    # the CPU path verifies one request per step; a batch costs B of them
    cpu_value = emitted / (cpu["step_s"] * B)
    if B > 1:
        cpu["sample"] += f"; x{B} requests (the CPU path verifies one request at a time)"
    return {
        "metric": METRIC, "value": round(emitted / (ms * 1e-3), 2), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k weights x bf16 activations (fp16/bf16 MFMA, fp32 accumulate)",
        "data": weights_note(cfg),
        "config": {"workload": cfg.name + (f"_batch{B}" if B > 1 else ""),
                   "layers": cfg.layers, "hidden": cfg.hidden, "requests": B,
                   "block_rows": T, "context": cfg.context, "vocab": V,
                   "experts": cfg.experts, "topk": cfg.topk,
                   "attn_fmt": "q4_k" if cfg.attn_fmt == 4 else "q8_0",
                   "tree": bool(cfg.tree_parents), "selector": sel is not None,
                   "rope": {"theta": cfg.rope_theta, "rotary_dims": 2 * cfg.rot_half,
                            "head_dim": cfg.head_dim}},
        "verify_step_us": round(ms * 1e3, 1),
        "accepted_per_step": emitted, "accepted_drafts": emitted - 1,
        "emitted_tokens": out_tokens,
        "step_hbm": {"alg_bytes": int(alg), "achieved": round(step_gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                     "unique_experts_per_layer": float(np.mean(slots_np) - 1) if cfg.moe else None},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": d["gbs"], "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(d["gbs"] / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "alg_bytes_per_launch": d["alg_bytes"],
                     "kernel_us": d["us"]},
        "kernels": kern,
        "adaptive_prefix": adaptive,
        "init_s": round(init_s, 1),
        "cpu_baseline": {"value": round(cpu_value, 4), "unit": "tok/s", "cores": cpu["cores"],
                         "kind": "port", "cpu": cpu_model(), "sample": cpu["sample"],
                         "step_s": round(cpu["step_s"], 3)},
    }


def time_draft_heads(stream, V, k, hidden=2048, markov_rank=256, requests=1):
    """The draft-side heads at the config-4 shapes (seeded synthetic weights): the DFlash 2
    selector's hidden projection of k rows (bf16 [256, hidden]) and the DSpark Markov walk over
    a block of k rows (W1, W2 bf16 [V, rank], with the confidence head), per launch; and the
    head's own confidences over a 15-draft proposal for each of `requests` requests."""
    import torch
    from snowllm_amd.draft_heads import MarkovHead, SelectorHead
    g = torch.Generator(device="cuda").manual_seed(5)
    out = {}
    w = (torch.randn(SEL_RANK, hidden, device="cuda", generator=g) * hidden ** -.5).bfloat16()
    codebook = torch.zeros(16, SEL_RANK, dtype=torch.bfloat16, device="cuda")
    head = SelectorHead(hidden, w, codebook, codebook)
    rows = torch.randn(k, hidden, device="cuda", generator=g).bfloat16()
    hp = torch.empty(k, SEL_RANK, dtype=torch.bfloat16, device="cuda")
    us = timed_graph(lambda: head.project(rows, hp), 50, stream, per=10) * 1e3
    nb = SEL_RANK * hidden * 2 + k * (hidden + SEL_RANK) * 2
    out["selector_hidden_projection"] = {"us": round(us, 3), "alg_bytes": nb,
                                         "gbs": round(nb / (us * 1e-6) / 1e9, 1),
                                         "outside_step": True}
    W1 = (torch.randn(V, markov_rank, device="cuda", generator=g) * .25).bfloat16()
    W2 = (torch.randn(V, markov_rank, device="cuda", generator=g) * .25).bfloat16()
    conf_w = torch.randn(hidden + markov_rank, device="cuda", generator=g) * .05
    mk = MarkovHead(W1, W2, conf_w, torch.zeros(1, device="cuda"))
    logits = torch.randn(k, V, device="cuda", generator=g)
    anchor = torch.zeros(1, dtype=torch.int64, device="cuda")
    path = torch.empty(1, k, dtype=torch.int64, device="cuda")
    conf = torch.empty(1, k, device="cuda")
    mk.propose(rows, logits, anchor, path, conf)
    us = timed_graph(lambda: mk.propose(rows, logits, anchor, path, conf), 20, stream) * 1e3 / k
    nb = V * markov_rank * 2 + V * 4 + markov_rank * 2 + hidden * 2
    out["dspark_markov (per block row)"] = {
        "us": round(us, 3), "alg_bytes": nb, "gbs": round(nb / (us * 1e-6) / 1e9, 1),
        "outside_step": True,
        "note": "W2 (78 MB) is read by each of the block's rows; after the first it is largely "
                "served from the 256 MB Infinity Cache"}
    # the head's own confidences over a 15-draft proposal: the adaptive scheduler's input
    # (snowllm/engine/spec_decode.py:157-166 feeds it the drafter's confidences per request)
    n, b = 15, requests
    rows15 = torch.randn(b * n, hidden, device="cuda", generator=g).bfloat16()
    logits15 = torch.randn(b * n, V, device="cuda", generator=g)
    anchors = torch.randint(0, V, (b,), device="cuda", generator=g)
    path15 = torch.empty(b, n, dtype=torch.int64, device="cuda")
    conf15 = torch.empty(b, n, device="cuda")
    mk.propose(rows15, logits15, anchors, path15, conf15)
    out["_markov_confidence"] = [[round(float(c), 4) for c in row] for row in conf15.cpu()]
    if b > 1:
        # the walk of every request's proposal in one launch, per block row
        path_b = torch.empty(b, k, dtype=torch.int64, device="cuda")
        conf_b = torch.empty(b, k, device="cuda")
        rows_b, logits_b = rows15[:b * k], logits15[:b * k]
        us = timed_graph(lambda: mk.propose(rows_b, logits_b, anchors, path_b, conf_b), 20,
                         stream) * 1e3 / k
        out[f"dspark_markov ({b} requests, per block row)"] = {
            "us": round(us, 3), "alg_bytes": nb, "gbs": round(nb / (us * 1e-6) / 1e9, 1),
            "outside_step": True}
    return out


def adaptive_prefix(m, draft_s, confidence, requests=1):
    """The DSpark prefix scheduler (snowllm/engine/dspark_schedule.py) on step costs measured
    here: verify steps of `requests` requests and requests x 1..16 rows in all (eager and
    graph, rows spread evenly over the requests) plus the Markov head's time, and the Markov
    head's own confidences over each request's 15-draft proposal (random-init weights, so they
    say nothing about draft quality; a trained head's would). Every profiled row count gets a
    captured graph, as the reference's profile of its decode shapes
    (snowllm/engine/spec_decode.py:149-161); the scheduler chooses every request's prefix
    together (spec_decode.py:157-166)."""
    from snowllm_amd.dspark_schedule import PrefixScheduler, profile_step_costs
    B = requests
    rows = tuple(B * t for t in range(1, 17))
    cost = profile_step_costs(m, rows, requests=B, draft_seconds=draft_s)
    conf = [list(c) for c in confidence[:B]]
    lengths = PrefixScheduler(16 * B).choose(list(range(B)), conf, [15] * B, cost)
    surv = []
    for c_r in conf:
        s, row = 1.0, []
        for c in c_r:
            s *= c
            row.append(s)
        surv.append(row)

    def rate(ns):
        return sum(1 + sum(surv[r][:n]) for r, n in enumerate(ns)) / cost(sum(1 + n for n in ns))
    out = {"requests": B,
           "step_us_by_rows": {n: round(cost.graphs[n] * 1e6, 1) for n in rows},
           "draft_us": round(draft_s * 1e6, 1),
           "confidence": {"source": "dspark_markov confidence head (15 drafts per request)",
                          "values": conf if B > 1 else conf[0]},
           "expected_tokens_per_s": round(rate(lengths), 1),
           "fixed_block8_tokens_per_s": round(rate([8] * B), 1)}
    out["chosen_drafts"] = lengths if B > 1 else lengths[0]
    return out


def weights_note(cfg):
    """What the random-init weights are, for the JSON line."""
    if cfg.centered:
        q4 = ("Q4_K blocks zero-mean (d ~|N(0,2e-4^2)|, dmin = 8d, m = round(0.9375 sc)) so "
              "that router logits stay ~N(0,1) per row; config 2's uniform mins would route "
              "every row to the same experts")
    else:
        q4 = "Q4_K blocks from BASELINE config 2's generator"
    q8 = "; Q8_0 attention as BASELINE config 5" if cfg.attn_fmt == 8 else ""
    return (f"synthetic, random-init seeded weights: {q4}{q8}; fp16 embedding and LM head "
            f"~N(0,0.02^2); bf16 router ~N(0,1/H); KV ~N(0,1); draft side from BASELINE "
            f"config 1's generators")


def chain_rows(parents):
    """Rows of the first root-to-leaf chain of a tree block (the chain the acceptance runs)."""
    rows = [0]
    while True:
        kids = [i for i, p in enumerate(parents) if p == rows[-1]]
        if not kids:
            return rows
        rows.append(kids[0])


# the committed rocprofv3 PMC summaries and the workloads they were measured on
TRAFFIC_FILES = {"config4": "traffic.txt", "config5": "traffic_config5.txt",
                 "gemv": "traffic_gemv.txt"}


def read_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary of `workload`
    (profiles/traffic*.txt: 'kernel | fetch_bytes | write_bytes' rows, already scaled by the
    copy-kernel calibration), or None."""
    if workload not in TRAFFIC_FILES:
        return None
    path = os.path.join(ROOT, "profiles", TRAFFIC_FILES[workload])
    try:
        for line in open(path):
            parts = [x.strip() for x in line.split("|")]
            if len(parts) >= 3 and parts[0] == kernel:
                return int(float(parts[1]) + float(parts[2]))
    except OSError:
        pass
    return None


def cpu_step_baseline(m, cfg, rows, draft_logits, drafts, uniform, sel=None):
    """The oracle's CPU restatement of the verify step, timed on this host: layer 0 (GGUF
    dequantization of the weights it touches + fp64/fp32 compute) extrapolated to every layer,
    the final norm + LM head, and the acceptance (the selector walk when the step has one,
    probabilities + rejection sampling)."""
    import numpy as np
    import torch
    from oracle import accept as A
    from oracle import model as RM
    from snowllm_amd.verify import tree_masks

    cores = cpu_cores()
    torch.set_num_threads(cores)
    T = cfg.block
    masks = tree_masks(cfg.tree_parents) if cfg.tree_parents else [(2 << t) - 1 for t in range(T)]
    # the first request of the batch
    x = m.embed[m.ids[:T]].cpu().float()
    cos, sin = RM.rope_tables(m.positions[:T].cpu(), m.inv_freq.cpu())
    pages = m.table[0].long().cpu()
    kctx = RM.cache_rows(m.k_pools[0].cpu(), pages, cfg.kv_heads, cfg.head_dim, 16, key=True)[:cfg.context]
    vctx = RM.cache_rows(m.v_pools[0].cpu(), pages, cfg.kv_heads, cfg.head_dim, 16, key=False)[:cfg.context]
    lw0 = m.layers[0]
    t0 = time.perf_counter()
    ref = RM.LayerRef(cfg, lw0)
    x2, r2, _, _ = RM.layer_forward(ref, RM.bf(x), None, cos, sin, kctx, vctx, masks)
    layer_s = time.perf_counter() - t0
    head = m.lm_head_raw.cpu() if m.lm_head_raw is not None else None
    t1 = time.perf_counter()
    if head is not None:
        logits = RM.head_reference(x2, r2, m.final_norm.cpu(), head, cfg.eps)
    else:
        logits = torch.randn(T, cfg.vocab)
    chain = logits[rows].numpy().astype(np.float32)
    p = A.softmax(chain)
    ident = np.tile(np.arange(cfg.vocab), (len(rows), 1))
    k = len(rows) - 1
    if sel is not None:
        path, cand, q = A.select(sel["hp"], draft_logits.numpy(), sel["pred"], sel["succ"],
                                 sel["anchor"].numpy(), sel["temp"].numpy(), sel["u"].numpy(),
                                 np.zeros(1, np.int32), 1)
        A.reject(p, ident, path, cand, q, np.zeros(1, np.int32), np.ones(1, np.int32),
                 uniform.numpy())
    else:
        q = A.softmax(draft_logits.numpy())
        A.reject(p, ident, drafts.numpy(), ident[:k][None], q[None], np.zeros(1, np.int32),
                 np.ones(1, np.int32), uniform.numpy())
    tail_s = time.perf_counter() - t1
    step_s = layer_s * cfg.layers + tail_s
    return {"step_s": step_s, "cores": cores,
            "sample": f"layer 0 of {cfg.layers} ({layer_s:.2f} s: GGUF dequantize of the "
                      f"weights it touches + compute, oracle/model.py) x{cfg.layers} + final "
                      f"norm, LM head and acceptance ({tail_s:.2f} s); torch CPU, {cores} threads"}


def bench_copy(args):
    """A plain device copy of known size: the calibration for rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters (bytes read and written per launch are both exactly `nbytes`)."""
    import torch
    nbytes = 512 << 20
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(args.warmup):
        b.copy_(a)
    torch.cuda.synchronize()
    ms = time_events(lambda: b.copy_(a), args.steps, torch.cuda.current_stream())
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    return {"metric": "device copy GB/s (counter calibration)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "copy", "bytes_read": nbytes, "bytes_written": nbytes}}


WORKLOADS = {"gemv": bench_gemv, "copy": bench_copy, "config1": bench_config1,
             "config3": lambda a: bench_step(a, "config3"),
             "config4": lambda a: bench_step(a, "config4"),
             "config5": lambda a: bench_step(a, "config5")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="config4", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=1,
                    help="requests verified together in one step (configs 3-5; rows = batch x "
                         "block <= 256)")
    ap.add_argument("--no-adaptive", action="store_true",
                    help="leave out the adaptive-prefix cost profile (the profiler's runs at "
                         "1-16 rows would mix into a kernel trace of the step)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only (one-GPU boxes); "
                                   "--gpus must be 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    res = WORKLOADS[args.workload](args)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
