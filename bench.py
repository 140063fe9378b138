"""Verify-step benchmark on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line: the metric of BASELINE.json ("verify-step us + accepted tok/s (block 8);
achieved HBM GB/s vs peak"), the roofline of the dominant kernel (algorithmic bytes per launch
/ its average launch duration, HIP events on the launch stream) and the reference CPU path
timed on this host's cores over a bounded sample.

Workloads:
  gemv   BASELINE config 2: one Q4_K dequant-GEMV, M=9, K=4096, N=14336, bf16 out.
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
                     "traffic": None, "alg_bytes_per_launch": alg_bytes,
                     "kernel_us": round(ms_gemv * 1e3, 3)},
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


WORKLOADS = {"gemv": bench_gemv}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gemv", choices=sorted(WORKLOADS))
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
