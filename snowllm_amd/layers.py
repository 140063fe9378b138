"""Layer operators of the verify step (embedding, RMSNorm, RoPE, QK-norm + paged KV write,
dense 16-bit GEMV, SwiGLU, MoE routing/experts). Shapes are explicit; see
snowllm/ops/{norm,rope,cache,embedding,inference,moe}.py for the reference operators whose
arithmetic these follow."""
import ctypes

import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream

WT_F16, WT_BF16 = 1, 2


def gather_embedding(ids, table, out):
    M = ids.numel()
    _chk(ids, "input ids", torch.int64, M)
    if table.dtype not in (torch.float16, torch.bfloat16):
        raise SnowLLMError("embedding table must be fp16 or bf16")
    V, H = table.shape
    _chk(out, "embedding out", torch.bfloat16, M, H)
    check(lib.snowverify_gather_embedding(_p(ids), _p(table), _p(out), M, V, H,
                                          int(table.dtype == torch.float16), _stream()),
          "gather_embedding")


def rmsnorm(x, gamma, out, eps, residual=None):
    M, H = x.shape
    _chk(x, "x", torch.bfloat16, M, H)
    _chk(gamma, "gamma", torch.bfloat16, H)
    _chk(out, "out", torch.bfloat16, M, H)
    check(lib.snowverify_rmsnorm(_p(x), _p(residual), _p(gamma), _p(out), M, H, eps, _stream()),
          "rmsnorm")


def norm_prep(x, gamma, ws, eps, *, res_in=None, res_out=None, y_out=None):
    """res_out = x + res_in; y = RMSNorm(res_out) * gamma; y -> GEMV operand workspace ws."""
    M, H = x.shape
    _chk(x, "x", torch.bfloat16, M, H)
    _chk(gamma, "gamma", torch.bfloat16, H)
    for t, n in ((res_in, "res_in"), (res_out, "res_out"), (y_out, "y_out")):
        if t is not None:
            _chk(t, n, torch.bfloat16, M, H)
    check(lib.snowverify_norm_prep(_p(x), _p(res_in), _p(res_out), _p(gamma), _p(y_out), _p(ws),
                                   M, H, eps, _stream()), "norm_prep")


def norm_prep_moe(pairs, shared_out, topk, gamma, ws, eps, *, x_out=None, res_in=None,
                  res_out=None, y_out=None):
    """norm_prep on the MoE layer's output, combined in the same launch: x = bf16(sum_k
    pairs[r * topk + k] + shared_out[r]) (-> x_out if given), then as norm_prep."""
    M, H = pairs.shape[0] // topk, pairs.shape[1]
    _chk(pairs, "pairs", torch.float32, M * topk, H)
    if shared_out is not None:
        _chk(shared_out, "shared_out", torch.float32, M, H)
    _chk(gamma, "gamma", torch.bfloat16, H)
    for t, n in ((x_out, "x_out"), (res_in, "res_in"), (res_out, "res_out"), (y_out, "y_out")):
        if t is not None:
            _chk(t, n, torch.bfloat16, M, H)
    check(lib.snowverify_norm_prep_moe(_p(pairs), _p(shared_out), topk, _p(x_out), _p(res_in),
                                       _p(res_out), _p(gamma), _p(y_out), _p(ws), M, H, eps,
                                       _stream()), "norm_prep_moe")


def rope_cos_sin(positions, inv_freq, cos, sin):
    M, half = cos.shape
    _chk(positions, "positions", torch.int64, M)
    _chk(inv_freq, "inv_freq", torch.float32, half)
    _chk(cos, "cos", torch.float32, M, half)
    _chk(sin, "sin", torch.float32, M, half)
    check(lib.snowverify_rope_cos_sin(_p(positions), _p(inv_freq), _p(cos), _p(sin), M, half,
                                      _stream()), "rope_cos_sin")


def qk_norm_rope_cache(proj, q_gamma, k_gamma, cos, sin, q, k_pool, v_pool, slots, eps):
    """proj [M, (Hq + 2 Hkv) D] = q|k|v -> q [M, Hq, D] (normed, rotated); k (normed,
    rotated) and v into the paged pools at slots (snowllm/ops/attention_full.py:736-784)."""
    M, Hq, D = q.shape
    Hkv = k_pool.shape[1]
    _chk(proj, "projection", torch.bfloat16, M, proj.shape[1])
    if proj.shape[1] < (Hq + 2 * Hkv) * D:
        raise SnowLLMError("projection is narrower than q|k|v")
    _chk(q, "q", torch.bfloat16, M, Hq, D)
    _chk(slots, "slot mapping", torch.int32, M)
    half = cos.shape[1]
    check(lib.snowverify_qk_norm_rope_cache(_p(proj), proj.shape[1], _p(q_gamma), _p(k_gamma),
                                            _p(cos), _p(sin), _p(q), _p(k_pool), _p(v_pool),
                                            _p(slots), M, Hq, Hkv, D, half, 16, eps, _stream()),
          "qk_norm_rope_cache")


def resolve_slots(block_tables, row_seq, row_pos, block_size, *, out=None):
    """slot = table[seq, pos // page] * page + pos % page (snowllm/ops/cache.py:40-53)."""
    M = row_seq.numel()
    _chk(block_tables, "block_tables", torch.int32)
    _chk(row_seq, "row_seq", torch.int32)
    _chk(row_pos, "row_pos", torch.int32)
    if out is None:
        out = torch.empty(M, dtype=torch.int32, device="cuda")
    _chk(out, "slot_mapping", torch.int32, M)
    check(lib.snowllm_resolve_slots(_p(block_tables), block_tables.shape[1], _p(row_seq),
                                    _p(row_pos), _p(out), M, block_size, _stream()),
          "resolve_slots")
    return out


def dense_shuffle(w, wt=None):
    """Repack a row-major fp16/bf16 weight [N, K] for dense_gemv."""
    N, K = w.shape
    wt = wt or (WT_F16 if w.dtype == torch.float16 else WT_BF16)
    out = torch.empty(lib.snowverify_dense_bytes(N, K), dtype=torch.uint8, device="cuda")
    check(lib.snowverify_dense_shuffle(_p(w), _p(out), N, K, wt, _stream()), "dense_shuffle")
    return out


def dense_gemv(wt, w_shuffled, act, out, M, N, K):
    bf16 = out.dtype is torch.bfloat16
    check(lib.snowverify_dense_gemv(wt, _p(w_shuffled), _p(act), _p(out), M, N, K, bf16,
                                    _stream()), "dense_gemv")


def gate_up_swiglu(fmt, quant, meta, ws, act, M, F, K):
    _chk(act, "activation", torch.bfloat16, M, F)
    check(lib.snowverify_gate_up_swiglu(fmt, _p(quant), _p(meta), _p(ws), _p(act), M, F, K,
                                        _stream()), "gate_up_swiglu")


def swiglu(gate_up, out):
    M, F = out.shape
    check(lib.snowverify_swiglu(_p(gate_up), gate_up.stride(0), _p(out), M, F, _stream()), "swiglu")


def moe_route(logits, E, topk, weights, ids, shared_w=None):
    M = logits.shape[0]
    _chk(weights, "routing weights", torch.float32, M, topk)
    _chk(ids, "routing ids", torch.int32, M, topk)
    check(lib.snowverify_moe_route(_p(logits), logits.stride(0), M, E, topk, _p(weights), _p(ids),
                                   _p(shared_w), _stream()), "moe_route")


MOE_PLAN_BYTES = int(lib.snowverify_moe_plan_bytes())


def moe_plan(ids, E, plan, shared=True):
    M, topk = ids.shape
    check(lib.snowverify_moe_plan(_p(ids), M, topk, E, int(shared), _p(plan), _stream()), "moe_plan")


def moe_route_plan(logits, E, topk, weights, ids, shared_w, plan):
    """moe_route + moe_plan in one launch (shared-expert slot iff shared_w is given)."""
    M = logits.shape[0]
    _chk(weights, "routing weights", torch.float32, M, topk)
    _chk(ids, "routing ids", torch.int32, M, topk)
    check(lib.snowverify_moe_route_plan(_p(logits), logits.stride(0), M, E, topk, _p(weights),
                                        _p(ids), _p(shared_w), _p(plan), _stream()),
          "moe_route_plan")


def norm_router_plan(x, gamma, ws, eps, router, logits, topk, weights, ids, shared_w, plan, *,
                     res_in=None, res_out=None, y_out=None):
    """norm_prep + the bf16 router GEMV (dense_gemv) + moe_route_plan in one launch, with their
    bits: logits [M, E (+1 with shared_w)] f32."""
    M, H = x.shape
    _chk(x, "x", torch.bfloat16, M, H)
    _chk(gamma, "gamma", torch.bfloat16, H)
    for t, n in ((res_in, "res_in"), (res_out, "res_out"), (y_out, "y_out")):
        if t is not None:
            _chk(t, n, torch.bfloat16, M, H)
    E = logits.shape[1] - (1 if shared_w is not None else 0)
    _chk(logits, "router logits", torch.float32, M, logits.shape[1])
    _chk(weights, "routing weights", torch.float32, M, topk)
    _chk(ids, "routing ids", torch.int32, M, topk)
    check(lib.snowverify_norm_router_plan(_p(x), _p(res_in), _p(res_out), _p(gamma), eps, _p(ws),
                                          _p(y_out), _p(router), _p(logits), M, H, E, topk,
                                          _p(weights), _p(ids), _p(shared_w), _p(plan),
                                          _stream()), "norm_router_plan")


def moe_experts(fmt, gu, dn, sh_gu, sh_dn, plan, ws, weights, shared_w, act, pairs, shared_out,
                out, M, topk, E, H, F):
    """gu/dn/sh_gu/sh_dn: (quant, meta) pairs of the stacked expert weights; fmt: the gate/up
    format id (4, 5, 6 for Q4_K, Q5_K, Q6_K) | the down format id << 8 (0: the gate/up's)."""
    check(lib.snowverify_moe_experts(fmt, _p(gu[0]), _p(gu[1]), _p(dn[0]), _p(dn[1]),
                                     _p(sh_gu[0]), _p(sh_gu[1]), _p(sh_dn[0]), _p(sh_dn[1]),
                                     _p(plan), _p(ws), _p(weights), _p(shared_w), _p(act),
                                     _p(pairs), _p(shared_out), _p(out), M, topk, E, H, F,
                                     _stream()), "moe_experts")


def moe_gate_up(fmt, gu, sh_gu, plan, ws, act, M, max_slots, E, H, F):
    """fmt: the gate/up format id (4, 5, 6)."""
    check(lib.snowverify_moe_gate_up(fmt, _p(gu[0]), _p(gu[1]), _p(sh_gu[0]), _p(sh_gu[1]), _p(plan),
                                     _p(ws), _p(act), M, max_slots, E, H, F, _stream()),
          "moe_gate_up")


def moe_down(fmt, dn, sh_dn, plan, act, weights, shared_w, pairs, shared_out, max_slots, E, H, F):
    """fmt: the down format id (4, 5, 6)."""
    check(lib.snowverify_moe_down(fmt, _p(dn[0]), _p(dn[1]), _p(sh_dn[0]), _p(sh_dn[1]), _p(plan),
                                  _p(act), _p(weights), _p(shared_w), _p(pairs), _p(shared_out),
                                  max_slots, E, H, F, _stream()), "moe_down")


def moe_gate_up_down(fmt, gu, dn, sh_gu, sh_dn, plan, ws, weights, shared_w, act, pairs,
                     shared_out, M, max_slots, E, H, F):
    """moe_gate_up then moe_down in one launch (same bits); launches on one device must be
    stream-ordered (library-owned counters). fmt as moe_experts'; down in the gate/up format
    or a wider one."""
    check(lib.snowverify_moe_gate_up_down(fmt, _p(gu[0]), _p(gu[1]), _p(dn[0]), _p(dn[1]),
                                          _p(sh_gu[0]), _p(sh_gu[1]), _p(sh_dn[0]),
                                          _p(sh_dn[1]), _p(plan), _p(ws), _p(weights),
                                          _p(shared_w), _p(act), _p(pairs), _p(shared_out), M,
                                          max_slots, E, H, F, _stream()), "moe_gate_up_down")


def moe_sync_error():
    """Non-zero once a fused expert launch timed out waiting for its activations."""
    return int(lib.snowverify_moe_sync_error())


def moe_combine(pairs, shared_out, out, M, topk, H):
    check(lib.snowverify_moe_combine(_p(pairs), _p(shared_out), _p(out), M, topk, H, _stream()),
          "moe_combine")


def parse_plan(plan):
    """Host view of a MoE plan buffer (tests and accounting): dict of numpy arrays."""
    import numpy as np
    a = plan.view(torch.int32).cpu().numpy()
    S = MOE_MAX_SLOTS
    n = int(a[0])
    o = 2
    slot_expert = a[o:o + S]; o += S
    slot_rows = a[o:o + S]; o += S
    row_of = a[o:o + S * 16].reshape(S, 16); o += S * 16
    pair_of = a[o:o + S * 16].reshape(S, 16)
    return {"n_slots": n, "n_routed": int(a[1]), "slot_expert": slot_expert[:n].copy(),
            "slot_rows": slot_rows[:n].copy(), "row_of": row_of[:n].copy(),
            "pair_of": pair_of[:n].copy()}


MOE_MAX_SLOTS = 292   # slots a plan struct holds (csrc/ffn.hip MoePlan)
MOE_MAX_ROWS = 64     # block rows per plan


def moe_max_slots(M, topk, E, shared=True):
    """The most slots a plan of M rows can take (one per 16 rows of an expert, the shared
    expert's ceil(M / 16)): the expert launches' max_slots and their activation scratch rows."""
    n = int(lib.snowverify_moe_max_slots(M, topk, E, int(bool(shared))))
    if n <= 0:
        raise SnowLLMError(f"a MoE plan takes at most {MOE_MAX_ROWS} rows and 512 picks "
                           f"(M={M}, topk={topk}, E={E})")
    return n
