# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/attention_full.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Paged GQA attention of a verify block (snowllm/ops/attention_full.py:120-177).

KV pools use the reference's page layouts (tests/test_lfm2_dspark_reference.py:30-36):
K [blocks, Hkv, d/16, page, 16], V [blocks, Hkv, page/4, d, 4], bf16, page = 16.
"""
import ctypes

import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _chk_rows, _p, _stream
from .geometry import build_geometry

PAGE = 16


def paged_attention_explicit_scratch_bytes(batch: int, tokens: int, num_heads: int,
                                           num_kv_heads: int, head_size: int) -> int:
    return int(lib.snowverify_paged_attention_scratch_bytes(batch, tokens, num_heads,
                                                            num_kv_heads, head_size))


def kv_pool_bytes(num_blocks: int, num_kv_heads: int, head_size: int, block_size: int = PAGE):
    """Bytes of one K and one V pool (snowllm/ops/attention_full.py:521-528), bf16."""
    n = num_blocks * num_kv_heads * head_size * block_size * 2
    return n, n


def paged_attention_explicit(q, k_pool, v_pool, out, table, lens, scale, scratch, *, tree=None):
    """out[b*T + t, h] = softmax(q k^T * scale) v over the keys row t may see.

    q, out: bf16 [batch*T, Hq, d]; table: int32 [batch, pages]; lens: int32 [batch] = context
    + T; tree: optional uint64-valued int64 [batch*T] ancestor masks (bit j: block row j is
    visible), causal when None. The block's own K/V must already be in the pools.
    """
    batch = lens.numel()
    M, Hq, D = q.shape
    if M % batch:
        raise SnowLLMError("attention rows are not a whole number of requests")
    T = M // batch
    _chk(q, "attention Q", torch.bfloat16, M, Hq, D)
    _chk(out, "attention output", torch.bfloat16, M, Hq, D)
    _chk(table, "attention block table", torch.int32, batch, table.shape[1])
    _chk(lens, "attention sequence lengths", torch.int32, batch)
    _chk(k_pool, "K pool", torch.bfloat16)
    _chk(v_pool, "V pool", torch.bfloat16)
    hkv = k_pool.shape[1] if k_pool.dim() == 5 else None
    if hkv is None:
        raise SnowLLMError("K pool must be viewed as [blocks, Hkv, d/16, page, 16]")
    if tree is not None:
        _chk(tree, "tree masks", torch.int64, M)
    need = paged_attention_explicit_scratch_bytes(batch, T, Hq, hkv, D)
    if scratch is None or scratch.nbytes < need:
        raise SnowLLMError(f"paged attention needs {need} scratch bytes")
    check(lib.snowverify_paged_attention(_p(q), _p(k_pool), _p(v_pool), _p(out), _p(table),
                                         _p(lens), _p(tree), batch, T, Hq, hkv, D, PAGE,
                                         table.shape[1], float(scale), _p(scratch), scratch.nbytes,
                                         _stream()), "paged_attention")


# Widest rotation (pairs per head) the fused QK-norm attention takes; wider ones run the
# standalone writer first (the kernel refuses them with hipErrorNotSupported).
FUSED_QK_MAX_HALF = 64


def paged_attention_qk(proj, q_gamma, k_gamma, cos, sin, eps, slots, k_pool, v_pool, out, table,
                       lens, scale, scratch, *, num_heads, num_kv_heads, tree=None, q_out=None,
                       ws_out=None):
    """QK-norm + RoPE + the block's K/V write fused into the attention (extension): proj
    [batch*T, n] bf16 = [q heads | k heads | v heads] (head size d); cos/sin [batch*T, half]
    f32; slots int32 [batch*T]. Same bits as qk_norm_rope_cache followed by
    paged_attention_explicit; q_out receives the rotated q if given. half <= FUSED_QK_MAX_HALF.
    ws_out (head size 256): the output projection's operand workspace for `out` as
    [batch*T, num_heads*d], written as gemm_kquant_prepare_a would."""
    batch = lens.numel()
    M, n = proj.shape
    D = out.shape[2]
    T = M // batch
    _chk(proj, "projection", torch.bfloat16, M, n)
    _chk(out, "attention output", torch.bfloat16, M, num_heads, D)
    _chk(cos, "cos", torch.float32, M, cos.shape[1])
    _chk(sin, "sin", torch.float32, M, cos.shape[1])
    _chk(slots, "slot mapping", torch.int32, M)
    _chk(table, "attention block table", torch.int32, batch, table.shape[1])
    _chk(lens, "attention sequence lengths", torch.int32, batch)
    if q_out is not None:
        _chk(q_out, "q", torch.bfloat16, M, num_heads, D)
    if tree is not None:
        _chk(tree, "tree masks", torch.int64, M)
    need = paged_attention_explicit_scratch_bytes(batch, T, num_heads, num_kv_heads, D)
    if scratch is None or scratch.nbytes < need:
        raise SnowLLMError(f"paged attention needs {need} scratch bytes")
    args = (_p(proj), n, D, num_heads * D, (num_heads + num_kv_heads) * D, _p(q_gamma),
            _p(k_gamma), _p(cos), _p(sin), cos.shape[1], cos.shape[1], eps, _p(slots), _p(q_out),
            _p(k_pool), _p(v_pool), _p(out), _p(table), _p(lens), _p(tree), batch, T, num_heads,
            num_kv_heads, D, PAGE, table.shape[1], float(scale), _p(scratch), scratch.nbytes)
    if ws_out is None:
        check(lib.snowverify_paged_attention_qk(*args, _stream()), "paged_attention_qk")
        return
    from .gemm import gemm_kquant_a_ws_bytes
    wneed = gemm_kquant_a_ws_bytes(M, num_heads * D)
    if ws_out.nbytes < wneed or not ws_out.is_contiguous():
        raise SnowLLMError(f"paged_attention_qk: the projection workspace needs {wneed} bytes")
    check(lib.snowverify_paged_attention_qk_ws(*args, _p(ws_out), _stream()),
          "paged_attention_qk_ws")


# ---------------------------------------------------------------------------------------
# Geometry-driven forms with the reference's signatures (snowllm/ops/attention_full.py)
# ---------------------------------------------------------------------------------------
class _PagedAttentionStep(ctypes.Structure):  # snowllm/ops/attention_full.py:120-123
    _fields_ = [("inputs", ctypes.c_void_p * 10), ("outputs", ctypes.c_void_p * 3)] + [
        (n, ctypes.c_int64) for n in ("batch", "pages", "q_blocks", "slots", "tokens",
                                      "page_size", "gate_stride", "gate_row0")] + [
        ("scale", ctypes.c_float), ("varlen", ctypes.c_int)]


def paged_attention_scratch_bytes(batch: int, tokens: int, varlen: bool) -> int:
    return int(lib.snowllm_paged_attention_scratch_bytes(batch, tokens, int(varlen)))


def paged_attention_varlen(prefill: bool, tokens: int, chunk_decode: bool) -> bool:
    return bool(lib.snowllm_paged_attention_varlen(int(prefill), tokens, int(chunk_decode)))


def paged_attention(q, pools, out, cu, table, lens, qmap, total_blocks, plan, workspace, slots,
                    tokens, block_size, scale, varlen, scratch, gate=(0, 0, 0), *,
                    host_seq_lens=None, prepared=False):
    """snowllm/ops/attention_full.py:152-177: the step descriptor form (decode/verify)."""
    batch = lens.numel()
    _chk(q, "attention Q", torch.bfloat16)
    _chk(out, "attention output", torch.bfloat16)
    _chk(table, "attention block table", torch.int32)
    _chk(lens, "attention sequence lengths", torch.int32, batch)
    need = paged_attention_scratch_bytes(batch, tokens, varlen)
    if need and (scratch is None or scratch.nbytes < need):
        raise SnowLLMError(f"paged attention needs {need} scratch bytes")
    ks, vs = pools[2:] if len(pools) == 4 else (None, None)
    mode = int(varlen) | (4 if prepared else 0)
    if varlen and batch == 1 and host_seq_lens is not None and host_seq_lens[0] == tokens:
        mode |= 2
    step = _PagedAttentionStep(
        (ctypes.c_void_p * 10)(*[_p(t) for t in (q, pools[0], pools[1], ks, vs, cu, table, lens,
                                                 qmap)], gate[0]),
        (ctypes.c_void_p * 3)(_p(out), _p(plan), _p(workspace)), batch, table.shape[1],
        total_blocks, slots, tokens, block_size, gate[1], gate[2], scale, mode)
    check(lib.snowllm_paged_attention(ctypes.byref(step), _p(scratch),
                                      scratch.nbytes if scratch is not None else 0, _stream()),
          "paged_attention")


def paged_attention_prepare(lens, tokens, slots, block_size, varlen, arena=None):
    """attention_full.py:136-150: this build needs no prepared metadata (size 0) -> None."""
    batch = lens.numel()
    if not lib.snowllm_paged_attention_prepared_bytes(batch, tokens, slots, int(varlen)):
        return None
    raise SnowLLMError("prepared attention metadata is not expected from this library")


def paged_attention_uses_prepared(batch, tokens, varlen):
    """attention_full.py:131-133."""
    return bool(paged_attention_scratch_bytes(batch, tokens, varlen))


PAGED_DECODE_MAX_Q_TOKENS = int(lib.snowllm_paged_decode_max_q_tokens())
KV_BLOCK_SIZES = (PAGE,)


def paged_decode_num_slots(num_seqs: int) -> int:
    return int(lib.snowllm_paged_decode_num_slots(num_seqs))


def paged_decode_workspace_size(num_slots: int, q_tokens: int = 1) -> int:
    return int(lib.snowllm_paged_decode_workspace_size(num_slots, q_tokens))


def paged_decode_plan_elems(num_seqs: int, num_slots: int) -> int:
    return int(lib.snowllm_paged_decode_plan_elems(num_seqs, num_slots))


def paged_attn_decode_plan(seq_lens, plan, num_slots, block_size, uniform=False) -> None:
    """attention_full.py:1232-1238 (nothing to plan here; the arguments are checked)."""
    _chk(seq_lens, "seq_lens", torch.int32)
    _chk(plan, "plan", torch.int32)
    check(lib.snowllm_paged_attn_decode_plan(_p(seq_lens), _p(plan), seq_lens.numel(), num_slots,
                                             block_size, int(uniform), _stream()),
          "paged_attn_decode_plan")


def paged_attn_decode(q, seq_lens, k_cache, v_cache, out, block_tables, plan, workspace,
                      num_seqs, num_slots, scale, block_size, q_tokens=1, q_pitch=0, q_row0=0):
    """attention_full.py:1147-1161: split-KV decode attention of q_tokens rows per sequence,
    causal within them; q rows q_pitch elements apart (0: contiguous) from row q_row0."""
    _chk(block_tables, "block_tables", torch.int32)
    _chk(plan, "plan", torch.int32)
    _chk(seq_lens, "seq_lens", torch.int32)
    check(lib.snowllm_paged_attn_decode(_p(q), _p(seq_lens), _p(k_cache), _p(v_cache), _p(out),
                                        _p(block_tables), _p(plan), num_seqs,
                                        block_tables.shape[1], num_slots, _p(workspace), scale,
                                        q_tokens, block_size, q_pitch, q_row0, _stream()),
          "paged_attn_decode")


def prefill_q_plan(query_lens):
    """attention_full.py:539-547: (query blocks, device map of (sequence, first row) pairs)."""
    B = len(query_lens)
    lens = (ctypes.c_int32 * B)(*query_lens)
    total = lib.snowllm_prefill_q_blocks(lens, B)
    buf = (ctypes.c_int32 * (total * 2))()
    lib.snowllm_prefill_q_block_map(lens, B, buf)
    return total, torch.frombuffer(memoryview(buf), dtype=torch.int32).clone().cuda()


def attn_output_plan(m: int, prefill: bool, kv_int8: bool) -> tuple:
    """(elements of the attention output, scratch bytes) (attention_full.py:54-64)."""
    out = (ctypes.c_int64 * 2)()
    check(lib.snowllm_attn_output_plan(m, int(prefill), int(kv_int8), out), "attn_output_plan")
    return out[0], out[1]


def attn_output_shape(m: int, prefill: bool, kv_int8: bool) -> tuple:
    g = build_geometry()
    elements, _ = attn_output_plan(m, prefill, kv_int8)
    return elements // (g.num_heads * g.head_size), g.num_heads, g.head_size


def attn_output_gating(proj, prefill: bool, kv_int8: bool, row0: int = 0) -> tuple:
    return (lib.snowllm_attn_output_gate(_p(proj), int(prefill), int(kv_int8)) or 0,
            proj.shape[1], row0)


def attn_output_project(a, proj, w, scale, scratch, out, prefill: bool, kv_int8: bool) -> None:
    """out [m, hidden] = attention output . Wo^T (attention_full.py:98-117); w: a
    KQuantProjWeight (quant, meta, fmt)."""
    m = out.shape[0]
    g = build_geometry()
    _chk(a, "attention output", torch.bfloat16)
    _chk(proj, "projection", torch.bfloat16, m, proj.shape[1])
    _chk(out, "attention projection output", torch.bfloat16, m, g.hidden)
    elements, need = attn_output_plan(m, prefill, kv_int8)
    if a.numel() < elements:
        raise SnowLLMError(f"attention output needs {elements} elements")
    if need and (scratch is None or scratch.nbytes < need):
        raise SnowLLMError(f"attention output needs {need} scratch bytes")
    dense, q, meta, fmt = (None, w.quant, w.meta, w.fmt) if hasattr(w, "quant") else (w, None, None, 8)
    check(lib.snowllm_attn_output_project(_p(a), _p(proj), proj.shape[1], _p(dense), _p(q),
                                          _p(meta), _p(scale), fmt, _p(scratch), _p(out), m,
                                          int(prefill), int(kv_int8), _stream()),
          "attn_output_project")


def rope_cos_sin(position_ids, inv_freq, cos, sin) -> None:
    """cos/sin [M, 64] for the reference's rotary dimension (snowllm/ops/rope.py:11-24)."""
    M = cos.shape[0]
    _chk(position_ids, "position_ids", torch.int64)
    _chk(inv_freq, "inv_freq", torch.float32, 32)
    _chk(cos, "cos", torch.float32, M, 64)
    _chk(sin, "sin", torch.float32, M, 64)
    check(lib.snowllm_rope_cos_sin(_p(position_ids), _p(inv_freq), _p(cos), _p(sin), M,
                                   _stream()), "rope_cos_sin")


def qk_norm_rope_cache(proj, q_gamma, k_gamma, cos, sin, q, v, k_cache, v_cache, slots, eps,
                       block_size, *, k_proj=None, k_scale=None, v_scale=None):
    """Normalize/rotate QK and publish K/V to the pools (attention_full.py:736-784)."""
    g = build_geometry()
    m, n = proj.shape
    d, nk, nh = g.head_size, g.num_kv_heads, g.num_heads
    _chk(proj, "projection", torch.bfloat16, m, n)
    _chk(q_gamma, "q gamma", torch.bfloat16, d)
    _chk(k_gamma, "k gamma", torch.bfloat16, d)
    _chk(q, "q", torch.bfloat16, m, nh, d)
    _chk(cos, "cos", torch.float32, m, 64)
    _chk(sin, "sin", torch.float32, m, 64)
    _chk(slots, "slot mapping", torch.int32, m)
    _chk_rows(v, "v projection", torch.bfloat16)
    if v.shape != (m, nk * d) or n < (nh - 1) * g.qkv_q_head_stride + d:
        raise SnowLLMError("QK/cache projection shape mismatch")
    if k_proj is None:
        if n < g.qkv_off_k + nk * d:
            raise SnowLLMError("projection does not contain K")
        kp, ks = _p(proj) + g.qkv_off_k * 2, n
    else:
        _chk_rows(k_proj, "k projection", torch.bfloat16)
        kp, ks = _p(k_proj), k_proj.stride(0)
    if (k_scale is None) != (v_scale is None):
        raise SnowLLMError("KV scales must be paired")
    _chk(k_cache, "k cache", torch.bfloat16)
    _chk(v_cache, "v cache", torch.bfloat16)
    if block_size != g.block_size or k_cache.numel() % (block_size * nk * d):
        raise SnowLLMError("KV pool size or block size mismatch")
    check(lib.snowllm_qk_norm_rope_cache(_p(proj), n, kp, ks, _p(v), v.stride(0), _p(q_gamma),
                                         _p(k_gamma), _p(cos), _p(sin), _p(q), _p(k_cache),
                                         _p(v_cache), _p(k_scale), _p(v_scale), _p(slots), m,
                                         eps, block_size, _stream()), "qk_norm_rope_cache")
