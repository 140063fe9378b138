"""Paged GQA attention of a verify block (snowllm/ops/attention_full.py:120-177).

KV pools use the reference's page layouts (tests/test_lfm2_dspark_reference.py:30-36):
K [blocks, Hkv, d/16, page, 16], V [blocks, Hkv, page/4, d, 4], bf16, page = 16.
"""
import torch

from ._capi import SnowLLMError, check, lib
from ._common import _chk, _p, _stream

PAGE = 16


def paged_attention_scratch_bytes(batch: int, tokens: int, num_heads: int, num_kv_heads: int,
                                  head_size: int) -> int:
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
    need = paged_attention_scratch_bytes(batch, T, Hq, hkv, D)
    if scratch is None or scratch.nbytes < need:
        raise SnowLLMError(f"paged attention needs {need} scratch bytes")
    check(lib.snowverify_paged_attention(_p(q), _p(k_pool), _p(v_pool), _p(out), _p(table),
                                         _p(lens), _p(tree), batch, T, Hq, hkv, D, PAGE,
                                         table.shape[1], float(scale), _p(scratch), scratch.nbytes,
                                         _stream()), "paged_attention")
