"""GPU parity of paged GQA attention against fp32 dense attention (rel L2 < 2e-3, bf16)."""
import math

import pytest
import torch

from oracle import reference as R
from tests.kvcache import pools_from_dense, to_i64, tree_masks

pytestmark = pytest.mark.gpu

TOL = 2e-3  # BASELINE: attention outputs within 2e-3 for bf16


def _mask(ctx, T, masks):
    L = ctx + T
    m = torch.zeros(T, L, dtype=torch.bool)
    m[:, :ctx] = True
    for t in range(T):
        for j in range(T):
            if (masks[t] >> j) & 1:
                m[t, ctx + j] = True
    return m


def _case(lengths, T, Hq, Hkv, D, seed, tree_parents=None, extra_blocks=7):
    from snowllm_amd import ops
    g = torch.Generator().manual_seed(seed)
    batch = len(lengths)
    pages = [(L + 15) // 16 for L in lengths]
    total_blocks = sum(pages) + extra_blocks
    perm = torch.randperm(total_blocks, generator=g).int()
    width = max(pages)
    table = torch.zeros(batch, width, dtype=torch.int32)
    kps, vps, qs, ks, vs = [], [], [], [], []
    off = 0
    kp = torch.zeros(total_blocks, Hkv, D // 16, 16, 16, dtype=torch.bfloat16)
    vp = torch.zeros(total_blocks, Hkv, 4, D, 4, dtype=torch.bfloat16)
    for b, L in enumerate(lengths):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
        k = torch.randn(L, Hkv, D, generator=g).bfloat16()
        v = torch.randn(L, Hkv, D, generator=g).bfloat16()
        kb, vb = pools_from_dense(k, v, table[b], total_blocks)
        used = table[b, :pages[b]].long()
        kp[used] = kb[used]
        vp[used] = vb[used]
        ks.append(k)
        vs.append(v)
        qs.append(torch.randn(T, Hq, D, generator=g).bfloat16())
    q = torch.cat(qs)
    masks = tree_masks(tree_parents) if tree_parents else [(2 << t) - 1 for t in range(T)]
    tree = torch.tensor(to_i64(masks) * batch, dtype=torch.int64) if tree_parents else None
    scale = D ** -0.5
    out = torch.empty_like(q).cuda()
    lens = torch.tensor(lengths, dtype=torch.int32)
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(batch, T, Hq, Hkv, D), dtype=torch.uint8, device="cuda")
    print(f"attention lengths={lengths} T={T} Hq={Hq} Hkv={Hkv} D={D} tree={bool(tree_parents)}", flush=True)
    ops.paged_attention_explicit(q.cuda(), kp.cuda(), vp.cuda(), out, table.cuda(), lens.cuda(), scale,
                                 scratch, tree=None if tree is None else tree.cuda())
    torch.cuda.synchronize()
    got = out.cpu().float()
    for b, L in enumerate(lengths):
        want = R.dense_attention(qs[b], ks[b], vs[b], scale, _mask(L - T, T, masks))
        err = ((got[b * T:(b + 1) * T] - want).norm() / want.norm()).item()
        print(f"  request {b}: rel L2 {err:.2e}", flush=True)
        assert err < TOL, (b, err)


def test_config3_shape():
    _case([8192 + 9], 9, 32, 8, 128, seed=4)


def test_config4_shape():
    _case([8192 + 9], 9, 16, 2, 256, seed=5)


def test_config5_tree_long_context():
    parents = [-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9]  # k = 5, two branches of the root
    _case([220000 + 11], 11, 16, 2, 256, seed=6, tree_parents=parents)


@pytest.mark.parametrize("lengths,T", [([1000, 37], 4), ([9], 9), ([17, 16 * 7 + 3, 5], 5)])
def test_ragged_batches(lengths, T):
    _case(lengths, T, 8, 2, 128, seed=sum(lengths))


def test_single_kv_head_d256_tree_batch():
    _case([300, 1201], 3, 4, 1, 256, seed=9, tree_parents=[-1, 0, 0])
