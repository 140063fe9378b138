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


def _case(lengths, T, Hq, Hkv, D, seed, tree_parents=None, extra_blocks=7, v_scale=1.0):
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
        v = (torch.randn(L, Hkv, D, generator=g) * v_scale).bfloat16()
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


@pytest.mark.parametrize("v_scale", [3e6, 1e-12])
def test_value_magnitudes_outside_fp16(v_scale):
    """Values far outside fp16's range: the f32 split partials and the bf16 P.V products
    (P as a bf16 hi + lo pair) merge without overflow or flush."""
    _case([2000 + 9], 9, 16, 2, 256, seed=7, v_scale=v_scale)


def test_config5_tree_long_context():
    parents = [-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9]  # k = 5, two branches of the root
    _case([220000 + 11], 11, 16, 2, 256, seed=6, tree_parents=parents)


@pytest.mark.parametrize("lengths,T", [([1000, 37], 4), ([9], 9), ([17, 16 * 7 + 3, 5], 5)])
def test_ragged_batches(lengths, T):
    _case(lengths, T, 8, 2, 128, seed=sum(lengths))


def test_single_kv_head_d256_tree_batch():
    _case([300, 1201], 3, 4, 1, 256, seed=9, tree_parents=[-1, 0, 0])


@pytest.mark.parametrize("lengths,T,Hq,Hkv,D,half,pps,tree", [
    ([8192 + 9], 9, 16, 2, 256, 32, 0, False),      # config 4 shape
    ([8190 + 9, 301 + 9], 9, 32, 8, 128, 64, 0, False),  # block rows over two pages
    ([100 + 11], 11, 16, 2, 256, 32, 5, True),     # tree; splits of 5 pages
    ([77 + 9], 9, 4, 2, 128, 32, 1, False),        # one page per split: rows over two splits
    ([500 + 9], 9, 8, 2, 256, 64, 0, False),       # widest rotation the fused form takes
])
def test_fused_qk_attention_equals_separate_kernels(lengths, T, Hq, Hkv, D, half, pps, tree):
    """QK-norm + RoPE + the block's K/V write inside the attention gives the same q, pools and
    output bits as qk_norm_rope_cache followed by paged_attention_explicit."""
    from snowllm_amd import layers as L, ops
    from snowllm_amd._capi import lib
    print(f"fused qk attention lengths={lengths} T={T} D={D} pps={pps} tree={tree}", flush=True)
    g = torch.Generator().manual_seed(len(lengths) * 100 + D + pps)
    batch = len(lengths)
    pages = [(n + 15) // 16 for n in lengths]
    total = sum(pages) + 5
    perm = torch.randperm(total, generator=g).int()
    width = max(pages)
    table = torch.zeros(batch, width, dtype=torch.int32)
    off = 0
    for b in range(batch):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    kp0 = torch.randn(total, Hkv, D // 16, 16, 16, generator=g).bfloat16()
    vp0 = torch.randn(total, Hkv, 4, D, 4, generator=g).bfloat16()
    n = (Hq + 2 * Hkv) * D
    proj = torch.randn(batch * T, n, generator=g).bfloat16()
    qg = (torch.rand(D, generator=g) + .5).bfloat16()
    kg = (torch.rand(D, generator=g) + .5).bfloat16()
    pos = torch.cat([torch.arange(n - T, n) for n in lengths])
    inv = 1.0 / (1e4 ** (torch.arange(half).float() / half))
    ang = pos[:, None].float() * inv[None]
    cos, sin = ang.cos(), ang.sin()
    slots = torch.cat([(table[b, (torch.arange(n - T, n) // 16)] * 16 + torch.arange(n - T, n) % 16)
                       for b, n in enumerate(lengths)]).int()
    masks = tree_masks([-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9]) if tree else None
    tr = torch.tensor(to_i64(masks) * batch, dtype=torch.int64).cuda() if tree else None
    lens = torch.tensor(lengths, dtype=torch.int32).cuda()
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(batch, T, Hq, Hkv, D),
                          dtype=torch.uint8, device="cuda")
    dev = lambda x: x.cuda()
    prev = lib.snowverify_attention_pages_per_split(pps)
    try:
        res = []
        for fused in (False, True):
            kp, vp = kp0.clone().cuda(), vp0.clone().cuda()
            q = torch.zeros(batch * T, Hq, D, dtype=torch.bfloat16, device="cuda")
            out = torch.empty_like(q)
            if fused:
                ops.paged_attention_qk(dev(proj), dev(qg), dev(kg), dev(cos), dev(sin), 1e-6,
                                       dev(slots), kp, vp, out, dev(table), lens, D ** -0.5,
                                       scratch, num_heads=Hq, num_kv_heads=Hkv, tree=tr, q_out=q)
            else:
                L.qk_norm_rope_cache(dev(proj), dev(qg), dev(kg), dev(cos), dev(sin), q, kp, vp,
                                     dev(slots), 1e-6)
                ops.paged_attention_explicit(q, kp, vp, out, dev(table), lens, D ** -0.5,
                                             scratch, tree=tr)
            torch.cuda.synchronize()
            res.append((q, kp, vp, out))
        for a, b in zip(*res):
            assert torch.equal(a, b)
    finally:
        lib.snowverify_attention_pages_per_split(prev)


def test_fused_qk_attention_refuses_wide_rotation():
    """Rotations wider than FUSED_QK_MAX_HALF pairs are refused before any launch."""
    from snowllm_amd import ops
    from snowllm_amd._capi import SnowLLMError
    T, Hq, Hkv, D, half = 9, 8, 2, 256, 96
    assert half > ops.FUSED_QK_MAX_HALF
    c = lambda *s, dt=torch.bfloat16: torch.zeros(*s, dtype=dt, device="cuda")
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(1, T, Hq, Hkv, D),
                          dtype=torch.uint8, device="cuda")
    with pytest.raises(SnowLLMError):
        ops.paged_attention_qk(c(T, (Hq + 2 * Hkv) * D), c(D), c(D), c(T, half, dt=torch.float32),
                               c(T, half, dt=torch.float32), 1e-6, c(T, dt=torch.int32),
                               c(2, Hkv, D // 16, 16, 16), c(2, Hkv, 4, D, 4), c(T, Hq, D),
                               c(1, 2, dt=torch.int32),
                               torch.tensor([T + 7], dtype=torch.int32, device="cuda"), D ** -0.5,
                               scratch, num_heads=Hq, num_kv_heads=Hkv)


@pytest.mark.parametrize("lengths,T,Hq,Hkv,tree", [
    ([8192 + 9], 9, 16, 2, False),        # config 4 shape
    ([300 + 3, 1201 + 3], 3, 8, 2, True),  # two requests: workspace rows b * T + t
])
def test_merge_writes_projection_operands(lengths, T, Hq, Hkv, tree):
    """With 256-wide heads the merge can also write the O projection's operand workspace: the
    attention output and the projection (prepared operands) give the bits of the plain merge
    followed by the projection converting the bf16 output itself."""
    from snowllm_amd import ops
    from snowllm_amd.verify import packed_random
    D, half, N = 256, 32, 512
    print(f"merge -> projection operands lengths={lengths} T={T} Hq={Hq} tree={tree}", flush=True)
    g = torch.Generator().manual_seed(sum(lengths) + T)
    batch = len(lengths)
    pages = [(n + 15) // 16 for n in lengths]
    total = sum(pages) + 3
    perm = torch.randperm(total, generator=g).int()
    table = torch.zeros(batch, max(pages), dtype=torch.int32)
    off = 0
    for b in range(batch):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    kp0 = torch.randn(total, Hkv, D // 16, 16, 16, generator=g).bfloat16()
    vp0 = torch.randn(total, Hkv, 4, D, 4, generator=g).bfloat16()
    proj = torch.randn(batch * T, (Hq + 2 * Hkv) * D, generator=g).bfloat16()
    qg = (torch.rand(D, generator=g) + .5).bfloat16()
    kg = (torch.rand(D, generator=g) + .5).bfloat16()
    pos = torch.cat([torch.arange(n - T, n) for n in lengths])
    ang = pos[:, None].float() * (1.0 / (1e4 ** (torch.arange(half).float() / half)))[None]
    slots = torch.cat([(table[b, (torch.arange(n - T, n) // 16)] * 16 + torch.arange(n - T, n) % 16)
                       for b, n in enumerate(lengths)]).int()
    tr = None
    if tree:
        tr = torch.tensor(to_i64(tree_masks([-1, 0, 0][:T])) * batch, dtype=torch.int64).cuda()
    w = packed_random(4, N, Hq * D, 77)
    M, K = batch * T, Hq * D
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(batch, T, Hq, Hkv, D),
                          dtype=torch.uint8, device="cuda")
    res = []
    for fused_ws in (False, True, True):
        kp, vp = kp0.clone().cuda(), vp0.clone().cuda()
        out = torch.empty(M, Hq, D, dtype=torch.bfloat16, device="cuda")
        ws = torch.full((ops.gemm_kquant_a_ws_bytes(M, K),), 0x7f, dtype=torch.uint8, device="cuda")
        c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ops.paged_attention_qk(proj.cuda(), qg.cuda(), kg.cuda(), ang.cos().cuda(), ang.sin().cuda(),
                               1e-6, slots.cuda(), kp, vp, out, table.cuda(),
                               torch.tensor(lengths, dtype=torch.int32).cuda(), D ** -0.5, scratch,
                               num_heads=Hq, num_kv_heads=Hkv, tree=tr,
                               ws_out=ws if fused_ws else None)
        if fused_ws:
            ops.gemm_kquant_a_prepared(4, w[0], w[1], c, M, N, K, ws)
        else:
            ops.gemm_kquant_a(4, out.view(M, K), w[0], w[1], c, M, N, K, ws)
        torch.cuda.synchronize()
        res.append((out, c, kp, vp))
    for got in res[1:]:
        for a_, b_ in zip(res[0], got):
            assert torch.equal(a_, b_)


@pytest.mark.parametrize("lengths,T,Hq,Hkv,D,tree", [
    ([8192 + 9], 9, 16, 2, 256, False),          # config 4: five tiles (two single, three pairs)
    ([3000 + 11], 11, 16, 2, 256, True),          # config 5 rows: six tiles
    ([700 + 7, 333 + 7], 7, 16, 1, 128, False),   # seven tiles of 128-wide heads
])
def test_mixed_tile_waves_equal_one_wave_per_tile(lengths, T, Hq, Hkv, D, tree):
    """Eight waves with one or two waves per row tile (the pairs split the S products), and one
    wave per tile in two row groups (two workgroups per split, each with half of the tiles),
    give the bits of one wave per tile in one workgroup, at the same split length."""
    from snowllm_amd import ops
    from snowllm_amd._capi import lib
    print(f"mixed tile waves lengths={lengths} T={T} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    g = torch.Generator().manual_seed(sum(lengths) + D)
    batch = len(lengths)
    pages = [(n + 15) // 16 for n in lengths]
    total = sum(pages) + 3
    perm = torch.randperm(total, generator=g).int()
    table = torch.zeros(batch, max(pages), dtype=torch.int32)
    off = 0
    for b in range(batch):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    kp = torch.randn(total, Hkv, D // 16, 16, 16, generator=g).bfloat16().cuda()
    vp = torch.randn(total, Hkv, 4, D, 4, generator=g).bfloat16().cuda()
    q = torch.randn(batch * T, Hq, D, generator=g).bfloat16().cuda()
    tr = None
    if tree:
        parents = [-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9][:T]
        tr = torch.tensor(to_i64(tree_masks(parents)) * batch, dtype=torch.int64).cuda()
    lens = torch.tensor(lengths, dtype=torch.int32).cuda()
    scratch = torch.empty(ops.paged_attention_explicit_scratch_bytes(batch, T, Hq, Hkv, D),
                          dtype=torch.uint8, device="cuda")
    outs = []
    prev = lib.snowverify_attention_d_split(1)
    prev_rg = lib.snowverify_attention_row_groups(1)
    prev_pps = lib.snowverify_attention_pages_per_split(10)
    try:
        for dh, rg in ((1, 1), (1, 2), (3, 0)):
            lib.snowverify_attention_d_split(dh)
            lib.snowverify_attention_row_groups(rg)
            out = torch.empty_like(q)
            ops.paged_attention_explicit(q, kp, vp, out, table.cuda(), lens, D ** -0.5, scratch,
                                         tree=tr)
            torch.cuda.synchronize()
            outs.append(out)
    finally:
        lib.snowverify_attention_d_split(prev)
        lib.snowverify_attention_row_groups(prev_rg)
        lib.snowverify_attention_pages_per_split(prev_pps)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(outs[0], outs[2])
