"""GPU parity of the Q4_K / Q8_0 dequant-GEMV against the fp64 oracle (rel L2 < 1e-3)."""
import numpy as np
import pytest
import torch

from oracle import quant as Q

pytestmark = pytest.mark.gpu

TOL = 1e-3  # BASELINE: matmul outputs within 1e-3 relative (fp32 accumulate)


def _run(fmt, raw, x, n, k, out_dtype=torch.float32):
    from snowllm_amd import ops
    quant, meta = ops.gemm_kquant_shuffle_b(fmt, torch.from_numpy(raw).cuda(), n, k)
    m = x.shape[0]
    c = torch.empty(m, n, dtype=out_dtype, device="cuda")
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(m, k), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_a(fmt, x.cuda(), quant, meta, c, m, n, k, ws)
    torch.cuda.synchronize()
    return c.float().cpu().numpy(), (quant, meta, ws)


@pytest.mark.parametrize("fmt", [4, 5, 6, 8])
@pytest.mark.parametrize("m", [1, 9, 16, 17])
@pytest.mark.parametrize("n,k", [(384, 1024), (5120, 2048), (2048, 4096)])
def test_gemv_matches_oracle(gpu, fmt, m, n, k):
    print(f"gemv fmt={fmt} M={m} N={n} K={k}", flush=True)
    raw = Q.make(fmt, n, k, seed=n + k)
    x = Q.make_activations(m, k, seed=m)
    got, _ = _run(fmt, raw, x, n, k)
    want = Q.gemv_reference(x, Q.dequant(raw, fmt, n, k))
    assert Q.rel_l2(got, want) < TOL


def test_config2_q4k_gemv(gpu):
    """M=9, K=4096, N=14336, bf16 output via fp32 accumulate."""
    n, k, m = 14336, 4096, 9
    raw = Q.make_q4_k(n, k, seed=2)
    x = Q.make_activations(m, k, seed=3)
    got, _ = _run(4, raw, x, n, k, torch.bfloat16)
    want = Q.gemv_reference(x, Q.dequant_q4_k(raw, n, k))
    err = Q.rel_l2(got, want)
    print(f"config 2 rel L2 {err:.2e}", flush=True)
    # bf16 output rounding alone is ~2^-9 per element; judge the fp32 path tightly too
    assert err < 3e-3
    got32, _ = _run(4, raw, x, n, k, torch.float32)
    assert Q.rel_l2(got32, want) < TOL


def test_gemv_activation_scales(gpu):
    """Rows spanning very different magnitudes (per-row fp16 scaling must stay exact)."""
    n, k, m = 512, 1024, 9
    raw = Q.make_q4_k(n, k, seed=5)
    x = Q.make_activations(m, k, seed=6).float()
    x[0] *= 3e4
    x[1] *= 1e-4
    x[2, :7] = 0
    x[3] = 0
    x = x.bfloat16()
    got, _ = _run(4, raw, x, n, k)
    want = Q.gemv_reference(x, Q.dequant_q4_k(raw, n, k))
    for r in range(m):
        if r == 3:
            assert np.all(got[r] == 0)
        else:
            assert Q.rel_l2(got[r], want[r]) < TOL, r


def test_gemv_graph_replay(gpu):
    from snowllm_amd import ops
    n, k, m = 1024, 2048, 9
    raw = Q.make_q4_k(n, k, seed=9)
    x = Q.make_activations(m, k, seed=10).cuda()
    quant, meta = ops.gemm_kquant_shuffle_b(4, torch.from_numpy(raw).cuda(), n, k)
    c = torch.empty(m, n, device="cuda")
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(m, k), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_a(4, x, quant, meta, c, m, n, k, ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.gemm_kquant_a(4, x, quant, meta, c, m, n, k, ws)
    w = Q.dequant_q4_k(raw, n, k)
    for seed in (11, 12):
        x.copy_(Q.make_activations(m, k, seed=seed))
        c.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert Q.rel_l2(c.cpu().numpy(), Q.gemv_reference(x.cpu(), w)) < TOL


@pytest.mark.parametrize("fmt", [4, 8])
def test_every_gemv_variant(gpu, fmt):
    """Each fixed tile shape (the tuning knob) agrees with the oracle, incl. K with S > waves."""
    from snowllm_amd import ops
    from snowllm_amd._capi import lib
    for n, k in [(1024, 14336), (768, 2048)]:
        raw = Q.make_q4_k(n, k, seed=n) if fmt == 4 else Q.make_q8_0(n, k, seed=n)
        x = Q.make_activations(9, k, seed=k)
        want = Q.gemv_reference(x, Q.dequant(raw, fmt, n, k))
        quant, meta = ops.gemm_kquant_shuffle_b(fmt, torch.from_numpy(raw).cuda(), n, k)
        ws = torch.empty(ops.gemm_kquant_a_ws_bytes(9, k), dtype=torch.uint8, device="cuda")
        c = torch.empty(9, n, device="cuda")
        c2 = torch.empty(9, n, device="cuda")
        try:
            for v in range(7):
                print(f"variant {v} fmt={fmt} N={n} K={k}", flush=True)
                lib.snowverify_gemv_variant(v)
                c.zero_()
                ops.gemm_kquant_a(fmt, x.cuda(), quant, meta, c, 9, n, k, ws)
                assert Q.rel_l2(c.cpu().numpy(), want) < TOL, v
                # the one-launch path (in-kernel conversion) and the prepared workspace path
                # build the same operands: identical results
                ops.gemm_kquant_prepare_a(x.cuda(), ws)
                ops.gemm_kquant_a_prepared(fmt, quant, meta, c2, 9, n, k, ws)
                assert torch.equal(c, c2), v
        finally:
            lib.snowverify_gemv_variant(0)


@pytest.mark.parametrize("fmt", [4, 5, 6, 8])
@pytest.mark.parametrize("n,k", [(5120, 2048), (512, 4096), (256, 1024)])
def test_wide_block_gemv_equals_row_tiles(gpu, fmt, n, k):
    """Verify steps wider than 16 rows (B x T <= 256): one launch decodes each weight tile once
    for up to four row tiles; every row gets the bits of the 16-row launch, and the result
    stays within the fp64 oracle's tolerance."""
    from snowllm_amd import ops
    raw = Q.make(fmt, n, k, seed=n + 3)
    quant, meta = ops.gemm_kquant_shuffle_b(fmt, torch.from_numpy(raw).cuda(), n, k)
    w = Q.dequant(raw, fmt, n, k)
    tb = ops.gemm_kquant_a_ws_bytes(16, k)
    for m in (17, 36, 48, 64, 100, 256):
        print(f"wide gemv fmt={fmt} M={m} N={n} K={k}", flush=True)
        x = Q.make_activations(m, k, seed=m + 1)
        ws = torch.empty(ops.gemm_kquant_a_ws_bytes(m, k), dtype=torch.uint8, device="cuda")
        c = torch.empty(m, n, device="cuda")
        ops.gemm_kquant_a(fmt, x.cuda(), quant, meta, c, m, n, k, ws)
        tiles = torch.empty_like(c)
        for r0 in range(0, m, 16):
            rows = min(16, m - r0)
            at = (r0 // 16) * tb
            ops.gemm_kquant_a_prepared(fmt, quant, meta, tiles[r0:r0 + rows], rows, n, k,
                                       ws[at:at + tb])
        torch.cuda.synchronize()
        assert torch.equal(c, tiles), m
        assert Q.rel_l2(c.cpu().numpy(), Q.gemv_reference(x, w)) < TOL


@pytest.mark.parametrize("fmt", [5, 6])
def test_q5k_q6k_config2_shape_and_forms(gpu, fmt):
    """Q5_K / Q6_K (the other k-quants of Q4_K_M checkpoints, snowllm/checkpoint/gguf/
    source.py:263-272) at the config-2 shape: the one-launch form equals the prepared form bit
    for bit, both within 1e-3 of the fp64 product of the oracle's decode; the repacked bytes
    add up to the GGUF bytes; the tile shapes of the variant knob agree."""
    from snowllm_amd import ops
    n, k, m = 14336, 4096, 9
    raw = Q.make(fmt, n, k, seed=fmt)
    quant_b, meta_b, gguf_b = ops.kquant_bytes(fmt, n, k)
    assert quant_b - 4 + meta_b == gguf_b == raw.size
    x = Q.make_activations(m, k, seed=7)
    got, (quant, meta, ws) = _run(fmt, raw, x, n, k)
    want = Q.gemv_reference(x, Q.dequant(raw, fmt, n, k))
    err = Q.rel_l2(got, want)
    print(f"fmt {fmt} config-2 shape rel L2 {err:.2e}", flush=True)
    assert err < TOL
    c2 = torch.empty(m, n, device="cuda")
    ops.gemm_kquant_prepare_a(x.cuda(), ws)
    ops.gemm_kquant_a_prepared(fmt, quant, meta, c2, m, n, k, ws)
    torch.cuda.synchronize()
    assert np.array_equal(c2.cpu().numpy(), got)
    from snowllm_amd import _capi
    for v in (1, 2, 4, 5):
        _capi.lib.snowverify_gemv_variant(v)
        try:
            ops.gemm_kquant_a_prepared(fmt, quant, meta, c2, m, n, k, ws)
            torch.cuda.synchronize()
        finally:
            _capi.lib.snowverify_gemv_variant(0)
        assert Q.rel_l2(c2.cpu().numpy(), want) < TOL, v


@pytest.mark.parametrize("m", [9, 40])   # one row tile; the wide-block form (three tiles)
def test_strided_gemv_fills_columns(gpu, m):
    """snowverify_gemm_kquant_a_prepared_ld: a Q4_K q|k weight and a Q6_K v weight fill their
    column ranges of one [M, N1 + N2] output with the bits of the contiguous launches, and the
    columns around them stay untouched."""
    from snowllm_amd import ops
    k, n1, n2 = 2048, 1536, 256
    raws = (Q.make(4, n1, k, seed=31), Q.make(6, n2, k, seed=32))
    packs = [ops.gemm_kquant_shuffle_b(f, torch.from_numpy(r).cuda(), n, k)
             for f, r, n in ((4, raws[0], n1), (6, raws[1], n2))]
    x = Q.make_activations(m, k, seed=m).cuda()
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(m, k), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_prepare_a(x, ws)
    for dtype in (torch.bfloat16, torch.float32):
        print(f"strided gemv M={m} {dtype}", flush=True)
        out = torch.full((m, n1 + n2 + 16), 7.0, dtype=dtype, device="cuda")
        ops.gemm_kquant_a_prepared(4, *packs[0], out, m, n1, k, ws, col=0)
        ops.gemm_kquant_a_prepared(6, *packs[1], out, m, n2, k, ws, col=n1 + 16)
        a = torch.empty(m, n1, dtype=dtype, device="cuda")
        b = torch.empty(m, n2, dtype=dtype, device="cuda")
        ops.gemm_kquant_a_prepared(4, *packs[0], a, m, n1, k, ws)
        ops.gemm_kquant_a_prepared(6, *packs[1], b, m, n2, k, ws)
        torch.cuda.synchronize()
        assert torch.equal(out[:, :n1], a) and torch.equal(out[:, n1 + 16:], b)
        assert bool((out[:, n1:n1 + 16] == 7.0).all())
