"""The no-allocation k-quant GEMV (snowverify_gemm_kquant_a_noalloc, called through the C ABI)
against snowllm_gemm_kquant_a with a caller workspace: same bits, on calls in a row, each
smaller than the one before (the shared device array still holds the previous call's
operands), above and below the 16-row one-launch form; sizes beyond the array are refused.
Collected last (the file name) and independent of the tests before it."""
import ctypes

import pytest
import torch

from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _noalloc(lib):
    f = lib.snowverify_gemm_kquant_a_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_int,
                                                                                ctypes.c_void_p]
    return f


def _case(fmt, M, N, K, seed):
    from snowllm_amd import ops
    from snowllm_amd._capi import lib
    raw = Q.make_q4_k(N, K, seed=seed) if fmt == 4 else Q.make_q8_0(N, K, seed=seed)
    quant, meta = ops.gemm_kquant_shuffle_b(fmt, torch.from_numpy(raw).cuda(), N, K)
    x = Q.make_activations(M, K, seed=seed + 1).cuda()
    want = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(ops.gemm_kquant_a_ws_bytes(M, K), dtype=torch.uint8, device="cuda")
    ops.gemm_kquant_a(fmt, x, quant, meta, want, M, N, K, ws)
    got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc = _noalloc(lib)(fmt, x.data_ptr(), quant.data_ptr(), meta.data_ptr(), got.data_ptr(),
                       M, N, K, 1, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("fmt", [4, 8])
def test_noalloc_gemv_equals_workspace_gemv(gpu, fmt):
    for M, N, K in ((64, 4096, 16384), (48, 2048, 8192), (20, 1024, 4096), (9, 4096, 4096)):
        print(f"noalloc gemv fmt={fmt} M={M} N={N} K={K}", flush=True)
        got, want = _case(fmt, M, N, K, seed=M + K)
        assert torch.equal(got, want), (M, N, K)


def test_noalloc_gemv_refuses_sizes_beyond_its_array(gpu):
    from snowllm_amd._capi import lib
    f = _noalloc(lib)
    s = torch.cuda.current_stream().cuda_stream
    # the size checks come before any pointer is read
    assert f(4, None, None, None, None, 65, 1024, 4096, 1, s) != 0
    assert f(4, None, None, None, None, 32, 1024, 16384 + 256, 1, s) != 0
    from snowllm_amd import ops
    from snowllm_amd.errors import SnowLLMError
    x = torch.zeros(65, 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(SnowLLMError, match="exceed its workspace"):
        ops.gemm_kquant_a_noalloc(4, x, x, x, torch.empty(65, 16, device="cuda"), 65, 16, 256)
