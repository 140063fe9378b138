"""The C-ABI library loads without a GPU, exports every symbol the header declares, and its
size queries follow the reference's invariants. No kernel is launched."""
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "snowverify.h").read_text()
    return sorted(set(re.findall(r"\b((?:snowllm|snowverify)_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from snowllm_amd import _capi
    names = declared_symbols()
    assert names, "header declares no entry points"
    missing = [n for n in names if not hasattr(_capi.lib, n)]
    assert not missing, missing
    # and the binding table covers the header exactly
    assert sorted(_capi.SYMBOLS) == names


def test_single_hip_runtime():
    from snowllm_amd import _capi
    _capi.assert_single_hip_runtime()
    assert _capi.lib.snowllm_abi_version() == _capi.ABI_VERSION


def test_kquant_size_invariants():
    from snowllm_amd import ops
    for fmt, (n, k) in [(4, (14336, 4096)), (4, (384, 1024)), (8, (384, 1024)), (8, (2048, 4096))]:
        quant, meta, gguf = ops.kquant_bytes(fmt, n, k)
        # tests/test_mixed_gguf.py:60-61: packed bytes preserve the GGUF size
        assert quant - 4 + meta == gguf
    assert ops.kquant_bytes(4, 14336, 4096)[2] == 33030144
    assert ops.gemm_kquant_a_ws_bytes(9, 4096) > 0


def test_error_strings():
    from snowllm_amd import _capi
    assert _capi.lib.snowllm_error_string(1)
    with pytest.raises(Exception):
        _capi.check(1, "probe")
