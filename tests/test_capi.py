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


def _type_name(t):
    import ctypes
    from snowllm_amd import _capi
    if t is None:
        return "None"
    if t is _capi.Stream:
        return "S"
    if t is ctypes.c_void_p:
        return "P"
    if t is ctypes.c_int64:   # an alias of c_long here
        return "c_int64"
    return t.__name__


def test_bindings_match_the_reference_signatures():
    """Every snowllm_* entry point keeps the reference binding's ctypes signature
    (snowllm/_capi.py:201-831, as recorded by tests/golden/make_reference_capi_signatures.py),
    so that the reference's ops wrappers can call this library unchanged."""
    import json
    from snowllm_amd import _capi
    ref = json.loads((ROOT / "tests" / "golden" / "reference_capi_signatures.json").read_text())
    ref = ref["signatures"]
    ours = {n: (r, a) for n, r, a in _capi._SIGS if n.startswith("snowllm_")}
    # the ABI check is bound outside the table in the reference (snowllm/_capi.py:179-194)
    ours.pop("snowllm_abi_version")
    missing = sorted(set(ours) - set(ref))
    assert not missing, f"snowllm_* names the reference does not declare: {missing}"
    bad = []
    for name, (res, args) in sorted(ours.items()):
        want = ref[name]
        got = {"restype": _type_name(res), "argtypes": [_type_name(a) for a in args]}
        if got != want:
            bad.append((name, got, want))
    assert not bad, "\n".join(f"{n}: ours {g} reference {w}" for n, g, w in bad)
    # the symbols the reference's hot-path ops modules look up at import are bound
    # (ops/_common.py:42-43, attention_full.py:511-513, 565, dflash.py:337-338,
    # embedding.py:44, moe.py:89, 279, mlp.py:71)
    for name in ("snowllm_sampling_max_k", "snowllm_kv_block_sizes",
                 "snowllm_paged_decode_max_q_tokens", "snowllm_paged_decode_plan_elems",
                 "snowllm_qkv_proj_scratch_bytes", "snowllm_attn_out_scale_oproj_scratch_bytes",
                 "snowllm_draft_paged_attn_workspace_size", "snowllm_draft_paged_attn_num_slots",
                 "snowllm_lm_head_scratch_bytes", "snowllm_moe_workspace_bytes",
                 "snowllm_fused_mlp_workspace_bytes", "snowllm_moe_router_shuffle_bytes"):
        assert name in ours


def test_decode_plan_queries():
    """The split-KV decode sizing queries answer for the default geometry without a GPU."""
    import ctypes
    from snowllm_amd import _capi
    lib = _capi.lib
    buf = (ctypes.c_int64 * 4)()
    assert lib.snowllm_kv_block_sizes(None, 0) == 1
    assert lib.snowllm_kv_block_sizes(buf, 4) == 1 and buf[0] == 16
    assert 1 <= lib.snowllm_paged_decode_max_q_tokens() <= 64
    assert lib.snowllm_paged_decode_num_slots(3) == 3
    assert lib.snowllm_paged_decode_plan_elems(3, 3) >= 1
    lens = (ctypes.c_int32 * 3)(1, 17, 32)
    total = lib.snowllm_prefill_q_blocks(lens, 3)
    assert total == 1 + 2 + 2
    m = (ctypes.c_int32 * (2 * total))()
    lib.snowllm_prefill_q_block_map(lens, 3, m)
    assert list(m) == [0, 0, 1, 0, 1, 16, 2, 0, 2, 16]
    assert lib.snowllm_paged_attention_prepared_bytes(1, 9, 1, 0) == 0


def test_moe_plan_layout_and_slot_bound():
    """The host view of a MoE plan (layers.parse_plan) matches the library's struct, and the slot
    bound is what the plan can take: one slot per used expert up to 16 rows; above, one per 16
    rows of an expert and the shared expert's ceil(M / 16); 0 past 64 rows or 512 picks."""
    from snowllm_amd import layers as L
    from snowllm_amd._capi import lib
    S = L.MOE_MAX_SLOTS
    assert L.MOE_PLAN_BYTES == (2 + 2 * S + 2 * S * 16 + 1) * 4
    bound = lib.snowverify_moe_max_slots
    assert bound(9, 8, 256, 1) == 73 and bound(9, 8, 256, 0) == 72
    assert bound(1, 8, 256, 1) == 9 and bound(16, 16, 256, 1) == 257
    assert bound(36, 8, 256, 1) == 256 + 288 // 16 + 3
    assert bound(64, 8, 256, 1) == S and bound(64, 8, 64, 0) == 64 + 32
    assert bound(65, 8, 256, 1) == 0 and bound(64, 9, 256, 1) == 0 and bound(0, 8, 256, 1) == 0
    # the bound holds for every routing: experts with c rows take ceil(c / 16) slots
    import numpy as np
    rng = np.random.default_rng(0)
    for _ in range(200):
        M, K, E = int(rng.integers(1, 65)), int(rng.integers(1, 9)), int(rng.integers(8, 257))
        if M * K > 512 or K > E:
            continue
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(M)])
        counts = np.bincount(ids.ravel(), minlength=E)
        slots = int(((counts + 15) // 16).sum()) + (M + 15) // 16
        assert slots <= bound(M, K, E, 1), (M, K, E)
