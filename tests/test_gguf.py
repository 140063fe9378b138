"""GGUF reader and writer on the CPU, against files built byte by byte here (the reference's own
GGUF tests build their fixtures the same way: tests/test_qwen4exp_fused_gguf.py:26-45), and the
checkpoint's config and layer checks (snowllm/checkpoint/gguf/names.py:37-100)."""
import pathlib
import struct

import numpy as np
import pytest
import torch

from snowllm_amd.errors import SnowLLMError
from snowllm_amd.gguf import GGUF, QUANTS, split_parts, write_gguf


def s(text):
    raw = text.encode()
    return struct.pack("<Q", len(raw)) + raw


def handmade(path, kv_bytes, n_kv, tensors, alignment=32, version=3, pad_data=True):
    """A GGUF file from explicit bytes: kv_bytes already encoded; tensors (name, dims innermost
    first, ggml type id, payload) laid out at aligned offsets."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), n_kv) + kv_bytes
    data = b""
    for name, dims, kind, payload in tensors:
        head += s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", kind, len(data))
        data += payload + b"\0" * (-len(payload) % alignment)
    head += b"\0" * (-len(head) % alignment)
    path.write_bytes(head + (data if pad_data else data.rstrip(b"\0")))
    return path


def test_known_answer_header(tmp_path):
    kv = (s("general.architecture") + struct.pack("<I", 8) + s("qwen35moe")
          + s("a.u8") + struct.pack("<IB", 0, 200)
          + s("a.i8") + struct.pack("<Ib", 1, -5)
          + s("a.u16") + struct.pack("<IH", 2, 65000)
          + s("a.i16") + struct.pack("<Ih", 3, -300)
          + s("a.u32") + struct.pack("<II", 4, 4000000000)
          + s("a.i32") + struct.pack("<Ii", 5, -7)
          + s("a.f32") + struct.pack("<If", 6, 0.25)
          + s("a.bool") + struct.pack("<I?", 7, True)
          + s("a.u64") + struct.pack("<IQ", 10, 1 << 40)
          + s("a.i64") + struct.pack("<Iq", 11, -(1 << 40))
          + s("a.f64") + struct.pack("<Id", 12, -1.5)
          + s("a.ints") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 1, -2, 3)
          + s("a.strs") + struct.pack("<IIQ", 9, 8, 2) + s("x") + s("yz")
          + s("a.nested") + struct.pack("<IIQ", 9, 9, 2)
          + struct.pack("<IQ", 4, 2) + struct.pack("<2I", 1, 2)
          + struct.pack("<IQ", 8, 1) + s("w"))
    q4k = bytes(range(256)) + bytes(range(32))          # 2 blocks of 144 bytes
    f32 = struct.pack("<3f", 1.0, -2.0, 0.5)
    q80 = bytes((7 * i) % 256 for i in range(34 * 4))   # 4 blocks of 34 bytes
    p = handmade(tmp_path / "m.gguf", kv, 15, [
        ("w.q4k", (256, 2), 12, q4k), ("n.f32", (3,), 0, f32), ("w.q8", (64, 2), 8, q80)])
    g = GGUF(p)
    assert g.version == 3 and g.alignment == 32 and g.arch == "qwen35moe"
    assert g.kv["a.u8"] == 200 and g.kv["a.i8"] == -5 and g.kv["a.u16"] == 65000
    assert g.kv["a.i16"] == -300 and g.kv["a.u32"] == 4000000000 and g.kv["a.i32"] == -7
    assert g.kv["a.f32"] == 0.25 and g.kv["a.bool"] is True and g.kv["a.u64"] == 1 << 40
    assert g.kv["a.i64"] == -(1 << 40) and g.kv["a.f64"] == -1.5
    assert g.kv["a.ints"] == [1, -2, 3] and g.kv["a.strs"] == ["x", "yz"]
    assert g.kv["a.nested"] == [[1, 2], ["w"]]
    assert g.get("{arch}.missing", 9) == 9 and g.get("general.architecture") == "qwen35moe"
    t = g["w.q4k"]
    assert t.shape == (2, 256) and t.dims == (256, 2) and t.quant.name == "Q4_K"
    assert t.nbytes == 288 and t.offset == 0
    assert g["n.f32"].offset == 288 and g["w.q8"].offset == 288 + 32
    assert g.read("w.q4k") == q4k and g.read("w.q8") == q80
    assert g.tensor("n.f32").tolist() == [1.0, -2.0, 0.5]
    assert bytes(g.payload("w.q8").numpy()) == q80
    with pytest.raises(SnowLLMError):
        g.tensor("w.q4k")
    with pytest.raises(SnowLLMError):
        g["absent"]
    with pytest.raises(SnowLLMError):
        g.need("{arch}.block_count")
    g.close()


def test_block_geometry_matches_the_format():
    """Q4_K: fp16 d + fp16 dmin + 12 bytes of scales + 128 nibble bytes per 256 weights;
    Q8_0: fp16 d + 32 int8 per 32; and the library's repack size query agrees."""
    assert (QUANTS["Q4_K"].block, QUANTS["Q4_K"].size) == (256, 2 + 2 + 12 + 128)
    assert (QUANTS["Q8_0"].block, QUANTS["Q8_0"].size) == (32, 2 + 32)
    assert (QUANTS["F16"].size, QUANTS["BF16"].size, QUANTS["F32"].size) == (2, 2, 4)
    from snowllm_amd import ops
    for name, fmt in (("Q4_K", 4), ("Q8_0", 8)):
        assert ops.kquant_bytes(fmt, 512, 1024)[2] == QUANTS[name].nbytes(512 * 1024)
    with pytest.raises(SnowLLMError):
        QUANTS["Q4_K"].nbytes(100)


def test_writer_is_the_byte_layout(tmp_path):
    """write_gguf's bytes equal the hand-built file for the same content."""
    payload = bytes(range(34))
    want = handmade(tmp_path / "a.gguf", s("general.architecture") + struct.pack("<I", 8)
                    + s("x") + s("x.n") + struct.pack("<II", 4, 7), 2,
                    [("t", (32, 1), 8, payload), ("u", (2,), 0, struct.pack("<2f", 1, 2))])
    got = write_gguf(tmp_path / "b.gguf", {"general.architecture": "x", "x.n": 7},
                     [("t", (1, 32), "Q8_0", payload),
                      ("u", (2,), "F32", np.array([1, 2], np.float32))])
    assert got.read_bytes() == want.read_bytes()


def test_round_trip_and_alignment(tmp_path):
    g0 = torch.Generator().manual_seed(0)
    tensors = [("a", (3, 256), "Q4_K", torch.randint(0, 256, (3 * 144,), generator=g0,
                                                     dtype=torch.uint8)),
               ("b", (5,), "F16", torch.randn(5, generator=g0).half()),
               ("c", (2, 4), "BF16", torch.randn(2, 4, generator=g0).bfloat16()),
               ("d", (64,), "Q8_0", torch.randint(0, 256, (68,), generator=g0,
                                                 dtype=torch.uint8))]
    meta = {"general.architecture": "qwen35", "qwen35.list": [0.5, 1.5], "qwen35.flag": False}
    for alignment in (32, 64, 256):
        p = write_gguf(tmp_path / f"r{alignment}.gguf", meta, tensors, alignment=alignment)
        g = GGUF(p)
        assert g.alignment == alignment
        for name, shape, q, data in tensors:
            assert g[name].shape == shape and g[name].quant.name == q
            assert g[name].offset % alignment == 0
            assert torch.equal(g.payload(name), data.contiguous().view(-1).view(torch.uint8))
        assert torch.equal(g.tensor("c"), tensors[2][3])
        assert g.kv["qwen35.list"] == [0.5, 1.5] and g.kv["qwen35.flag"] is False
        g.close()


@pytest.mark.parametrize("corrupt, message", [
    (lambda b: b"GGUX" + b[4:], "magic"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "version"),
    (lambda b: b[:40], "truncated"),
])
def test_bad_files_are_refused(tmp_path, corrupt, message):
    good = write_gguf(tmp_path / "g.gguf", {"general.architecture": "x", "x.k": "some text"},
                      [("t", (32,), "Q8_0", bytes(34))]).read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(corrupt(good))
    with pytest.raises(SnowLLMError, match=message):
        GGUF(bad)


def test_structural_errors(tmp_path):
    ok_kv = s("general.architecture") + struct.pack("<I", 8) + s("x")
    with pytest.raises(SnowLLMError, match="ggml type 99"):
        GGUF(handmade(tmp_path / "a.gguf", ok_kv, 1, [("t", (4,), 99, bytes(16))]))
    with pytest.raises(SnowLLMError, match="second tensor"):
        GGUF(handmade(tmp_path / "b.gguf", ok_kv, 1, [("t", (4,), 0, bytes(16)),
                                                      ("t", (4,), 0, bytes(16))]))
    with pytest.raises(SnowLLMError, match="past the end"):
        GGUF(handmade(tmp_path / "c.gguf", ok_kv, 1, [("t", (40,), 0, bytes(16))]))
    bad_align = ok_kv + s("general.alignment") + struct.pack("<II", 4, 24)
    with pytest.raises(SnowLLMError, match="power of two"):
        GGUF(handmade(tmp_path / "d.gguf", bad_align, 2, [("t", (4,), 0, bytes(16))]))
    # an offset off the alignment
    p = tmp_path / "e.gguf"
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 1) + ok_kv + s("t") + struct.pack("<IQIQ", 1, 4, 0, 8)
    head += b"\0" * (-len(head) % 32)
    p.write_bytes(head + bytes(64))
    with pytest.raises(SnowLLMError, match="alignment"):
        GGUF(p)


def test_split_checkpoint(tmp_path):
    tensors = [(f"t{i}", (32,), "Q8_0", bytes([i]) * 34) for i in range(5)]
    kv = {"general.architecture": "x"}
    for i, chunk in enumerate((tensors[:2], tensors[2:4], tensors[4:])):
        meta = dict(kv, **{"split.no": i, "split.count": 3, "split.tensors.count": 5})
        write_gguf(tmp_path / f"m-{i + 1:05d}-of-00003.gguf", meta, chunk)
    g = GGUF(tmp_path / "m-00001-of-00003.gguf")
    assert len(g.parts) == 3 and sorted(g.tensors) == [f"t{i}" for i in range(5)]
    for i in range(5):
        assert g.read(f"t{i}") == bytes([i]) * 34
    assert g["t4"].part == 2
    # any part names the whole checkpoint
    assert split_parts(tmp_path / "m-00002-of-00003.gguf") == g.parts
    g.close()
    (tmp_path / "m-00003-of-00003.gguf").unlink()
    with pytest.raises(SnowLLMError, match="absent"):
        GGUF(tmp_path / "m-00001-of-00003.gguf")
    write_gguf(tmp_path / "m-00003-of-00003.gguf", dict(kv, **{"split.count": 3}), tensors[4:])
    write_gguf(tmp_path / "m-00001-of-00003.gguf",
               dict(kv, **{"split.count": 3, "split.tensors.count": 6}), tensors[:2])
    with pytest.raises(SnowLLMError, match="split.tensors.count"):
        GGUF(tmp_path / "m-00001-of-00003.gguf")


# ---- the checkpoint's config and layer checks (no kernel runs) -------------------------------
def _tiny_cfg(moe=True):
    from snowllm_amd.verify import VerifyConfig
    base = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rot_half=32,
                rope_theta=1e4, vocab=1024, context=300, block=9)
    if moe:
        return VerifyConfig("tiny_moe", experts=8, expert_ffn=256, topk=2, **base)
    return VerifyConfig("tiny_dense", ffn=512, **base)


def _fake_tensors(cfg, fmt="Q4_K", **override):
    """Tensor list of the right names, shapes and formats, zero payloads."""
    H, d = cfg.hidden, cfg.head_dim
    out = []

    def add(name, shape, q):
        nbytes = QUANTS[q].nbytes(int(np.prod(shape)))
        out.append((name, shape, q, bytes(nbytes)))
    for i in range(cfg.layers):
        p = f"blk.{i}."
        q_rows = override.get("q_rows", cfg.heads * d)
        add(p + "attn_q.weight", (q_rows, H), fmt)
        add(p + "attn_k.weight", (cfg.kv_heads * d, H), override.get("k_fmt", fmt))
        add(p + "attn_v.weight", (cfg.kv_heads * d, H), fmt)
        add(p + "attn_output.weight", (H, cfg.heads * d), fmt)
        for n, w in (("attn_norm", H), ("post_attention_norm", H), ("attn_q_norm", d),
                     ("attn_k_norm", d)):
            add(p + n + ".weight", (w,), "F32")
        if cfg.moe:
            E, F = cfg.experts, cfg.expert_ffn
            add(p + "ffn_gate_inp.weight", (E, H), "F32")
            add(p + "ffn_gate_inp_shexp.weight", (H,), "F32")
            for n, shape in (("ffn_gate_exps", (E, F, H)), ("ffn_up_exps", (E, F, H)),
                             ("ffn_down_exps", (E, H, F)), ("ffn_gate_shexp", (F, H)),
                             ("ffn_up_shexp", (F, H)), ("ffn_down_shexp", (H, F))):
                q = override.get("ffn_fmt", fmt)
                add(p + n + ".weight", shape, override.get("down_fmt", q) if "down" in n else q)
        else:
            add(p + "ffn_gate.weight", (cfg.ffn, H), fmt)
            add(p + "ffn_up.weight", (cfg.ffn, H), fmt)
            add(p + "ffn_down.weight", (H, cfg.ffn), fmt)
        for extra in override.get("extra", ()):
            add(p + extra, (H,), "F32")
    add("token_embd.weight", (cfg.vocab, H), "F16")
    add("output_norm.weight", (H,), "F32")
    return out


@pytest.mark.parametrize("moe", [True, False])
def test_config_from_metadata(tmp_path, moe):
    from snowllm_amd.checkpoint import config_from_gguf, gguf_metadata
    cfg = _tiny_cfg(moe)
    p = write_gguf(tmp_path / "m.gguf", gguf_metadata(cfg), _fake_tensors(cfg))
    g = GGUF(p)
    got = config_from_gguf(g, context=cfg.context, block=cfg.block)
    for f in ("layers", "hidden", "heads", "kv_heads", "head_dim", "rot_half", "rope_theta",
              "vocab", "ffn", "experts", "expert_ffn", "topk", "attn_fmt", "ffn_fmt", "eps"):
        assert getattr(got, f) == pytest.approx(getattr(cfg, f)), f
    assert g.arch == ("qwen35moe" if moe else "qwen35")
    g.close()


def _refused(tmp_path, cfg, kv=None, layer=False, **override):
    from snowllm_amd import checkpoint as C
    meta = C.gguf_metadata(cfg)
    meta.update(kv or {})
    g = GGUF(write_gguf(tmp_path / "m.gguf", meta, _fake_tensors(cfg, **override)))
    try:
        if layer:
            C._layer(g, C.config_from_gguf(g, context=300, block=9), 0)
        else:
            C.config_from_gguf(g, context=300, block=9)
    finally:
        g.close()


def test_checkpoints_outside_the_path_are_refused(tmp_path):
    cfg = _tiny_cfg(True)
    with pytest.raises(SnowLLMError, match="linear attention"):
        _refused(tmp_path, cfg, {"qwen35moe.full_attention_interval": 4})
    with pytest.raises(SnowLLMError, match="shared expert width"):
        _refused(tmp_path, cfg, {"qwen35moe.expert_shared_feed_forward_length": 512})
    with pytest.raises(SnowLLMError, match="Q6_K experts"):
        _refused(tmp_path, cfg, ffn_fmt="Q8_0")
    with pytest.raises(SnowLLMError, match="narrower than the experts' gate/up"):
        _refused(tmp_path, cfg, layer=True, ffn_fmt="Q6_K", down_fmt="Q4_K")
    with pytest.raises(SnowLLMError, match="'llama' checkpoint"):
        _refused(tmp_path, cfg, {"general.architecture": "llama",
                                 **{k.replace("qwen35moe", "llama"): v
                                    for k, v in C_meta(cfg).items() if k.startswith("qwen35moe")}})
    with pytest.raises(SnowLLMError, match="without experts"):
        _refused(tmp_path, _tiny_cfg(False), {"general.architecture": "qwen35moe",
                                              **{k.replace("qwen35", "qwen35moe", 1): v
                                                 for k, v in C_meta(_tiny_cfg(False)).items()
                                                 if k.startswith("qwen35.")}})
    with pytest.raises(SnowLLMError, match="output gate"):
        _refused(tmp_path, cfg, layer=True, q_rows=2 * cfg.heads * cfg.head_dim)
    with pytest.raises(SnowLLMError, match="linear-attention"):
        _refused(tmp_path, cfg, layer=True, extra=("ssm_a",))
    with pytest.raises(SnowLLMError, match="one k-quant format"):
        _refused(tmp_path, cfg, layer=True, k_fmt="Q8_0")


def C_meta(cfg):
    from snowllm_amd import checkpoint as C
    return C.gguf_metadata(cfg)


@pytest.mark.parametrize("gu,dn", [("Q5_K", "Q5_K"), ("Q6_K", "Q6_K"), ("Q4_K", "Q6_K")])
def test_expert_formats_taken(tmp_path, gu, dn):
    """Q4_K_M / Q5_K_M / Q6_K files: experts in Q4_K, Q5_K or Q6_K, down as wide or wider."""
    from snowllm_amd import checkpoint as C
    from snowllm_amd.gguf import KQUANT_FORMAT
    cfg = _tiny_cfg(True)
    g = GGUF(write_gguf(tmp_path / "m.gguf", C.gguf_metadata(cfg),
                        _fake_tensors(cfg, ffn_fmt=gu, down_fmt=dn)))
    try:
        assert C.config_from_gguf(g, context=300, block=9).ffn_fmt == KQUANT_FORMAT[gu]
    finally:
        g.close()


def test_norm_weight_convention():
    """The stored norm weight passes through bf16(w - 1) before the one is added back
    (source.py:338-340, qwen3_5_weights.py:39-40): weights near one whose bf16 form is exact
    come back unchanged; a small weight loses itself (bf16(0.001 - 1) is -1)."""
    from snowllm_amd.checkpoint import norm_weight
    w = torch.tensor([1.0, 1.0078125, 0.99609375, 1.5, 0.001, 3.0e-4, 2.0])
    got = norm_weight(w)
    assert got.dtype == torch.bfloat16
    assert got.float().tolist() == [1.0, 1.0078125, 0.99609375, 1.5, 0.0, 0.0, 2.0]
    # 1 + 2^-9 is not a bf16 value: bf16(2^-9) = 2^-9 is exact, then 1 + 2^-9 rounds to 1
    assert norm_weight(torch.tensor([1.0 + 2.0 ** -9])).item() == 1.0
