"""Pins the GGUF decode oracle (oracle/quant.py) with hand-built known-answer blocks and
closed-form special cases. CPU only."""
import numpy as np
import torch

from oracle import quant as Q


def _block(d, dmin, scale_bytes, nibbles):
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    b[4:16] = scale_bytes
    b[16:] = nibbles
    return b


def test_q4k_known_answer():
    # scale bytes: s[0..3] = 1,2,3,4 (sc 0..3), s[4..7] = 5,6,7,8 (m 0..3),
    # s[8..11] = 0x21,0x43,0x65,0x87 (low nibble sc 4..7 = 1,3,5,7; high nibble m 4..7 = 2,4,6,8)
    sb = np.array([1, 2, 3, 4, 5, 6, 7, 8, 0x21, 0x43, 0x65, 0x87], dtype=np.uint8)
    # byte l of group g: low nibble = 1 (sub-block 2g), high nibble = 2 (sub-block 2g+1)
    nib = np.full(128, 0x21, dtype=np.uint8)
    w = Q.dequant_q4_k(_block(1.0, 0.5, sb, nib), 1, 256)[0]
    # sub-block j: weight = 1.0 * sc_j * q - 0.5 * m_j, q = 1 on even j, 2 on odd j
    sc = [1, 2, 3, 4, 1, 3, 5, 7]
    mn = [5, 6, 7, 8, 2, 4, 6, 8]
    for j in range(8):
        q = 1 if j % 2 == 0 else 2
        assert np.all(w[32 * j:32 * j + 32] == sc[j] * q - 0.5 * mn[j]), j


def test_q4k_high_scale_bits():
    # top two bits of s[0..3] / s[4..7] become bits 4..5 of sc/m 4..7
    sb = np.array([0xC0 | 1, 0x40, 0x80, 0, 0xC0, 0, 0, 0, 0x0F, 0, 0, 0xF0], dtype=np.uint8)
    sc, mn = Q.scales_min_k4(sb[None])
    assert list(sc[0]) == [1, 0, 0, 0, 15 | (3 << 4), 1 << 4, 2 << 4, 0]
    assert list(mn[0]) == [0, 0, 0, 0, 3 << 4, 0, 0, 15]


def test_q4k_special_cases():
    g = np.random.default_rng(0)
    sb = g.integers(0, 256, 12, dtype=np.uint8)
    nib = g.integers(0, 256, 128, dtype=np.uint8)
    assert np.all(Q.dequant_q4_k(_block(0.0, 0.0, sb, nib), 1, 256) == 0)      # d = dmin = 0
    sc, mn = Q.scales_min_k4(sb[None])
    w = Q.dequant_q4_k(_block(0.0, 0.25, sb, nib), 1, 256)[0]                 # d = 0: -dmin*m
    assert np.all(w == np.repeat(-0.25 * mn[0], 32))
    w = Q.dequant_q4_k(_block(0.5, 0.0, sb, np.zeros(128, np.uint8)), 1, 256)[0]  # q = 0
    assert np.all(w == 0)
    w = Q.dequant_q4_k(_block(0.5, 0.0, sb, np.full(128, 0xFF, np.uint8)), 1, 256)[0]  # q = 15
    assert np.all(w == np.repeat(0.5 * 15 * sc[0], 32))


def test_scale_pack_roundtrip():
    g = np.random.default_rng(1)
    sc = g.integers(0, 64, (100, 8))
    mn = g.integers(0, 64, (100, 8))
    s2, m2 = Q.scales_min_k4(Q.pack_scales_min_k4(sc, mn))
    assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


def test_q80_known_answer():
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    q = np.arange(-16, 16, dtype=np.int8)
    b[2:] = q.view(np.uint8)
    assert np.array_equal(Q.dequant_q8_0(b, 1, 32)[0], 0.5 * q.astype(np.float32))


def test_generators_match_baseline_ranges():
    raw = Q.make_q4_k(32, 512, seed=2)
    assert raw.size == 32 * 2 * 144
    b = raw.reshape(-1, 144)
    sc, mn = Q.scales_min_k4(b[:, 4:16])
    assert sc.min() >= 0 and sc.max() <= 63 and mn.max() <= 63
    d = b[:, 0:2].copy().view(np.float16)
    assert np.all(d >= 0) and 1e-5 < float(np.abs(d.astype(np.float32)).mean()) < 2e-3
    raw8 = Q.make_q8_0(16, 256, seed=3)
    q = raw8.reshape(-1, 34)[:, 2:].copy().view(np.int8)
    assert q.min() >= -127 and q.max() <= 127


def test_gemv_reference_brute_force():
    raw = Q.make_q4_k(4, 256, seed=7)
    w = Q.dequant_q4_k(raw, 4, 256)
    x = Q.make_activations(3, 256, seed=8)
    y = Q.gemv_reference(x, w)
    for r in range(3):
        for n in range(4):
            s = sum(float(x[r, i]) * float(w[n, i]) for i in range(256))
            assert abs(y[r, n] - s) <= 1e-9 * max(1.0, abs(s))
