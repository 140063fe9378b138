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


def _q5k_scalar(b):
    """One Q5_K block decoded weight by weight in the GGML reference order (64 weights per
    step j: the low nibbles of qs[32 j ..] with qh bit 2j, then the high nibbles with bit
    2j + 1), a formulation independent of the oracle's vectorised one."""
    d = float(np.frombuffer(b[0:2].tobytes(), np.float16)[0])
    dmin = float(np.frombuffer(b[2:4].tobytes(), np.float16)[0])
    sc, mn = Q.scales_min_k4(b[None, 4:16])
    qh, qs = b[16:48], b[48:176]
    y = np.zeros(256, np.float64)
    for j in range(4):
        d1, m1 = d * sc[0, 2 * j], dmin * mn[0, 2 * j]
        d2, m2 = d * sc[0, 2 * j + 1], dmin * mn[0, 2 * j + 1]
        for l in range(32):
            q = qs[32 * j + l]
            y[64 * j + l] = d1 * ((q & 15) + (16 if qh[l] & (1 << 2 * j) else 0)) - m1
            y[64 * j + 32 + l] = d2 * ((q >> 4) + (16 if qh[l] & (2 << 2 * j) else 0)) - m2
    return y


def _q6k_scalar(b):
    """One Q6_K block decoded weight by weight in the GGML reference order (per 128-weight
    half: four 32-weight runs from ql[l], ql[l + 32] low and high nibbles and the four bit
    pairs of qh[l], scale index l // 16 + 0, 2, 4, 6)."""
    d = float(np.frombuffer(b[208:210].tobytes(), np.float16)[0])
    y = np.zeros(256, np.float64)
    for n in range(2):
        ql, qh = b[64 * n:64 * n + 64], b[128 + 32 * n:128 + 32 * n + 32]
        sc = b[192 + 8 * n:192 + 8 * n + 8].view(np.int8)
        for l in range(32):
            s = l // 16
            q1 = (int(ql[l]) & 15 | ((int(qh[l]) >> 0) & 3) << 4) - 32
            q2 = (int(ql[l + 32]) & 15 | ((int(qh[l]) >> 2) & 3) << 4) - 32
            q3 = (int(ql[l]) >> 4 | ((int(qh[l]) >> 4) & 3) << 4) - 32
            q4 = (int(ql[l + 32]) >> 4 | ((int(qh[l]) >> 6) & 3) << 4) - 32
            y[128 * n + l] = d * sc[s] * q1
            y[128 * n + 32 + l] = d * sc[s + 2] * q2
            y[128 * n + 64 + l] = d * sc[s + 4] * q3
            y[128 * n + 96 + l] = d * sc[s + 6] * q4
    return y


def test_q5k_known_answer():
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:4] = np.array([0.5], np.float16).view(np.uint8)
    b[4:16] = Q.pack_scales_min_k4(np.array([[1, 2, 3, 4, 5, 6, 7, 8]]),
                                   np.array([[0, 1, 0, 1, 0, 1, 0, 2]]))
    b[48 + 0] = 0x3A        # group 0, l = 0: low 10 (sub-block 0), high 3 (sub-block 1)
    b[16 + 0] = 0b00000011  # qh[0]: fifth bits of sub-blocks 0 and 1
    b[48 + 96 + 5] = 0xF0   # group 3, l = 5: low 0, high 15 (sub-block 7)
    b[16 + 5] = 0b10000000  # qh[5] bit 7: sub-block 7's fifth bit
    w = Q.dequant_q5_k(b, 1, 256)[0]
    assert w[0] == 1 * (10 + 16) - 0
    assert w[32] == 2 * (3 + 16) - 0.5
    assert w[192 + 5] == 7 * 0 - 0
    assert w[224 + 5] == 8 * (15 + 16) - 1.0
    assert w[1] == 0 and w[33] == -0.5
    assert np.array_equal(w.astype(np.float64), _q5k_scalar(b))


def test_q6k_known_answer():
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([1.0], np.float16).view(np.uint8)
    b[192:208] = (np.arange(16) + 1).astype(np.int8).view(np.uint8)   # scales 1..16
    b[0] = 0x05; b[128 + 0] = 0b10          # n 0, p 0, l 0: q = 5 | 2 << 4 = 37 -> +5 x sc 1
    b[17] = 0x90; b[128 + 17] = 0b110000     # n 0, p 2, l 17: q = 9 | 3 << 4 = 57 -> 25 x sc 6
    b[127] = 0xF0                            # n 1, p 3, l 31: q = 15 -> -17 x sc 16
    b[99] = 0x00; b[128 + 35] = 0b0100       # n 1, p 1, l 3: q = 0 | 1 << 4 = 16 -> -16 x sc 11
    w = Q.dequant_q6_k(b, 1, 256)[0]
    assert w[0] == 5 * 1
    assert w[64 + 17] == 25 * 6
    assert w[128 + 96 + 31] == -17 * 16
    assert w[128 + 32 + 3] == -16 * 11
    assert w[1] == -32 * 1 and w[16] == -32 * 2      # empty weights: q = 0, scale per 16
    assert np.array_equal(w.astype(np.float64), _q6k_scalar(b))


def test_q5k_q6k_random_blocks_match_scalar_decode():
    for fmt, scalar, size in ((5, _q5k_scalar, 176), (6, _q6k_scalar, 210)):
        raw = Q.make(fmt, 4, 256, seed=11).reshape(-1, size)
        got = Q.dequant(raw.reshape(-1), fmt, 4, 256)
        for i in range(4):
            want = scalar(raw[i])
            assert np.allclose(got[i], want, rtol=1e-6, atol=0), fmt
