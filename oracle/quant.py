"""GGUF Q4_K / Q5_K / Q6_K / Q8_0 oracle -- TEST INFRASTRUCTURE ONLY.

Block formats and decode follow the reference's GGUF decoder
(snowllm/checkpoint/gguf/dequant.py:20-32 `_scales_min_k4`, :31-32 `_q8_0`, :82-92 `_q4_k`;
block sizes snowllm/checkpoint/gguf/__init__.py:45,49):

  Q4_K, 144 bytes per 256 weights: d fp16 @0, dmin fp16 @2, 12 bytes of 6-bit scales/mins @4,
  128 bytes of nibbles @16. Group g (0..3) of 32 bytes holds sub-block 2g in the low nibbles
  and sub-block 2g+1 in the high nibbles. w = d * sc_j * q - dmin * m_j.
  Q8_0, 34 bytes per 32 weights: d fp16 @0, 32 int8 @2. w = d * q.
  Q5_K, 176 bytes per 256 weights (dequant.py:95-109): d, dmin fp16 @0, @2, the Q4_K scale
  bytes @4, 32 bytes qh @16, 128 bytes of nibbles @48. The nibbles as in Q4_K; bit j of qh[l]
  is the fifth bit of weight l of sub-block j. w = d * sc_j * q - dmin * m_j, q in 0..31.
  Q6_K, 210 bytes per 256 weights (dequant.py:112-123): ql 128 bytes @0, qh 64 @128, 16 int8
  scales @192, d fp16 @208. Half n (128 weights) uses ql[64 n ..], qh[32 n ..], scales[8 n ..];
  its weight 32 p + l (p 0..3, l 0..31) is the low (p < 2) or high nibble of ql[32 (p & 1) + l]
  with bits 2p, 2p+1 of qh[l] above it, scaled by scales[2 p + l // 16]: w = d * sc * (q - 32).

The GEMV reference is x.float() @ W.float().T in float64 (tests/test_mixed_gguf.py:57-67
uses the same form in fp32).
"""
import numpy as np
import torch

QK_K = 256
Q4_K_BYTES = 144
Q5_K_BYTES = 176
Q6_K_BYTES = 210
Q8_0_BYTES = 34


def scales_min_k4(s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """6-bit (scale, min) unpack of the 12 scale bytes (dequant.py:20-28)."""
    s = s.astype(np.int32)
    sc = np.empty((s.shape[0], 8), dtype=np.int32)
    mn = np.empty_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def pack_scales_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of scales_min_k4 for values 0..63: [nb, 8] x2 -> [nb, 12] bytes."""
    sc = sc.astype(np.int32)
    mn = mn.astype(np.int32)
    s = np.zeros((sc.shape[0], 12), dtype=np.int32)
    s[:, 0:4] = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
    s[:, 4:8] = (mn[:, :4] & 63) | ((mn[:, 4:] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:] & 0xF) | ((mn[:, 4:] & 0xF) << 4)
    return s.astype(np.uint8)


def dequant_q4_k(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """[n*k/256*144] bytes -> float32 [n, k] (dequant.py:82-92, in fp32 like the reference).
    Each weight is fp32(d * sc_j) * q - fp32(dmin * m_j), as there; torch ops only for speed."""
    b = torch.from_numpy(np.ascontiguousarray(np.asarray(raw, dtype=np.uint8)).reshape(-1, Q4_K_BYTES))
    nb = b.shape[0]
    dd = b[:, 0:4].contiguous().view(torch.float16).float()
    d, dmin = dd[:, 0], dd[:, 1]
    s = b[:, 4:16].int()
    sc = torch.empty(nb, 8, dtype=torch.int32)
    mn = torch.empty_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    q = b[:, 16:144].reshape(nb, 4, 32)
    dsc = d[:, None] * sc.float()
    dmn = dmin[:, None] * mn.float()
    out = torch.empty(nb, 4, 2, 32)
    out[:, :, 0] = dsc[:, 0::2, None] * (q & 0xF).float() - dmn[:, 0::2, None]
    out[:, :, 1] = dsc[:, 1::2, None] * (q >> 4).float() - dmn[:, 1::2, None]
    return out.reshape(n, k).numpy()


def dequant_q5_k(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """[n*k/256*176] bytes -> float32 [n, k]: fp32(d * sc_j) * q - fp32(dmin * m_j)."""
    b = np.ascontiguousarray(np.asarray(raw, dtype=np.uint8)).reshape(-1, Q5_K_BYTES)
    nb = b.shape[0]
    dd = b[:, 0:4].copy().view(np.float16).astype(np.float32)
    d, dmin = dd[:, 0], dd[:, 1]
    sc, mn = scales_min_k4(b[:, 4:16])
    qh = b[:, 16:48].astype(np.int32)                    # [nb, 32]
    q = b[:, 48:176].astype(np.int32).reshape(nb, 4, 32)
    dsc = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    dmn = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    out = np.empty((nb, 4, 2, 32), dtype=np.float32)
    for g in range(4):
        lo = (q[:, g] & 0xF) | (((qh >> (2 * g)) & 1) << 4)
        hi = (q[:, g] >> 4) | (((qh >> (2 * g + 1)) & 1) << 4)
        out[:, g, 0] = dsc[:, 2 * g, None] * lo.astype(np.float32) - dmn[:, 2 * g, None]
        out[:, g, 1] = dsc[:, 2 * g + 1, None] * hi.astype(np.float32) - dmn[:, 2 * g + 1, None]
    return out.reshape(n, k)


def dequant_q6_k(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """[n*k/256*210] bytes -> float32 [n, k]: fp32(d * sc) * (q - 32)."""
    b = np.ascontiguousarray(np.asarray(raw, dtype=np.uint8)).reshape(-1, Q6_K_BYTES)
    nb = b.shape[0]
    ql = b[:, 0:128].astype(np.int32).reshape(nb, 2, 64)
    qh = b[:, 128:192].astype(np.int32).reshape(nb, 2, 32)
    sc = b[:, 192:208].copy().view(np.int8).astype(np.float32).reshape(nb, 2, 8)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.empty((nb, 2, 4, 32), dtype=np.float32)
    l = np.arange(32)
    for p in range(4):
        base = ql[:, :, 32 * (p & 1):32 * (p & 1) + 32]
        nib = (base & 0xF) if p < 2 else (base >> 4)
        code = nib | (((qh >> (2 * p)) & 3) << 4)
        scale = (d[:, None, None] * sc[:, :, 2 * p + l // 16]).astype(np.float32)
        out[:, :, p] = scale * (code - 32).astype(np.float32)
    return out.reshape(n, k)


def dequant_q8_0(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """[n*k/32*34] bytes -> float32 [n, k] (dequant.py:31-32)."""
    b = torch.from_numpy(np.ascontiguousarray(np.asarray(raw, dtype=np.uint8)).reshape(-1, Q8_0_BYTES))
    d = b[:, 0:2].contiguous().view(torch.float16).float()
    q = b[:, 2:34].contiguous().view(torch.int8).float()
    return (d * q).reshape(n, k).numpy()


def make_q4_k(n: int, k: int, seed: int, d_std: float = 1e-3) -> np.ndarray:
    """Synthetic Q4_K weight: 6-bit scales/mins uniform 0..63,
    d, dmin = fp16(|N(0, d_std^2)|), nibbles uniform 0..15. Returns uint8 [n*k/256*144]."""
    assert k % QK_K == 0
    g = torch.Generator().manual_seed(seed)
    nb = n * k // QK_K
    sc = torch.randint(0, 64, (nb, 8), generator=g).numpy()
    mn = torch.randint(0, 64, (nb, 8), generator=g).numpy()
    dd = (torch.randn(nb, 2, generator=g) * d_std).abs().half().numpy()
    qs = torch.randint(0, 256, (nb, 128), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    blk = np.empty((nb, Q4_K_BYTES), dtype=np.uint8)
    blk[:, 0:4] = dd.view(np.uint8).reshape(nb, 4)
    blk[:, 4:16] = pack_scales_min_k4(sc, mn)
    blk[:, 16:] = qs
    return blk.reshape(-1)


def make_q4_k_centered(n: int, k: int, seed: int, d_std: float = 2e-4) -> np.ndarray:
    """Zero-mean synthetic Q4_K weight: scales uniform 0..63, m_j = round(0.9375 sc_j),
    d = fp16(|N(0, d_std^2)|), dmin = fp16(8 d), so that w = d sc_j q - dmin m_j is about
    d sc_j (q - 7.5). Returns uint8 [n*k/256*144]."""
    assert k % QK_K == 0
    g = torch.Generator().manual_seed(seed)
    nb = n * k // QK_K
    sc = torch.randint(0, 64, (nb, 8), generator=g).numpy()
    mn = np.clip(np.round(sc * 0.9375), 0, 63).astype(np.int64)
    d = (torch.randn(nb, generator=g) * d_std).abs()
    dd = torch.stack([d, 8 * d], 1).half().numpy()
    qs = torch.randint(0, 256, (nb, 128), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    blk = np.empty((nb, Q4_K_BYTES), dtype=np.uint8)
    blk[:, 0:4] = dd.view(np.uint8).reshape(nb, 4)
    blk[:, 4:16] = pack_scales_min_k4(sc, mn)
    blk[:, 16:] = qs
    return blk.reshape(-1)


def make_q8_0(n: int, k: int, seed: int, d_std: float = 1e-2) -> np.ndarray:
    """Synthetic Q8_0 weight: d = fp16(|N(0, d_std^2)|), int8 uniform
    -127..127. Returns uint8 [n*k/32*34]."""
    assert k % 32 == 0
    g = torch.Generator().manual_seed(seed)
    nb = n * k // 32
    d = (torch.randn(nb, generator=g) * d_std).abs().half().numpy()
    q = torch.randint(-127, 128, (nb, 32), generator=g, dtype=torch.int32).numpy().astype(np.int8)
    blk = np.empty((nb, Q8_0_BYTES), dtype=np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = q.view(np.uint8)
    return blk.reshape(-1)


def make_q5_k(n: int, k: int, seed: int, d_std: float = 1e-3) -> np.ndarray:
    """Synthetic Q5_K weight: as make_q4_k plus uniform qh bytes. uint8 [n*k/256*176]."""
    assert k % QK_K == 0
    g = torch.Generator().manual_seed(seed)
    nb = n * k // QK_K
    sc = torch.randint(0, 64, (nb, 8), generator=g).numpy()
    mn = torch.randint(0, 64, (nb, 8), generator=g).numpy()
    dd = (torch.randn(nb, 2, generator=g) * d_std).abs().half().numpy()
    qs = torch.randint(0, 256, (nb, 160), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    blk = np.empty((nb, Q5_K_BYTES), dtype=np.uint8)
    blk[:, 0:4] = dd.view(np.uint8).reshape(nb, 4)
    blk[:, 4:16] = pack_scales_min_k4(sc, mn)
    blk[:, 16:] = qs
    return blk.reshape(-1)


def make_q6_k(n: int, k: int, seed: int, d_std: float = 1e-4) -> np.ndarray:
    """Synthetic Q6_K weight: ql/qh bytes uniform, int8 scales uniform -128..127,
    d = fp16(|N(0, d_std^2)|). uint8 [n*k/256*210]."""
    assert k % QK_K == 0
    g = torch.Generator().manual_seed(seed)
    nb = n * k // QK_K
    q = torch.randint(0, 256, (nb, 192), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    sc = torch.randint(-128, 128, (nb, 16), generator=g, dtype=torch.int32).numpy().astype(np.int8)
    d = (torch.randn(nb, generator=g) * d_std).abs().half().numpy()
    blk = np.empty((nb, Q6_K_BYTES), dtype=np.uint8)
    blk[:, 0:192] = q
    blk[:, 192:208] = sc.view(np.uint8)
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def make(fmt: int, n: int, k: int, seed: int) -> np.ndarray:
    return {4: make_q4_k, 5: make_q5_k, 6: make_q6_k, 8: make_q8_0}[fmt](n, k, seed)


def make_activations(m: int, k: int, seed: int) -> torch.Tensor:
    """bf16 ~N(0,1) activations [m, k]."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).bfloat16()


def gemv_reference(x_bf16: torch.Tensor, w: np.ndarray) -> np.ndarray:
    """x.float() @ W.T in float64: [m, n]."""
    x = x_bf16.float().double().numpy()
    return x @ w.astype(np.float64).T


def dequant(raw: np.ndarray, fmt: int, n: int, k: int) -> np.ndarray:
    if fmt == 4:
        return dequant_q4_k(raw, n, k)
    if fmt == 5:
        return dequant_q5_k(raw, n, k)
    if fmt == 6:
        return dequant_q6_k(raw, n, k)
    if fmt == 8:
        return dequant_q8_0(raw, n, k)
    raise ValueError(fmt)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    """Relative L2 error, the reference harness's `rel` (tests/_harness.py:71-74)."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-9))
