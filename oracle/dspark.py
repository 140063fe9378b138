"""CPU restatement of the DSpark Markov head (snowllm/ops/dspark.py:53-77, semantics from the
PyTorch reference the reference's own test runs: tests/test_lfm2_dspark_reference.py:143-152).
Test infrastructure only: tests, smoke() and bench.py's cpu_baseline may import it; the product
never does.

For each request r and block row j (row index r * block + j of base / pre_head):
    prev     = anchor[r] for j = 0, else path[r, j - 1]
    latent   = W1[prev]                                      bf16 [rank]
    bias[n]  = round(sum_i W2[n, i] * latent[i])             bf16 (fp32 when fp32_bias)
    conf     = sigmoid(cat(pre_head[row], latent) . conf_w + conf_b)
    path[r, j] = argmax_n fp32(base[row, n] + bias[n])

The reference's F.linear in bf16 accumulates in fp32 and rounds once; here the sum is taken in
fp64, where every product of two bf16 values is exact and the sum of a row's products is exact
while their magnitudes span less than 2^29 (beyond that its error stays below 2^-53 of the
largest product), then rounded once to nearest-even: the result does not depend on the
summation order, so a kernel that sums in another order gives the same bits. The
argmax counts NaN as -inf and -0 as +0 and takes the lowest index among equal maxima, as
ops.argmax (tests/test_sampling_argmax.py:29-30). A prev outside [0, V) gives a zero latent.
Parity of this restatement is pinned in tests/test_oracle_dspark.py.
"""
import numpy as np


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, np.float32))
    return np.where(nan, (u >> 16) | 0x40, r).astype(np.uint16)


def round_f64_to_bf16(d: np.ndarray) -> np.ndarray:
    """fp64 -> the nearest bf16 value (ties to even), rounded once, as fp32 values. Works on
    the fp64 bit pattern: keep 7 fraction bits of the 52, rounding on the 45 dropped ones."""
    d = np.ascontiguousarray(d, np.float64)
    tiny = np.abs(d) < 2.0 ** -126        # bf16 subnormals: multiples of 2^-133
    if tiny.any():
        d = d.copy()
        d[tiny] = np.round(d[tiny] * 2.0 ** 133) * 2.0 ** -133   # numpy rounds half to even
    u = d.view(np.uint64)
    drop = np.uint64(45)
    lsb = (u >> drop) & np.uint64(1)
    r = (u + np.uint64((1 << 44) - 1) + lsb) & ~np.uint64((1 << 45) - 1)   # half - 1 + lsb
    out = r.view(np.float64).astype(np.float32)   # exact: 8 significant bits
    return np.where(np.isfinite(d), out, d.astype(np.float32))


def ord_argmax(v: np.ndarray) -> int:
    """Lowest index of the maximum; NaN counts as -inf, -0 equals +0."""
    v = np.where(np.isnan(v), -np.inf, v).astype(np.float64)
    return int(np.argmax(v))


def markov(base, w1, w2, anchor, block, pre_head=None, conf_w=None, conf_b=None,
           fp32_bias=False):
    """base f32 [b * block, V]; w1, w2 bf16 bit patterns (uint16) [V, rank]; anchor i64 [b]
    -> path i64 [b, block], confidence f64 [b, block] (None without conf_w)."""
    base = np.asarray(base, np.float32)
    W1 = bf16_bits_to_f32(w1).astype(np.float64)
    W2 = bf16_bits_to_f32(w2).astype(np.float64)
    V, rank = W1.shape
    b = len(anchor)
    path = np.zeros((b, block), np.int64)
    conf = None if conf_w is None else np.zeros((b, block), np.float64)
    for r in range(b):
        prev = int(anchor[r])
        for j in range(block):
            row = r * block + j
            latent = W1[prev] if 0 <= prev < V else np.zeros(rank)
            exact = W2 @ latent
            bias = exact.astype(np.float32) if fp32_bias else round_f64_to_bf16(exact)
            vals = (base[row, :V] + bias).astype(np.float32)
            if conf is not None:
                hidden = bf16_bits_to_f32(pre_head[row]).astype(np.float64)
                z = np.dot(np.concatenate([hidden, latent]), np.asarray(conf_w, np.float64))
                z += 0.0 if conf_b is None else float(conf_b)
                conf[r, j] = 1.0 / (1.0 + np.exp(-z))
            prev = ord_argmax(vals)
            path[r, j] = prev
    return path, conf
