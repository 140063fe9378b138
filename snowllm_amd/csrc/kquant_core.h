// Shared device code of the k-quant GEMV family (plain GEMV, fused gate/up + SwiGLU, MoE
// experts): operand workspace layout, activation conversion, nibble/byte decoders, the
// per-superblock MFMA tile and the double-buffered superblock loop.
//
// Arithmetic (per 32-weight sub-block j, column n, row r):
//   y[r,n] = sum_j  a_j * sum_i q_i x_ri  - mn_j * sum_i x_ri
// Quants are turned into exact fp16 values with the 1024-offset trick (0x6400 | q == 1024+q;
// a high nibble left in bits 4..7 reads as 1024+16q), multiplied against fp16 activations on
// v_mfma_f32_16x16x32_f16 (K = 32 = one sub-block), and the sub-block result is scaled by
// a_j in fp32. The offset and min terms are one rank-8 product per superblock, done on
// v_mfma_f32_16x16x4_f32 with the sub-block sums of the activations. Activations are
// converted to fp16 with a power-of-two scale per (row, superblock): exact for bf16 input.
#pragma once
#include "common.h"

namespace kq {


typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int FMT_Q4_K = 4;
constexpr int FMT_Q5_K = 5;
constexpr int FMT_Q6_K = 6;
constexpr int FMT_Q8_0 = 8;
constexpr int QK = 256;          // weights per superblock
constexpr int TILE_N = 16;       // columns per MFMA tile
constexpr int TILE_M = 16;       // rows per MFMA tile

// Activation workspace (ws) for one 16-row tile and S superblocks. Each (row, superblock) has its
// own power-of-two scale so that the fp16 operands are exact for any bf16 input.
struct XPrepView {
  u32x4* xop;     // [S][8][64] fp16 A operands (8 halves per lane)
  float* sxop;    // [S][2][64] negated sub-block sums, f32 MFMA A operand
  float* scale;   // [S][16] 2^e per (superblock, row): undoes the operand scaling
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline size_t xprep_tile_bytes(int64_t S) {
  return align256((size_t)S * 8 * 64 * 16) + align256((size_t)S * 2 * 64 * 4) +
         align256((size_t)S * 16 * 4);
}

__host__ __device__ inline XPrepView xprep_view(void* base, int64_t S) {
  XPrepView v;
  char* p = (char*)base;
  v.xop = (u32x4*)p;
  p += ((size_t)S * 8 * 64 * 16 + 255) & ~(size_t)255;
  v.sxop = (float*)p;
  p += ((size_t)S * 2 * 64 * 4 + 255) & ~(size_t)255;
  v.scale = (float*)p;
  return v;
}

// Slot e of a lane's 8 fp16 operand values holds k-offset kperm(e) within its 8-wide k range:
// 0, 2, 1, 3, 4, 6, 5, 7 -- the order in which the nibble/byte decoders below emit weights.
__host__ __device__ constexpr int kperm_c(int e) { return (e & 4) | ((e & 1) << 1) | ((e >> 1) & 1); }

// ---------------------------------------------------------------------------------------
// Activation conversion for one (16-row tile, superblock): lane (row = lane & 15,
// kq = lane >> 4) owns k = 32 j + 8 kq + kperm(0..7) of every sub-block j. `src` points at
// the tile's first row; rows >= rows_valid read as zero.
// ---------------------------------------------------------------------------------------
struct XOperands {
  u32x4 x[8];      // fp16 A operands of the 8 sub-blocks
  float sx0, sx1;  // negated sub-block sums (f32 MFMA A operand: row lane&15, k = lane>>4)
  float scale;     // 2^e of this lane's row
};

// Conversion of one lane's 64 bf16 values: chunk j (get(j)) holds k = 32 j + 8 kq .. + 7 of
// sub-block j in natural order (two bf16 per dword, low half first); put(j, v) receives the
// fp16 A operand of sub-block j. get is called twice per chunk (the row maximum, then the
// conversion), so a source in LDS needs no registers for the whole superblock.
template <class Get, class Put>
__device__ __forceinline__ void convert_chunks(Get&& get, Put&& put, int lane, float& sx0,
                                               float& sx1, float& scale) {
  const int kq = lane >> 4;
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u32x4 rj = get(j);
    const uint32_t w4[4] = {rj.x, rj.y, rj.z, rj.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mx = fmaxf(mx, __builtin_fabsf(__uint_as_float(w4[i] << 16)));
      mx = fmaxf(mx, __builtin_fabsf(__uint_as_float(w4[i] & 0xffff0000u)));
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  int e = 0;
  if (mx > 0.0f && mx <= 3.40282346638528859812e38f) {
    int E = (int)((__float_as_uint(mx) >> 23) & 0xff) - 127;
    if (E < -126) E = -126;
    e = E - 14;  // scaled maximum lands in [2^14, 2^15)
  }
  sx0 = 0.0f;
  sx1 = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u32x4 rj = get(j);
    const uint32_t w4[4] = {rj.x, rj.y, rj.z, rj.w};
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w4[i] << 16);
      f[2 * i + 1] = __uint_as_float(w4[i] & 0xffff0000u);
    }
    uint16_t h[8];
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      _Float16 hv = (_Float16)__builtin_ldexpf(f[kperm_c(t)], -e);
      h[t] = __builtin_bit_cast(uint16_t, hv);
      sum += (float)hv;
    }
    put(j, u32x4{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                 h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16)});
    // the full sub-block sum: the four kq lanes of the row added in a fixed order; lane kq
    // keeps sub-blocks kq and 4 + kq
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (j == kq) sx0 = -sum;
    if (j == 4 + kq) sx1 = -sum;
  }
  scale = __builtin_ldexpf(1.0f, e);
}

__device__ __forceinline__ void convert_words(const u32x4 (&raw)[8], int lane, XOperands& o) {
  convert_chunks([&](int j) { return raw[j]; }, [&](int j, u32x4 v) { o.x[j] = v; }, lane,
                 o.sx0, o.sx1, o.scale);
}

__device__ __forceinline__ void convert_superblock(const uint16_t* __restrict__ src,
                                                   int64_t row_stride, int rows_valid, int s,
                                                   int lane, XOperands& o) {
  const int r = lane & 15, kq = lane >> 4;
  const bool live = r < rows_valid;
  u32x4 raw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    raw[j] = live ? *(const u32x4*)(src + r * row_stride + (int64_t)s * QK + j * 32 + kq * 8)
                  : u32x4{0u, 0u, 0u, 0u};
  convert_words(raw, lane, o);
}

// Operand conversion of one 8-value word of a row, for producers that hold a row as 16-byte
// words (thread wt of the row holds values 8 wt .. 8 wt + 7, so the 32 words of superblock
// wt / 32 lie in one half wave and a sub-block's 4 words in one quad): the (row, superblock)
// power-of-two scale from the maximum over the 32 words, the fp16 values in kperm order and
// the negated sub-block sums, stored into the workspace of S superblocks per row. The same
// operands as convert_superblock. Every lane of the wave calls it (DPP); store == false lanes
// write nothing.
__device__ __forceinline__ void word_operand(const float (&y)[8], int wt, int64_t row,
                                             void* __restrict__ ws, size_t tile_bytes, int64_t S,
                                             bool store) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) mx = fmaxf(mx, __builtin_fabsf(y[i]));
  mx = fmaxf(mx, __uint_as_float(dpp_u32<DPP_QUAD_XOR1>(__float_as_uint(mx))));
  mx = fmaxf(mx, __uint_as_float(dpp_u32<DPP_QUAD_XOR2>(__float_as_uint(mx))));
  mx = fmaxf(mx, __uint_as_float(dpp_u32<DPP_HALF_MIRROR>(__float_as_uint(mx))));
  mx = fmaxf(mx, __uint_as_float(dpp_u32<DPP_MIRROR>(__float_as_uint(mx))));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  int e = 0;
  if (mx > 0.0f && mx <= 3.40282346638528859812e38f) {
    int E = (int)((__float_as_uint(mx) >> 23) & 0xff) - 127;
    if (E < -126) E = -126;
    e = E - 14;  // scaled maximum lands in [2^14, 2^15)
  }
  uint16_t h[8];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 hv = (_Float16)__builtin_ldexpf(y[kperm_c(i)], -e);
    h[i] = __builtin_bit_cast(uint16_t, hv);
    sum += (float)hv;
  }
  // sub-block sum over its four k-groups: (g0 + g1) + (g2 + g3)
  sum += __uint_as_float(dpp_u32<DPP_QUAD_XOR1>(__float_as_uint(sum)));
  sum += __uint_as_float(dpp_u32<DPP_QUAD_XOR2>(__float_as_uint(sum)));
  if (!store) return;
  const int sb = wt >> 5, j = (wt >> 2) & 7, kq = wt & 3;
  const int tile = (int)(row / TILE_M), r = (int)(row % TILE_M);
  XPrepView view = xprep_view((char*)ws + tile * tile_bytes, S);
  view.xop[((int64_t)sb * 8 + j) * 64 + r + 16 * kq] =
      u32x4{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
            h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16)};
  if (kq == 0) view.sxop[((int64_t)sb * 2 + (j >> 2)) * 64 + r + 16 * (j & 3)] = -sum;
  if ((wt & 31) == 0) view.scale[sb * 16 + r] = __builtin_ldexpf(1.0f, e);
}

// Store one superblock's operands into the workspace view.
__device__ __forceinline__ void store_operands(const XPrepView& v, int64_t s, int lane,
                                               const XOperands& o) {
#pragma unroll
  for (int j = 0; j < 8; ++j) v.xop[(s * 8 + j) * 64 + lane] = o.x[j];
  v.sxop[(s * 2 + 0) * 64 + lane] = o.sx0;
  v.sxop[(s * 2 + 1) * 64 + lane] = o.sx1;
  if ((lane >> 4) == 0) v.scale[s * 16 + (lane & 15)] = o.scale;
}

// ---------------------------------------------------------------------------------------
// Decoders: packed words -> fp16 MFMA B operands (slot order kperm).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(half8, v);
}

// (w & mask) | orv: written in plain C so that the compiler, which tracks the wait states
// between VALU writes and in-flight MFMA reads, emits and schedules the v_and_or_b32 itself.
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t orv) {
  return (w & mask) | orv;
}

// Q4_K group (two dwords = 8 bytes of one 32-byte nibble group): low nibbles -> sub-block 2g
// as 1024+q, high nibbles -> sub-block 2g+1 as 1024+16q. 10 VALU ops for 16 weights.
__device__ __forceinline__ void q4_group(uint32_t wa, uint32_t wb, uint32_t M, half8& lo,
                                         half8& hi) {
  const uint32_t wa8 = wa >> 8, wb8 = wb >> 8;
  lo = as_half8(and_or(wa, 0x000f000fu, M), and_or(wa8, 0x000f000fu, M),
                and_or(wb, 0x000f000fu, M), and_or(wb8, 0x000f000fu, M));
  hi = as_half8(and_or(wa, 0x00f000f0u, M), and_or(wa8, 0x00f000f0u, M),
                and_or(wb, 0x00f000f0u, M), and_or(wb8, 0x00f000f0u, M));
}

// Q8_0 sub-block (two dwords = 8 int8): 1024 + (q + 128), byte-permuted next to the 0x64
// exponent byte (v_perm_b32: result bytes (w.b0, 0x64, w.b2, 0x64) and (w.b1, .., w.b3, ..)).
__device__ __forceinline__ half8 q8_sub(uint32_t wa, uint32_t wb, uint32_t M8) {
  wa ^= 0x80808080u;
  wb ^= 0x80808080u;
  return as_half8(__builtin_amdgcn_perm(M8, wa, 0x04020400u), __builtin_amdgcn_perm(M8, wa, 0x04030401u),
                  __builtin_amdgcn_perm(M8, wb, 0x04020400u), __builtin_amdgcn_perm(M8, wb, 0x04030401u));
}

__device__ __forceinline__ float byte_f(uint32_t w, int i) {
  return (float)((w >> (8 * i)) & 0xffu);
}

// One 16-column x 256-weight tile. Returns the superblock's contribution in the C layout
// (column lane & 15, rows 4*(lane >> 4) + i), still in units of the operand scaling.
// xa: A operands of the 8 sub-blocks, sx0/sx1: negated sub-block sums (f32 MFMA A operand).
// Q5_K: the fifth bit of sub-block j's weights, placed on the 16-bit lanes of q4_group's four
// words (bytes (0, 2), (1, 3) of qa and of qb), at bit `at` (4: low nibbles, 8: high nibbles,
// which q4_group leaves at 16 q).
__device__ __forceinline__ void q5_bits(uint32_t qa, uint32_t qb, int j, int at, uint32_t (&e)[4]) {
  e[0] = ((qa >> j) & 0x00010001u) << at;
  e[1] = ((qa >> (8 + j)) & 0x00010001u) << at;
  e[2] = ((qb >> j) & 0x00010001u) << at;
  e[3] = ((qb >> (8 + j)) & 0x00010001u) << at;
}

__device__ __forceinline__ half8 or_half8(half8 v, const uint32_t (&e)[4]) {
  u32x4 w = __builtin_bit_cast(u32x4, v);
  w.x |= e[0];
  w.y |= e[1];
  w.z |= e[2];
  w.w |= e[3];
  return __builtin_bit_cast(half8, w);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Q6_K: the exact fp16 values q - 32 of one 32-weight run in kperm slot order, from its ql
// words (wa, wb: bytes l = 8 kq .. 8 kq + 7), the nibble shift (0 low, 4 high) and its qh words
// (ha, hb) with the run's bit pair at hs.
__device__ __forceinline__ half8 q6_run(uint32_t wa, uint32_t wb, uint32_t ha, uint32_t hb, int sh,
                                        int hs, uint32_t M) {
  const uint32_t w0 = and_or((wa >> sh) & 0x000f000fu, 0xffffffffu, ((ha >> hs) & 0x00030003u) << 4);
  const uint32_t w1 = and_or((wa >> (8 + sh)) & 0x000f000fu, 0xffffffffu,
                             ((ha >> (8 + hs)) & 0x00030003u) << 4);
  const uint32_t w2 = and_or((wb >> sh) & 0x000f000fu, 0xffffffffu, ((hb >> hs) & 0x00030003u) << 4);
  const uint32_t w3 = and_or((wb >> (8 + sh)) & 0x000f000fu, 0xffffffffu,
                             ((hb >> (8 + hs)) & 0x00030003u) << 4);
  // 0x6400 | q = 1024 + q exactly; minus 1056 gives q - 32 exactly
  const half2v off = {(_Float16)1056.0f, (_Float16)1056.0f};
  const half2v v0 = __builtin_bit_cast(half2v, w0 | M) - off;
  const half2v v1 = __builtin_bit_cast(half2v, w1 | M) - off;
  const half2v v2 = __builtin_bit_cast(half2v, w2 | M) - off;
  const half2v v3 = __builtin_bit_cast(half2v, w3 | M) - off;
  return as_half8(__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                  __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3));
}

__device__ __forceinline__ float sbyte_f(uint32_t w, int i) {
  return (float)(int8_t)((w >> (8 * i)) & 0xffu);
}

template <int FMT>
__device__ __forceinline__ floatx4 tile_superblock(const u32x4* qv, u32x4 meta, uint32_t dq,
                                                   const half8* xa, float sx0, float sx1, int kq,
                                                   uint32_t M) {
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  floatx4 acc = zero;
  float a[8];
  float beta_lo, beta_hi;  // beta for sub-blocks kq and kq + 4
  if constexpr (FMT == FMT_Q6_K) {
    // w = d sc_g (q - 32) with a scale per 16 weights: each 32-weight run is multiplied twice,
    // once with the B lanes of its first 16 weights (kq < 2) and once with the rest, each
    // product scaled by its own sc; q - 32 is exact in fp16, so no offset term is needed
    const float d = f16_to_f32((uint16_t)((threadIdx.x & 1) ? (dq >> 16) : (dq & 0xffff)));
    const uint32_t keep_lo = kq < 2 ? 0xffffffffu : 0u, keep_hi = ~keep_lo;
    const uint32_t sw[4] = {meta.x, meta.y, meta.z, meta.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = j >> 2, p = j & 3;
      const u32x4 ql = qv[n];
      const uint32_t wa = (p & 1) ? ql.z : ql.x, wb = (p & 1) ? ql.w : ql.y;
      const uint32_t ha = n ? qv[2].z : qv[2].x, hb = n ? qv[2].w : qv[2].y;
      const half8 b = q6_run(wa, wb, ha, hb, (p >> 1) * 4, 2 * p, M);
      const u32x4 bw = __builtin_bit_cast(u32x4, b);
      const half8 b_lo = __builtin_bit_cast(half8, bw & keep_lo);
      const half8 b_hi = __builtin_bit_cast(half8, bw & keep_hi);
      const int si = 8 * n + 2 * p;  // scales of weights l < 16 and l >= 16
      const float s_lo = d * sbyte_f(sw[si >> 2], si & 3);
      const float s_hi = d * sbyte_f(sw[(si + 1) >> 2], (si + 1) & 3);
      floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], b_lo, zero, 0, 0, 0);
      acc += s_lo * c;
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], b_hi, zero, 0, 0, 0);
      acc += s_hi * c;
    }
    return acc;
  } else if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    const float d = f16_to_f32((uint16_t)(meta.x & 0xffff));
    const float dmin = f16_to_f32((uint16_t)(meta.x >> 16));
    const uint32_t s0 = meta.y, s1 = meta.z, s2 = meta.w;
    const uint32_t sc03 = s0 & 0x3f3f3f3fu;
    const uint32_t m03 = s1 & 0x3f3f3f3fu;
    const uint32_t sc47 = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m47 = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = d * byte_f(sc03, i);
      a[4 + i] = d * byte_f(sc47, i);
    }
    const float m_lo = dmin * byte_f(m03, kq);
    const float m_hi = dmin * byte_f(m47, kq);
    // even sub-blocks carry the 1024 offset; odd ones read 1024 + 16 q, i.e. 64 after the 1/16
    const float off = (kq & 1) ? 64.0f : 1024.0f;
    beta_lo = __builtin_fmaf(off, d * byte_f(sc03, kq), m_lo);  // a[kq] without a select chain
    beta_hi = __builtin_fmaf(off, d * byte_f(sc47, kq), m_hi);
    const u32x4 q0 = qv[0], q1 = qv[1];
    half8 lo, hi;
    floatx4 c;
    // Q5_K: OR the fifth bits into the nibble lanes (bit 4 of 1024 + q, bit 8 of 1024 + 16 q)
    auto fifth = [&](int j, half8& l, half8& h) {
      if constexpr (FMT == FMT_Q5_K) {
        uint32_t e[4];
        q5_bits(qv[2].x, qv[2].y, j, 4, e);
        l = or_half8(l, e);
        q5_bits(qv[2].x, qv[2].y, j + 1, 8, e);
        h = or_half8(h, e);
      }
    };
    q4_group(q0.x, q0.y, M, lo, hi);
    fifth(0, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0], lo, zero, 0, 0, 0);
    acc += a[0] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1], hi, zero, 0, 0, 0);
    acc += (a[1] * 0.0625f) * c;
    q4_group(q0.z, q0.w, M, lo, hi);
    fifth(2, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2], lo, zero, 0, 0, 0);
    acc += a[2] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[3], hi, zero, 0, 0, 0);
    acc += (a[3] * 0.0625f) * c;
    q4_group(q1.x, q1.y, M, lo, hi);
    fifth(4, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[4], lo, zero, 0, 0, 0);
    acc += a[4] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[5], hi, zero, 0, 0, 0);
    acc += (a[5] * 0.0625f) * c;
    q4_group(q1.z, q1.w, M, lo, hi);
    fifth(6, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[6], lo, zero, 0, 0, 0);
    acc += a[6] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[7], hi, zero, 0, 0, 0);
    acc += (a[7] * 0.0625f) * c;
  } else {
    const uint32_t dw[4] = {meta.x, meta.y, meta.z, meta.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = f16_to_f32((uint16_t)(dw[i] & 0xffff));
      a[2 * i + 1] = f16_to_f32((uint16_t)(dw[i] >> 16));
    }
    // a[kq], a[4 + kq] read straight from the packed scales (no select chain on kq)
    beta_lo = 1152.0f * f16_to_f32((uint16_t)(((kq & 1) ? (dw[kq >> 1] >> 16) : dw[kq >> 1]) & 0xffff));
    beta_hi = 1152.0f * f16_to_f32((uint16_t)(((kq & 1) ? (dw[2 + (kq >> 1)] >> 16) : dw[2 + (kq >> 1)]) & 0xffff));
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const u32x4 q = qv[jp];
      floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * jp], q8_sub(q.x, q.y, M), zero, 0,
                                                          0, 0);
      acc += a[2 * jp] * c;
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * jp + 1], q8_sub(q.z, q.w, M), zero, 0, 0, 0);
      acc += a[2 * jp + 1] * c;
    }
  }
  // offset/min term: acc += (-Sx) * beta over the 8 sub-blocks (k = lane >> 4 in each half)
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx0, beta_lo, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx1, beta_hi, acc, 0, 0, 0);
  return acc;
}

// Repacked weight layout per 16-column tile and superblock ("tile-superblock", ts):
//   Q4_K  quant 2 KiB: [half][lane][16 B] nibbles (bytes 0-7 of group 2 half + 8 kq.., 8-15
//         of group 2 half + 1); meta [col][16 B] = d, dmin, 12 scale bytes.
//   Q5_K  quant 2.5 KiB: the Q4_K nibbles, then [lane][8 B] = qh[8 kq ..]; meta as Q4_K.
//   Q6_K  quant 3 KiB: [3][lane][16 B]: ql of half 0 (bytes 0-7: ql[8 kq ..], 8-15:
//         ql[32 + 8 kq ..]), ql of half 1 (+64), qh (bytes 0-7: qh[8 kq ..], 8-15:
//         qh[32 + 8 kq ..]); meta [col][16 B] = the 16 int8 scales, then after all
//         tile-superblocks' scales one fp16 d per (ts, col).
//   Q8_0  quant 4 KiB: [4][lane][16 B] int8; meta [col][16 B] = the 8 fp16 scales.
template <int FMT>
struct QLayout {
  // u32x4 per lane per superblock (Q5_K's third holds the 8 qh bytes in .x, .y)
  static constexpr int kQuantVecs = FMT == FMT_Q4_K ? 2 : FMT == FMT_Q8_0 ? 4 : 3;
  static constexpr int kTsBytes = FMT == FMT_Q4_K ? 2048 : FMT == FMT_Q5_K ? 2560
                                  : FMT == FMT_Q6_K ? 3072 : 4096;  // quant bytes per ts
};

// Per-wave operands of one superblock for NTILE column tiles.
template <int FMT, int NTILE>
struct SbOperands {
  u32x4 x[8];
  float sx0, sx1;
  floatx4 scale;  // 2^e of rows 4*(lane>>4) + 0..3
  u32x4 q[NTILE][QLayout<FMT>::kQuantVecs];
  u32x4 m[NTILE];
  uint32_t dq[NTILE];  // Q6_K: the word holding this lane's column d (fp16)
};

__device__ __forceinline__ u32x4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float bload1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload1u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2 bload2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// Buffer resources and per-lane byte offsets of the streams one wave reads.
struct GemvStreams {
  __amdgpu_buffer_rsrc_t quant, meta, xop, sxop, scale;
  __amdgpu_buffer_rsrc_t dmeta;  // Q6_K: the fp16 d per (tile-superblock, column)
  uint32_t v_quant, v_meta, v_xop, v_sx, v_scale;  // per-lane byte offsets
  uint32_t v_dq;  // Q6_K: this lane's column's d word
  uint32_t v_scale_g[4];  // row-gathered streams: offsets of the scales of rows 4*kq + i
};

// The activation operands of superblock s from the workspace (GATHER: rows gathered per lane).
template <int FMT, int NTILE, bool GATHER = false>
__device__ __forceinline__ void load_sb_x(SbOperands<FMT, NTILE>& o, const GemvStreams& st,
                                          int s) {
#pragma unroll
  for (int j = 0; j < 8; ++j) o.x[j] = bload4(st.xop, st.v_xop, (uint32_t)((s * 8 + j) * 64 * 16));
  o.sx0 = bload1(st.sxop, st.v_sx, (uint32_t)((s * 2 + 0) * 64 * 4));
  o.sx1 = bload1(st.sxop, st.v_sx, (uint32_t)((s * 2 + 1) * 64 * 4));
  if constexpr (GATHER) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o.scale[i] = bload1(st.scale, st.v_scale_g[i], (uint32_t)(s * 16 * 4));
  } else {
    o.scale = __builtin_bit_cast(floatx4, bload4(st.scale, st.v_scale, (uint32_t)(s * 16 * 4)));
  }
}

// The weights of superblock s for tiles tile0 + t * tstride (t < NTILE).
template <int FMT, int NTILE>
__device__ __forceinline__ void load_sb_w(u32x4 (&q)[NTILE][QLayout<FMT>::kQuantVecs],
                                          u32x4 (&m)[NTILE], const GemvStreams& st, int s, int S,
                                          int tile0, int tstride) {
  constexpr int QV = QLayout<FMT>::kQuantVecs;
  constexpr uint32_t TB = QLayout<FMT>::kTsBytes;
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const uint32_t ts = (uint32_t)((tile0 + t * tstride) * S + s);
    if constexpr (FMT == FMT_Q5_K) {
      q[t][0] = bload4(st.quant, st.v_quant, ts * TB);
      q[t][1] = bload4(st.quant, st.v_quant, ts * TB + 1024);
      const u32x2 h = bload2(st.quant, st.v_quant >> 1, ts * TB + 2048);
      q[t][2] = u32x4{h.x, h.y, 0u, 0u};
    } else {
#pragma unroll
      for (int i = 0; i < QV; ++i) q[t][i] = bload4(st.quant, st.v_quant, ts * TB + i * 1024);
    }
    m[t] = bload4(st.meta, st.v_meta, ts * 16 * 16);
  }
}

// Q6_K: the word holding the fp16 d of this lane's column, for tiles tile0 + t * tstride.
template <int NTILE>
__device__ __forceinline__ void load_sb_d(uint32_t (&dq)[NTILE], const GemvStreams& st, int s,
                                          int S, int tile0, int tstride) {
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const uint32_t ts = (uint32_t)((tile0 + t * tstride) * S + s);
    dq[t] = bload1u(st.dmeta, st.v_dq, ts * 16 * 2);
  }
}

// Load the weights of superblock s for tiles tile0 + t * tstride (t < NTILE) and, when
// WITH_X, its activation operands from the workspace.
template <int FMT, int NTILE, bool WITH_X = true, bool GATHER = false>
__device__ __forceinline__ void load_sb(SbOperands<FMT, NTILE>& o, const GemvStreams& st, int s,
                                        int S, int tile0, int tstride = 1) {
  if constexpr (WITH_X) load_sb_x<FMT, NTILE, GATHER>(o, st, s);
  load_sb_w<FMT, NTILE>(o.q, o.m, st, s, S, tile0, tstride);
  if constexpr (FMT == FMT_Q6_K) load_sb_d<NTILE>(o.dq, st, s, S, tile0, tstride);
}

// Multiply one superblock's operands into acc.
template <int FMT, int NTILE>
__device__ __forceinline__ void gemv_superblock(const SbOperands<FMT, NTILE>& o, floatx4* acc,
                                                int kq, uint32_t Mv) {
  half8 xa[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xa[j] = __builtin_bit_cast(half8, o.x[j]);
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    floatx4 sb = tile_superblock<FMT>(o.q[t], o.m[t], o.dq[t], xa, o.sx0, o.sx1, kq, Mv);
    acc[t] += sb * o.scale;
  }
}


// Streams of a k-quant weight (`tiles` column tiles x S superblocks) and of the activation
// workspace. Lanes whose row is >= rows read activations at an out-of-range offset: the buffer
// unit returns zeros without touching memory.
template <int FMT>
__device__ __forceinline__ GemvStreams make_streams(const void* quant, const void* meta,
                                                    const void* ws, int tiles, int S, int lane,
                                                    int rows) {
  constexpr int QV = QLayout<FMT>::kQuantVecs;
  const int kq = lane >> 4, r = lane & 15;
  XPrepView xv = xprep_view((void*)ws, S);
  GemvStreams st;
  // byte ranges in 64 bits, clamped to what one buffer resource holds (the entry points refuse
  // weights whose offsets would not fit 32 bits)
  const int64_t qn = (int64_t)tiles * S * QLayout<FMT>::kTsBytes, mn = (int64_t)tiles * S * 16 * 16;
  st.quant = __builtin_amdgcn_make_buffer_rsrc((void*)quant, 0,
                                               (int)(uint32_t)(qn < 0xFFFFFFFFll ? qn : 0xFFFFFFFFll),
                                               0x00020000);
  st.meta = __builtin_amdgcn_make_buffer_rsrc((void*)meta, 0,
                                              (int)(uint32_t)(mn < 0xFFFFFFFFll ? mn : 0xFFFFFFFFll),
                                              0x00020000);
  st.xop = __builtin_amdgcn_make_buffer_rsrc((void*)xv.xop, 0, S * 8 * 64 * 16, 0x00020000);
  st.sxop = __builtin_amdgcn_make_buffer_rsrc((void*)xv.sxop, 0, S * 2 * 64 * 4, 0x00020000);
  st.scale = __builtin_amdgcn_make_buffer_rsrc((void*)xv.scale, 0, S * 16 * 4, 0x00020000);
  // Q6_K: the d values follow the scales (one fp16 per (tile-superblock, column))
  st.dmeta = __builtin_amdgcn_make_buffer_rsrc((char*)meta + mn, 0,
                                               (int)(uint32_t)(mn / 8 < 0xFFFFFFFFll ? mn / 8 : 0xFFFFFFFFll),
                                               0x00020000);
  st.v_dq = (uint32_t)((r & ~1) * 2);
  st.v_quant = lane * 16;
  st.v_meta = r * 16;
  st.v_xop = r < rows ? lane * 16 : 0x80000000u;
  st.v_sx = lane * 4;
  st.v_scale = kq * 16;
  return st;
}

// The decoders' 0x6400 exponent pattern, held in a vector register: a VOP3 v_and_or_b32 may
// read one scalar operand, the mask. The identity DPP move makes the value opaque to constant
// folding while remaining an ordinary instruction for the compiler's hazard tracking.
template <int FMT>
__device__ __forceinline__ uint32_t decode_magic() {
  constexpr int M = FMT == FMT_Q8_0 ? 0x64646464 : 0x64006400;
  return (uint32_t)__builtin_amdgcn_update_dpp(0, M, 0xE4, 0xF, 0xF, false);
}

// Wave w of NW walks superblocks s = w, w + NW, ... of the tiles tile0 + t * tstride, with the
// next superblock's operands in flight while the current one is multiplied.
template <int FMT, int NTILE, int NW, bool GATHER = false>
__device__ __forceinline__ void gemv_loop(const GemvStreams& st, int w, int S, int tile0,
                                          int tstride, int kq, uint32_t Mv, floatx4* acc) {
  if (w >= S) return;
  SbOperands<FMT, NTILE> bufA, bufB;
  load_sb<FMT, NTILE, true, GATHER>(bufA, st, w, S, tile0, tstride);
  for (int s = w;;) {
    if (s + NW < S) load_sb<FMT, NTILE, true, GATHER>(bufB, st, s + NW, S, tile0, tstride);
    gemv_superblock<FMT, NTILE>(bufA, acc, kq, Mv);
    s += NW;
    if (s >= S) break;
    if (s + NW < S) load_sb<FMT, NTILE, true, GATHER>(bufA, st, s + NW, S, tile0, tstride);
    gemv_superblock<FMT, NTILE>(bufB, acc, kq, Mv);
    s += NW;
    if (s >= S) break;
  }
}

// Wave w of NW walks SC superblocks (w, w + NW, ...) of the tiles tile0 + t * tstride with the
// weights of the next two in flight while one is multiplied (three weight buffers), and the
// activation operands, which come from L2, loaded one superblock at a time after the previous
// superblock's products have read them. Unrolled (SC a compile-time count) so that no load
// sits under a branch, which would make the compiler wait for every load in flight at the
// join. VW > 1: step i adds into acc[(i % VW) * NTILE + t], the sums VW waves would keep, so
// one wave can stand for VW of them with their bits.
template <int FMT, int NTILE, int SC, bool GATHER = false, int NW = 1, int VW = 1>
__device__ __forceinline__ void gemv_loop_deep(const GemvStreams& st, int w, int tile0,
                                               int tstride, int kq, uint32_t Mv, floatx4* acc) {
  SbOperands<FMT, NTILE> x;  // the activation part
  u32x4 q[3][NTILE][QLayout<FMT>::kQuantVecs];
  u32x4 m[3][NTILE];
  uint32_t dq[3][NTILE];
  // step i multiplies superblock w + NW i of the SC * NW
  auto load_w = [&](int b, int i) {
    load_sb_w<FMT, NTILE>(q[b], m[b], st, w + NW * i, SC * NW, tile0, tstride);
    if constexpr (FMT == FMT_Q6_K) load_sb_d<NTILE>(dq[b], st, w + NW * i, SC * NW, tile0, tstride);
  };
  load_w(0, 0);
  load_sb_x<FMT, NTILE, GATHER>(x, st, w);
  if constexpr (SC > 1) load_w(1, 1);
  if constexpr (SC > 2) load_w(2, 2);
#pragma unroll
  for (int s = 0; s < SC; ++s) {
    const int b = s % 3;
    half8 xa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xa[j] = __builtin_bit_cast(half8, x.x[j]);
#pragma unroll
    for (int t = 0; t < NTILE; ++t) {
      floatx4 sb = tile_superblock<FMT>(q[b][t], m[b][t], dq[b][t], xa, x.sx0, x.sx1, kq, Mv);
      acc[(s % VW) * NTILE + t] += sb * x.scale;
    }
    if (s + 1 < SC) load_sb_x<FMT, NTILE, GATHER>(x, st, w + NW * (s + 1));
    if (s + 3 < SC) load_w(b, s + 3);
  }
}

// Variant for bf16 activations read straight from [M, K] (no operand workspace): the raw words
// of superblock s are loaded with the weights and converted at multiply time (the same
// per-(row, superblock) power-of-two conversion as the workspace path, so results match it).
struct RawX {
  __amdgpu_buffer_rsrc_t act;
  uint32_t v_act;  // byte offset of this lane's row + 8 kq, or out of range for rows >= M
};

__device__ __forceinline__ RawX make_raw_x(const void* act, int M, int K, int lane) {
  RawX rx;
  const int r = lane & 15, kq = lane >> 4;
  rx.act = __builtin_amdgcn_make_buffer_rsrc((void*)act, 0, M * K * 2, 0x00020000);
  rx.v_act = r < M ? (uint32_t)((r * K + kq * 8) * 2) : 0x80000000u;
  return rx;
}

template <int FMT, int NTILE>
__device__ __forceinline__ void load_sb_raw(SbOperands<FMT, NTILE>& o, const GemvStreams& st,
                                            const RawX& rx, int s, int S, int tile0,
                                            int tstride) {
#pragma unroll
  for (int j = 0; j < 8; ++j) o.x[j] = bload4(rx.act, rx.v_act, (uint32_t)((s * QK + j * 32) * 2));
  load_sb<FMT, NTILE, false>(o, st, s, S, tile0, tstride);
}

template <int FMT, int NTILE>
__device__ __forceinline__ void gemv_superblock_raw(SbOperands<FMT, NTILE>& o, floatx4* acc,
                                                    int lane, uint32_t Mv) {
  XOperands xo;
  convert_words(o.x, lane, xo);
  const int kq = lane >> 4;
#pragma unroll
  for (int j = 0; j < 8; ++j) o.x[j] = xo.x[j];
  o.sx0 = xo.sx0;
  o.sx1 = xo.sx1;
  // per-row scales of rows 4 kq .. 4 kq + 3 live in lanes 4 kq + i (kq = 0 row group)
#pragma unroll
  for (int i = 0; i < 4; ++i) o.scale[i] = __shfl(xo.scale, 4 * kq + i, 64);
  gemv_superblock<FMT, NTILE>(o, acc, kq, Mv);
}

template <int FMT, int NTILE, int NW>
__device__ __forceinline__ void gemv_loop_raw(const GemvStreams& st, const RawX& rx, int w, int S,
                                              int tile0, int tstride, int lane, uint32_t Mv,
                                              floatx4* acc) {
  if (w >= S) return;
  SbOperands<FMT, NTILE> bufA, bufB;
  load_sb_raw<FMT, NTILE>(bufA, st, rx, w, S, tile0, tstride);
  for (int s = w;;) {
    if (s + NW < S) load_sb_raw<FMT, NTILE>(bufB, st, rx, s + NW, S, tile0, tstride);
    gemv_superblock_raw<FMT, NTILE>(bufA, acc, lane, Mv);
    s += NW;
    if (s >= S) break;
    if (s + NW < S) load_sb_raw<FMT, NTILE>(bufA, st, rx, s + NW, S, tile0, tstride);
    gemv_superblock_raw<FMT, NTILE>(bufB, acc, lane, Mv);
    s += NW;
    if (s >= S) break;
  }
}

// Sum the NW waves' accumulators in a fixed order; threads < NTILE*64 get tile t = idx >> 6,
// lane l = idx & 63 (C layout: column l & 15, rows 4*(l >> 4) + i).
template <int NTILE, int NW>
__device__ __forceinline__ void combine_waves(floatx4 (*part)[NTILE][64], const floatx4* acc,
                                              int w, int lane) {
#pragma unroll
  for (int t = 0; t < NTILE; ++t) part[w][t][lane] = acc[t];
  __syncthreads();
}

}  // namespace kq
