// GGUF Q4_K / Q8_0 dequant-GEMV for short verify blocks (M <= 16 rows per pass) on gfx950.
//
// Weights stay packed in HBM. A one-time repack (snowllm_gemm_kquant_shuffle_b) moves the
// GGUF bytes into MFMA lane order: a 16-column tile of one 256-weight superblock is a single
// contiguous 2 KiB run of nibbles (Q4_K) or 4 KiB of int8 (Q8_0), read with 16-byte loads
// that are fully coalesced across the wave, plus 16 bytes of block header per column.
//
// Arithmetic (per 32-weight sub-block j, column n, row r):
//   y[r,n] = sum_j  a_j * sum_i q_i x_ri  - mn_j * sum_i x_ri
// Quants are turned into exact fp16 values with the 1024-offset trick (0x6400 | q == 1024+q;
// a high nibble left in bits 4..7 reads as 1024+16q), multiplied against fp16 activations on
// v_mfma_f32_16x16x32_f16 (K = 32 = one sub-block), and the sub-block result is scaled by
// a_j in fp32. The offset and min terms are one rank-8 product per superblock, done on
// v_mfma_f32_16x16x4_f32 with the sub-block sums of the activations. Activations are
// converted to fp16 once per call with a per-row power-of-two scale (exact for bf16 input).
#include "common.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int FMT_Q4_K = 4;
constexpr int FMT_Q8_0 = 8;
constexpr int QK = 256;          // weights per superblock
constexpr int TILE_N = 16;       // columns per MFMA tile
constexpr int TILE_M = 16;       // rows per MFMA tile

// Activation workspace for one 16-row tile and S superblocks. Each (row, superblock) has its
// own power-of-two scale so that the fp16 operands are exact for any bf16 input.
struct XPrepView {
  u32x4* xop;     // [S][8][64] fp16 A operands (8 halves per lane)
  float* sxop;    // [S][2][64] negated sub-block sums, f32 MFMA A operand
  float* scale;   // [S][16] 2^e per (superblock, row): undoes the operand scaling
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

inline size_t xprep_tile_bytes(int64_t S) {
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
// Activation prep: bf16 [rows, K] -> fp16 MFMA operands. One wave per (row tile, superblock);
// lane (row = lane & 15, kq = lane >> 4) owns k = 32 j + 8 kq + 0..7 of every sub-block j.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) xprep_kernel(const uint16_t* __restrict__ a, int64_t M,
                                                   int64_t K, void* ws, size_t tile_bytes) {
  const int s = blockIdx.x, tile = blockIdx.y;
  const int lane = threadIdx.x, r = lane & 15, kq = lane >> 4;
  const int64_t S = K / QK;
  XPrepView v = xprep_view((char*)ws + tile * tile_bytes, S);
  const int64_t row = (int64_t)tile * TILE_M + r;
  const bool live = row < M;
  // raw bf16 (8 sub-blocks x 8 values)
  u32x4 raw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    raw[j] = live ? *(const u32x4*)(a + row * K + (int64_t)s * QK + j * 32 + kq * 8)
                  : u32x4{0u, 0u, 0u, 0u};
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
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
  float part[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
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
    part[j] = sum;
    u32x4 o;
    o.x = h[0] | ((uint32_t)h[1] << 16);
    o.y = h[2] | ((uint32_t)h[3] << 16);
    o.z = h[4] | ((uint32_t)h[5] << 16);
    o.w = h[6] | ((uint32_t)h[7] << 16);
    v.xop[((int64_t)s * 8 + j) * 64 + lane] = o;
  }
  // full sub-block sums: add the four kq lanes of the row (fixed order)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    part[j] += __shfl_xor(part[j], 16, 64);
    part[j] += __shfl_xor(part[j], 32, 64);
  }
  // f32 MFMA A layout: lane -> (row lane & 15, k = lane >> 4): half hh holds sub-block 4 hh + kq
  v.sxop[((int64_t)s * 2 + 0) * 64 + lane] = -part[kq];
  v.sxop[((int64_t)s * 2 + 1) * 64 + lane] = -part[4 + kq];
  if (kq == 0) v.scale[(int64_t)s * 16 + r] = __builtin_ldexpf(1.0f, e);
}

// ---------------------------------------------------------------------------------------
// Decoders: packed words -> fp16 MFMA B operands (slot order kperm).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(half8, v);
}

// Q4_K group (two dwords = 8 bytes of one 32-byte nibble group): low nibbles -> sub-block 2g
// as 1024+q, high nibbles -> sub-block 2g+1 as 1024+16q.
__device__ __forceinline__ void q4_group(uint32_t wa, uint32_t wb, half8& lo, half8& hi) {
  const uint32_t M = 0x64006400u;
  uint32_t wa8 = wa >> 8, wb8 = wb >> 8;
  lo = as_half8((wa & 0x000f000fu) | M, (wa8 & 0x000f000fu) | M, (wb & 0x000f000fu) | M,
                (wb8 & 0x000f000fu) | M);
  hi = as_half8((wa & 0x00f000f0u) | M, (wa8 & 0x00f000f0u) | M, (wb & 0x00f000f0u) | M,
                (wb8 & 0x00f000f0u) | M);
}

// Q8_0 sub-block (two dwords = 8 int8): 1024 + (q + 128).
__device__ __forceinline__ half8 q8_sub(uint32_t wa, uint32_t wb) {
  const uint32_t M = 0x64006400u;
  wa ^= 0x80808080u;
  wb ^= 0x80808080u;
  return as_half8((wa & 0x00ff00ffu) | M, ((wa >> 8) & 0x00ff00ffu) | M, (wb & 0x00ff00ffu) | M,
                  ((wb >> 8) & 0x00ff00ffu) | M);
}

__device__ __forceinline__ float byte_f(uint32_t w, int i) {
  return (float)((w >> (8 * i)) & 0xffu);
}

// One 16-column x 256-weight tile. Returns the superblock's contribution in the C layout
// (column lane & 15, rows 4*(lane >> 4) + i), still in units of the operand scaling.
// xa: A operands of the 8 sub-blocks, sx0/sx1: negated sub-block sums (f32 MFMA A operand).
template <int FMT>
__device__ __forceinline__ floatx4 tile_superblock(const u32x4* qv, u32x4 meta, const half8* xa,
                                                   float sx0, float sx1, int kq) {
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  floatx4 acc = zero;
  float a[8];
  float beta_lo, beta_hi;  // beta for sub-blocks kq and kq + 4
  if constexpr (FMT == FMT_Q4_K) {
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
    beta_lo = __builtin_fmaf(off, a[kq], m_lo);
    beta_hi = __builtin_fmaf(off, a[4 + kq], m_hi);
    const u32x4 q0 = qv[0], q1 = qv[1];
    half8 lo, hi;
    floatx4 c;
    q4_group(q0.x, q0.y, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0], lo, zero, 0, 0, 0);
    acc += a[0] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1], hi, zero, 0, 0, 0);
    acc += (a[1] * 0.0625f) * c;
    q4_group(q0.z, q0.w, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2], lo, zero, 0, 0, 0);
    acc += a[2] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[3], hi, zero, 0, 0, 0);
    acc += (a[3] * 0.0625f) * c;
    q4_group(q1.x, q1.y, lo, hi);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[4], lo, zero, 0, 0, 0);
    acc += a[4] * c;
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[5], hi, zero, 0, 0, 0);
    acc += (a[5] * 0.0625f) * c;
    q4_group(q1.z, q1.w, lo, hi);
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
    beta_lo = 1152.0f * a[kq];
    beta_hi = 1152.0f * a[4 + kq];
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const u32x4 q = qv[jp];
      floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * jp], q8_sub(q.x, q.y), zero, 0,
                                                          0, 0);
      acc += a[2 * jp] * c;
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * jp + 1], q8_sub(q.z, q.w), zero, 0, 0, 0);
      acc += a[2 * jp + 1] * c;
    }
  }
  // offset/min term: acc += (-Sx) * beta over the 8 sub-blocks (k = lane >> 4 in each half)
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx0, beta_lo, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx1, beta_hi, acc, 0, 0, 0);
  return acc;
}

template <int FMT>
struct QLayout {
  static constexpr int kQuantVecs = FMT == FMT_Q4_K ? 2 : 4;  // u32x4 per lane per superblock
};

// Per-wave operands of one superblock for NTILE column tiles.
template <int FMT, int NTILE>
struct SbOperands {
  u32x4 x[8];
  float sx0, sx1;
  floatx4 scale;
  u32x4 q[NTILE][QLayout<FMT>::kQuantVecs];
  u32x4 m[NTILE];
};

template <int FMT, int NTILE>
__device__ __forceinline__ void load_sb(SbOperands<FMT, NTILE>& o, const XPrepView& xv,
                                        const u32x4* __restrict__ quant,
                                        const u32x4* __restrict__ meta, int s, int S, int tile0,
                                        int tiles, int lane, bool live) {
  constexpr int QV = QLayout<FMT>::kQuantVecs;
  const int r = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    o.x[j] = live ? xv.xop[((int64_t)s * 8 + j) * 64 + lane] : u32x4{0u, 0u, 0u, 0u};
  o.sx0 = xv.sxop[((int64_t)s * 2 + 0) * 64 + lane];
  o.sx1 = xv.sxop[((int64_t)s * 2 + 1) * 64 + lane];
  o.scale = *(const floatx4*)(xv.scale + (int64_t)s * 16 + 4 * kq);
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const int tile = tile0 + t < tiles ? tile0 + t : tiles - 1;
    const int64_t ts = (int64_t)tile * S + s;
#pragma unroll
    for (int i = 0; i < QV; ++i) o.q[t][i] = quant[(ts * QV + i) * 64 + lane];
    o.m[t] = meta[ts * 16 + r];
  }
}

// NW waves split the superblocks of NTILE column tiles (wave w takes s = w, w + NW, ...) with
// the next superblock's operands in flight while the current one is multiplied; the waves'
// partial sums meet in LDS and are added in a fixed order.
template <int FMT, int NTILE, int NW>
__global__ void __launch_bounds__(NW * 64) kquant_gemv(const u32x4* __restrict__ quant,
                                                       const u32x4* __restrict__ meta,
                                                       const void* __restrict__ ws,
                                                       void* __restrict__ c, int M, int N, int S,
                                                       int c_bf16) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kq = lane >> 4, r = lane & 15;
  const int tiles = N / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  XPrepView xv = xprep_view((void*)ws, S);
  const bool live = r < M;
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (w < S) {
    SbOperands<FMT, NTILE> cur, nxt;
    load_sb<FMT, NTILE>(cur, xv, quant, meta, w, S, tile0, tiles, lane, live);
    for (int s = w; s < S; s += NW) {
      const bool more = s + NW < S;
      if (more) load_sb<FMT, NTILE>(nxt, xv, quant, meta, s + NW, S, tile0, tiles, lane, live);
      half8 xa[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) xa[j] = __builtin_bit_cast(half8, cur.x[j]);
#pragma unroll
      for (int t = 0; t < NTILE; ++t) {
        floatx4 sb = tile_superblock<FMT>(cur.q[t], cur.m[t], xa, cur.sx0, cur.sx1, kq);
        acc[t] += sb * cur.scale;
      }
      if (more) cur = nxt;
    }
  }
#pragma unroll
  for (int t = 0; t < NTILE; ++t) part[w][t][lane] = acc[t];
  __syncthreads();
  // combine waves in a fixed order and write rows < M
  for (int idx = threadIdx.x; idx < NTILE * 64; idx += NW * 64) {
    const int t = idx >> 6, l = idx & 63;
    const int tile = tile0 + t;
    if (tile >= tiles) continue;
    floatx4 v = part[0][t][l];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) v += part[ww][t][l];
    const int n = tile * TILE_N + (l & 15);
    const int rb = 4 * (l >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rb + i;
      if (row >= M) break;
      if (c_bf16) ((uint16_t*)c)[(int64_t)row * N + n] = f32_to_bf16(v[i]);
      else ((float*)c)[(int64_t)row * N + n] = v[i];
    }
  }
}

// ---------------------------------------------------------------------------------------
// Repack GGUF blocks into (quant, meta).
// ---------------------------------------------------------------------------------------
__global__ void shuffle_q4k(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const uint8_t* blk = gguf + (n * S + s) * 144;
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  uint8_t* mo = meta + (ts * 16 + col) * 16;
  for (int i = 0; i < 16; ++i) mo[i] = blk[i];
  const uint8_t* qs = blk + 16;
  for (int h = 0; h < 2; ++h)
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = col + 16 * kq;
      uint8_t* qo = quant + ((ts * 2 + h) * 64 + lane) * 16;
      for (int i = 0; i < 8; ++i) {
        qo[i] = qs[64 * h + 8 * kq + i];
        qo[8 + i] = qs[64 * h + 32 + 8 * kq + i];
      }
    }
}

__global__ void shuffle_q80(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  for (int j = 0; j < 8; ++j) {
    const uint8_t* blk = gguf + ((n * S + s) * 8 + j) * 34;
    uint8_t* mo = meta + (ts * 16 + col) * 16 + 2 * j;
    mo[0] = blk[0];
    mo[1] = blk[1];
    const int jp = j >> 1, half = j & 1;
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = col + 16 * kq;
      uint8_t* qo = quant + ((ts * 4 + jp) * 64 + lane) * 16 + 8 * half;
      for (int i = 0; i < 8; ++i) qo[i] = blk[2 + 8 * kq + i];
    }
  }
}

bool fmt_ok(int fmt) { return fmt == FMT_Q4_K || fmt == FMT_Q8_0; }

template <int FMT, int NTILE, int NW>
int launch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N, int S,
                int c_bf16, hipStream_t s) {
  const int tiles = N / TILE_N;
  const int grid = (tiles + NTILE - 1) / NTILE;
  hipLaunchKernelGGL((kquant_gemv<FMT, NTILE, NW>), dim3(grid), dim3(NW * 64), 0, s,
                     (const u32x4*)quant, (const u32x4*)meta, ws, c, M, N, S, c_bf16);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

int g_gemv_variant = 0;  // 0 = automatic; see snowverify_gemv_variant

template <int FMT>
int dispatch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N,
                  int S, int c_bf16, hipStream_t s) {
  switch (g_gemv_variant) {
    case 1: return launch_gemv<FMT, 1, 4>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 2: return launch_gemv<FMT, 2, 4>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 3: return launch_gemv<FMT, 4, 4>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 4: return launch_gemv<FMT, 1, 8>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 5: return launch_gemv<FMT, 2, 8>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 6: return launch_gemv<FMT, 1, 16>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 7: return launch_gemv<FMT, 2, 16>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 8: return launch_gemv<FMT, 4, 8>(quant, meta, ws, c, M, N, S, c_bf16, s);
    default: break;
  }
  const int tiles = N / TILE_N;
  if (S >= 16) {
    if (tiles >= 2 * 256) return launch_gemv<FMT, 2, 8>(quant, meta, ws, c, M, N, S, c_bf16, s);
    return launch_gemv<FMT, 1, 8>(quant, meta, ws, c, M, N, S, c_bf16, s);
  }
  if (tiles >= 2 * 256) return launch_gemv<FMT, 2, 4>(quant, meta, ws, c, M, N, S, c_bf16, s);
  return launch_gemv<FMT, 1, 4>(quant, meta, ws, c, M, N, S, c_bf16, s);
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

SV_API int64_t snowllm_kquant_gguf_bytes(int fmt, int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  if (fmt == FMT_Q4_K) return K % 256 ? -1 : N * (K / 256) * 144;
  if (fmt == FMT_Q8_0) return K % 32 ? -1 : N * (K / 32) * 34;
  return -1;
}

SV_API int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  return (fmt == FMT_Q4_K ? N * K / 2 : N * K) + 4;
}

SV_API int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  return N * (K / 256) * 16;
}

SV_API int snowllm_kquant_supported(int fmt) { return fmt_ok(fmt) ? 1 : 0; }

// Extension (tuning knob, no counterpart in the reference): force a GEMV tile shape
// (0 = automatic, 1..8 = fixed (tiles per workgroup, waves) pairs). Process-global.
SV_API void snowverify_gemv_variant(int v) { g_gemv_variant = v; }

SV_API int snowllm_gemm_kquant_shuffle_b(int fmt, const uint8_t* gguf, uint8_t* quant,
                                         uint8_t* meta, int64_t N, int64_t K, void* stream) {
  if (!fmt_ok(fmt) || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  const int64_t S = K / 256;
  const int64_t total = N * S;
  const int nt = 256;
  hipStream_t s = (hipStream_t)stream;
  if (fmt == FMT_Q4_K)
    hipLaunchKernelGGL(shuffle_q4k, dim3((unsigned)((total + nt - 1) / nt)), dim3(nt), 0, s, gguf,
                       quant, meta, N, S);
  else
    hipLaunchKernelGGL(shuffle_q80, dim3((unsigned)((total + nt - 1) / nt)), dim3(nt), 0, s, gguf,
                       quant, meta, N, S);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

SV_API int64_t snowllm_gemm_kquant_a_ws_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 256) return 0;
  const int64_t tiles = (M + TILE_M - 1) / TILE_M;
  return (int64_t)(tiles * xprep_tile_bytes(K / 256));
}

// Extension (no counterpart in the reference): convert activations once into the operand
// workspace so several weights that share an input (gate/up, Q/K/V) reuse it.
SV_API int snowllm_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws,
                                         void* stream) {
  if (M < 0 || K <= 0 || K % 256) return SV_EINVAL;
  if (M == 0) return SV_OK;
  const int64_t S = K / 256;
  const int64_t mt = (M + TILE_M - 1) / TILE_M;
  hipLaunchKernelGGL(xprep_kernel, dim3((unsigned)S, (unsigned)mt), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)a, M, K, ws, xprep_tile_bytes(S));
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension (no counterpart in the reference): the GEMV on a prepared operand workspace.
SV_API int snowllm_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta,
                                          void* c, int64_t M, int64_t N, int64_t K,
                                          int c_is_bf16, const void* ws, void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t S = K / 256;
  const size_t tb = xprep_tile_bytes(S);
  const int64_t mt = (M + TILE_M - 1) / TILE_M;
  const size_t esz = c_is_bf16 ? 2 : 4;
  for (int64_t t = 0; t < mt; ++t) {
    const int rows = (int)((M - t * TILE_M) < TILE_M ? (M - t * TILE_M) : TILE_M);
    void* ct = (char*)c + (size_t)t * TILE_M * N * esz;
    const void* wst = (const char*)ws + t * tb;
    int rc = fmt == FMT_Q4_K
                 ? dispatch_gemv<FMT_Q4_K>(quant, meta, wst, ct, rows, (int)N, (int)S, c_is_bf16, s)
                 : dispatch_gemv<FMT_Q8_0>(quant, meta, wst, ct, rows, (int)N, (int)S, c_is_bf16, s);
    if (rc) return rc;
  }
  return SV_OK;
}

SV_API int snowllm_gemm_kquant_a(int fmt, const void* a, const uint8_t* quant, const uint8_t* meta,
                                 void* c, int64_t M, int64_t N, int64_t K, int c_is_bf16, void* ws,
                                 void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  int rc = snowllm_gemm_kquant_prepare_a(a, M, K, ws, stream);
  if (rc) return rc;
  return snowllm_gemm_kquant_a_prepared(fmt, quant, meta, c, M, N, K, c_is_bf16, ws, stream);
}
