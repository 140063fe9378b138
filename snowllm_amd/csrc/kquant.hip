// GGUF Q4_K / Q8_0 dequant-GEMV for short verify blocks (M <= 16 rows per pass) on gfx950:
// repack, activation prep and the plain GEMV (shared device code in kquant_core.h).
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
// converted to fp16 once per call with a power-of-two scale per (row, superblock), exact for
// bf16 input.
#include "kquant_core.h"

#include <mutex>
#include <type_traits>

namespace {
using namespace kq;

// ---------------------------------------------------------------------------------------
// Activation prep kernel: one wave per (row tile, superblock), writing the workspace.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) xprep_kernel(const uint16_t* __restrict__ a, int64_t M,
                                                   int64_t K, void* ws, size_t tile_bytes) {
  const int s = blockIdx.x, tile = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t S = K / QK;
  XPrepView v = xprep_view((char*)ws + tile * tile_bytes, S);
  const int64_t r0 = (int64_t)tile * TILE_M;
  XOperands o;
  convert_superblock(a + r0 * K, K, (int)(M - r0 < TILE_M ? M - r0 : TILE_M), s, lane, o);
  store_operands(v, s, lane, o);
}

// NW waves split the superblocks of NTILE column tiles; the waves' partial sums meet in LDS
// and are added in a fixed order. Reads past the end of a buffer return zero (buffer range
// checking), so the last partial tile group needs no clamping.
// RAW: ws is the bf16 activation matrix [M, S*256] itself, converted in-kernel (one launch
// for the whole operator instead of a prep pass + GEMV).
template <int FMT, int NTILE, int NW, bool RAW = false>
__global__ void __launch_bounds__(NW * 64) kquant_gemv(const u32x4* __restrict__ quant,
                                                       const u32x4* __restrict__ meta,
                                                       const void* __restrict__ ws,
                                                       void* __restrict__ c, int M, int N, int S,
                                                       int c_bf16, int ldc) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int kq = lane >> 4;
  const int tiles = N / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  const GemvStreams st = make_streams<FMT>(quant, meta, ws, tiles, S, lane, M);
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (RAW) {
    const RawX rx = make_raw_x(ws, M, S * QK, lane);
    gemv_loop_raw<FMT, NTILE, NW>(st, rx, w, S, tile0, 1, lane, Mv, acc);
  } else {
    gemv_loop<FMT, NTILE, NW>(st, w, S, tile0, 1, kq, Mv, acc);
  }
  combine_waves<NTILE, NW>(part, acc, w, lane);
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
      if (c_bf16) ((uint16_t*)c)[(int64_t)row * ldc + n] = f32_to_bf16(v[i]);
      else ((float*)c)[(int64_t)row * ldc + n] = v[i];
    }
  }
}

// ---------------------------------------------------------------------------------------
// The same GEMV over MT 16-row tiles at once (a verify step wider than 16 rows): each wave
// loads a superblock's weights once, decodes them once into the fp16 B operands, and multiplies
// them against the prepared operands of every row tile (blockIdx.y: the group of MT tiles).
// The per-row arithmetic and the waves' superblock split are those of kquant_gemv with NW
// waves, so every row gets the bits of the 16-row launch.
// ---------------------------------------------------------------------------------------
template <int FMT>
struct DecodedSb {
  half8 b[8];     // B operands of the 8 sub-blocks
  float a[8];     // per-sub-block scales (odd Q4_K sub-blocks: x 1/16 for the 16 q encoding)
  float beta_lo, beta_hi;
};

template <int FMT>
__device__ __forceinline__ void decode_sb(const u32x4* qv, u32x4 meta, int kq, uint32_t M,
                                          DecodedSb<FMT>& d) {
  if constexpr (FMT == FMT_Q4_K) {
    const float dd = f16_to_f32((uint16_t)(meta.x & 0xffff));
    const float dmin = f16_to_f32((uint16_t)(meta.x >> 16));
    const uint32_t s0 = meta.y, s1 = meta.z, s2 = meta.w;
    const uint32_t sc03 = s0 & 0x3f3f3f3fu;
    const uint32_t m03 = s1 & 0x3f3f3f3fu;
    const uint32_t sc47 = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m47 = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    float a[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = dd * byte_f(sc03, i);
      a[4 + i] = dd * byte_f(sc47, i);
    }
    const float m_lo = dmin * byte_f(m03, kq);
    const float m_hi = dmin * byte_f(m47, kq);
    const float off = (kq & 1) ? 64.0f : 1024.0f;
    d.beta_lo = __builtin_fmaf(off, dd * byte_f(sc03, kq), m_lo);
    d.beta_hi = __builtin_fmaf(off, dd * byte_f(sc47, kq), m_hi);
#pragma unroll
    for (int j = 0; j < 8; ++j) d.a[j] = (j & 1) ? a[j] * 0.0625f : a[j];
    q4_group(qv[0].x, qv[0].y, M, d.b[0], d.b[1]);
    q4_group(qv[0].z, qv[0].w, M, d.b[2], d.b[3]);
    q4_group(qv[1].x, qv[1].y, M, d.b[4], d.b[5]);
    q4_group(qv[1].z, qv[1].w, M, d.b[6], d.b[7]);
  } else {
    const uint32_t dw[4] = {meta.x, meta.y, meta.z, meta.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d.a[2 * i] = f16_to_f32((uint16_t)(dw[i] & 0xffff));
      d.a[2 * i + 1] = f16_to_f32((uint16_t)(dw[i] >> 16));
    }
    d.beta_lo = 1152.0f * f16_to_f32((uint16_t)(((kq & 1) ? (dw[kq >> 1] >> 16) : dw[kq >> 1]) & 0xffff));
    d.beta_hi = 1152.0f * f16_to_f32((uint16_t)(((kq & 1) ? (dw[2 + (kq >> 1)] >> 16) : dw[2 + (kq >> 1)]) & 0xffff));
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      d.b[2 * jp] = q8_sub(qv[jp].x, qv[jp].y, M);
      d.b[2 * jp + 1] = q8_sub(qv[jp].z, qv[jp].w, M);
    }
  }
}

// tile_superblock's arithmetic on decoded weights: the same products and sums in the same order.
template <int FMT>
__device__ __forceinline__ floatx4 apply_sb(const DecodedSb<FMT>& d, const half8* xa, float sx0,
                                            float sx1) {
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  floatx4 acc = zero;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], d.b[j], zero, 0, 0, 0);
    acc += d.a[j] * c;
  }
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx0, d.beta_lo, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sx1, d.beta_hi, acc, 0, 0, 0);
  return acc;
}

template <int FMT, int NW, int MT, int NT = 1>
__global__ void __launch_bounds__(NW * 64) kquant_gemv_mt(const u32x4* __restrict__ quant,
                                                          const u32x4* __restrict__ meta,
                                                          const void* __restrict__ ws,
                                                          void* __restrict__ c, int M, int N,
                                                          int S, int c_bf16, size_t tile_bytes,
                                                          int ldc) {
  constexpr int QV = QLayout<FMT>::kQuantVecs;
  __shared__ floatx4 part[NW][NT][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4, r = lane & 15;
  const int tiles = N / TILE_N;
  const int tile0 = blockIdx.x * NT;  // NT column tiles share each row tile's operands
  const int m0 = blockIdx.y * MT;
  const int row_tiles = (M + TILE_M - 1) / TILE_M;
  const int mt = row_tiles - m0 < MT ? row_tiles - m0 : MT;
  const GemvStreams st = make_streams<FMT>(quant, meta, ws, tiles, S, lane, 16);
  __amdgpu_buffer_rsrc_t xr[MT], sxr[MT], scr[MT];
  uint32_t vx[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    XPrepView xv = xprep_view((char*)ws + (size_t)(m0 + m) * tile_bytes, S);
    xr[m] = __builtin_amdgcn_make_buffer_rsrc((void*)xv.xop, 0, S * 8 * 64 * 16, 0x00020000);
    sxr[m] = __builtin_amdgcn_make_buffer_rsrc((void*)xv.sxop, 0, S * 2 * 64 * 4, 0x00020000);
    scr[m] = __builtin_amdgcn_make_buffer_rsrc((void*)xv.scale, 0, S * 16 * 4, 0x00020000);
    vx[m] = r < M - (m0 + m) * TILE_M ? lane * 16 : 0x80000000u;
  }
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[MT][NT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s = w; s < S; s += NW) {
    // (a tile past the last reads nothing: its buffer offsets are out of range)
    u32x4 q[NT][QV], mt4[NT];
    uint32_t dq[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) dq[t] = 0u;
    load_sb_w<FMT, NT>(q, mt4, st, s, S, tile0, 1);
    if constexpr (FMT == FMT_Q6_K) load_sb_d<NT>(dq, st, s, S, tile0, 1);
    // every row tile's operands of this superblock in flight with the weights
    u32x4 x[MT][8];
    float sx0[MT], sx1[MT];
    floatx4 sc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= mt) break;  // uniform
#pragma unroll
      for (int j = 0; j < 8; ++j) x[m][j] = bload4(xr[m], vx[m], (uint32_t)((s * 8 + j) * 64 * 16));
      sx0[m] = bload1(sxr[m], lane * 4, (uint32_t)((s * 2 + 0) * 64 * 4));
      sx1[m] = bload1(sxr[m], lane * 4, (uint32_t)((s * 2 + 1) * 64 * 4));
      sc[m] = __builtin_bit_cast(floatx4, bload4(scr[m], kq * 16, (uint32_t)(s * 16 * 4)));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q8_0) {
        DecodedSb<FMT> d;
        decode_sb<FMT>(q[t], mt4[t], kq, Mv, d);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m >= mt) break;  // uniform
          half8 xa[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) xa[j] = __builtin_bit_cast(half8, x[m][j]);
          const floatx4 sb = apply_sb<FMT>(d, xa, sx0[m], sx1[m]);
          acc[m][t] += sb * sc[m];
        }
      } else {
        // Q5_K / Q6_K: the weights loaded once, decoded again for each row tile by the 16-row
        // kernel's own routine (their decoded operands do not fit the registers of four tiles)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m >= mt) break;  // uniform
          half8 xa[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) xa[j] = __builtin_bit_cast(half8, x[m][j]);
          const floatx4 sb =
              tile_superblock<FMT>(q[t], mt4[t], dq[t], xa, sx0[m], sx1[m], kq, Mv);
          acc[m][t] += sb * sc[m];
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m >= mt) break;  // uniform
    if (m) __syncthreads();
    combine_waves<NT, NW>(part, acc[m], w, lane);
    for (int idx = threadIdx.x; idx < NT * 64; idx += NW * 64) {
      const int t = idx >> 6, l = idx & 63;
      const int tile = tile0 + t;
      if (tile >= tiles) continue;
      floatx4 v = part[0][t][l];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) v += part[ww][t][l];
      const int n = tile * TILE_N + (l & 15);
      const int rb = (m0 + m) * TILE_M + 4 * (l >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rb + i;
        if (row >= M) break;
        if (c_bf16) ((uint16_t*)c)[(int64_t)row * ldc + n] = f32_to_bf16(v[i]);
        else ((float*)c)[(int64_t)row * ldc + n] = v[i];
      }
    }
  }
}

template <int FMT, int NW>
int launch_gemv_mt(const void* quant, const void* meta, const void* ws, void* c, int M, int N,
                   int S, int c_bf16, int ldc, hipStream_t s) {
  const int tiles = N / TILE_N;
  const int row_tiles = (M + TILE_M - 1) / TILE_M;
  const size_t tb = xprep_tile_bytes(S);
  // One row tile per workgroup (blockIdx.y), two column tiles per workgroup where that still
  // leaves 192 or more workgroups. Measured on MI355X (prepared operands, the weights from
  // HBM): decoding a weight superblock once for several row tiles saves less than the
  // workgroups it takes away. N = 2048, K = 4096 at 36 / 54 / 128 rows: 9.3 / 11.2 / 11.6 us
  // with three or four row tiles per workgroup against 6.0 / 6.1 / 8.6 us; N = 5120, K = 2048
  // at 128 rows 20.8 against 11.1 us; N = 14336, K = 4096 at 72 rows 42.8 against 30.4 us.
  // One column tile only wins at N = 2048 and 18 rows (4.9 against 6.0 us). The same bits
  // either way (every row gets the 16-row launch's arithmetic).
  const int nt = (int64_t)(tiles / 2) * row_tiles >= 192 ? 2 : 1;
  auto go = [&](auto kern, int mt, int ntile) {
    hipLaunchKernelGGL(kern, dim3((tiles + ntile - 1) / ntile, (row_tiles + mt - 1) / mt),
                       dim3(NW * 64), 0, s, (const u32x4*)quant, (const u32x4*)meta, ws, c, M,
                       N, S, c_bf16, tb, ldc);
  };
  if (nt == 2) go(kquant_gemv_mt<FMT, NW, 1, 2>, 1, 2);
  else go(kquant_gemv_mt<FMT, NW, 1>, 1, 1);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// ---------------------------------------------------------------------------------------
// Repack GGUF blocks into (quant, meta).
// ---------------------------------------------------------------------------------------
// Rows n >= n_split come from `bottom` (row n - n_split), so that two GGUF tensors of one
// format repack as one matrix ([gate; up] of an expert); single matrices pass n_split = N.
__device__ __forceinline__ const uint8_t* src_block(const uint8_t* top, const uint8_t* bottom,
                                                    int64_t n_split, int64_t n, int64_t s,
                                                    int64_t S, int64_t bytes) {
  return n < n_split ? top + (n * S + s) * bytes : bottom + ((n - n_split) * S + s) * bytes;
}

__global__ void shuffle_q4k(const uint8_t* __restrict__ gguf, const uint8_t* __restrict__ gguf2,
                            int64_t n_split, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const uint8_t* blk = src_block(gguf, gguf2, n_split, n, s, S, 144);
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

__global__ void shuffle_q80(const uint8_t* __restrict__ gguf, const uint8_t* __restrict__ gguf2,
                            int64_t n_split, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  for (int j = 0; j < 8; ++j) {
    const uint8_t* blk = src_block(gguf, gguf2, n_split, n, s, S, 8 * 34) + j * 34;
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

// Q5_K: the Q4_K nibble layout of qs (@48), then each lane's 8 qh bytes (@16) after the tile-
// superblock's nibbles; meta as Q4_K (d, dmin, scales: the block's first 16 bytes).
__global__ void shuffle_q5k(const uint8_t* __restrict__ gguf, const uint8_t* __restrict__ gguf2,
                            int64_t n_split, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const uint8_t* blk = src_block(gguf, gguf2, n_split, n, s, S, 176);
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  uint8_t* mo = meta + (ts * 16 + col) * 16;
  for (int i = 0; i < 16; ++i) mo[i] = blk[i];
  const uint8_t* qh = blk + 16;
  const uint8_t* qs = blk + 48;
  uint8_t* base = quant + ts * 2560;
  for (int kq = 0; kq < 4; ++kq) {
    const int lane = col + 16 * kq;
    for (int h = 0; h < 2; ++h) {
      uint8_t* qo = base + (h * 64 + lane) * 16;
      for (int i = 0; i < 8; ++i) {
        qo[i] = qs[64 * h + 8 * kq + i];
        qo[8 + i] = qs[64 * h + 32 + 8 * kq + i];
      }
    }
    uint8_t* ho = base + 2048 + lane * 8;
    for (int i = 0; i < 8; ++i) ho[i] = qh[8 * kq + i];
  }
}

// Q6_K: per lane three 16-byte vectors (ql of half 0, ql of half 1, qh of both halves, each
// the bytes l = 8 kq .. 8 kq + 7 of its two 32-byte runs); meta: the 16 int8 scales per
// column, and after every tile-superblock's scales the fp16 d per (tile-superblock, column).
__global__ void shuffle_q6k(const uint8_t* __restrict__ gguf, const uint8_t* __restrict__ gguf2,
                            int64_t n_split, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const uint8_t* blk = src_block(gguf, gguf2, n_split, n, s, S, 210);
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  uint8_t* mo = meta + (ts * 16 + col) * 16;
  for (int i = 0; i < 16; ++i) mo[i] = blk[192 + i];
  uint8_t* dd = meta + N * S * 16 + (ts * 16 + col) * 2;
  dd[0] = blk[208];
  dd[1] = blk[209];
  const uint8_t* ql = blk;
  const uint8_t* qh = blk + 128;
  uint8_t* base = quant + ts * 3072;
  for (int kq = 0; kq < 4; ++kq) {
    const int lane = col + 16 * kq;
    for (int half = 0; half < 2; ++half) {
      uint8_t* qo = base + (half * 64 + lane) * 16;
      for (int i = 0; i < 8; ++i) {
        qo[i] = ql[64 * half + 8 * kq + i];
        qo[8 + i] = ql[64 * half + 32 + 8 * kq + i];
      }
    }
    uint8_t* ho = base + (2 * 64 + lane) * 16;
    for (int i = 0; i < 8; ++i) {
      ho[i] = qh[8 * kq + i];
      ho[8 + i] = qh[32 + 8 * kq + i];
    }
  }
}

bool fmt_ok(int fmt) {
  return fmt == FMT_Q4_K || fmt == FMT_Q5_K || fmt == FMT_Q6_K || fmt == FMT_Q8_0;
}

// The GEMV kernels address a weight through one buffer resource with 32-bit offsets: its
// packed quants (N * K / 2 bytes for Q4_K, N * K for Q8_0) must stay below 4 GiB.
bool weight_fits(int fmt, int64_t N, int64_t K) {
  const int64_t qbytes = fmt == FMT_Q4_K ? N * (K / 2) : fmt == FMT_Q5_K ? N * (K / 256) * 160
                         : fmt == FMT_Q6_K ? N * (K / 256) * 192 : N * K;
  return qbytes <= (int64_t)0xFFFFFC00 && N * (K / 256) * 256 <= (int64_t)0xFFFFFFFF;
}

template <int FMT, int NTILE, int NW, bool RAW = false>
int launch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N, int S,
                int c_bf16, int ldc, hipStream_t s) {
  const int tiles = N / TILE_N;
  const int grid = (tiles + NTILE - 1) / NTILE;
  hipLaunchKernelGGL((kquant_gemv<FMT, NTILE, NW, RAW>), dim3(grid), dim3(NW * 64), 0, s,
                     (const u32x4*)quant, (const u32x4*)meta, ws, c, M, N, S, c_bf16, ldc);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

int g_gemv_variant = 0;  // 0 = automatic; see snowverify_gemv_variant

// Calls f with std::integral_constant<int, FMT> for a supported format id.
template <class F>
int by_format(int fmt, F&& f) {
  switch (fmt) {
    case FMT_Q4_K: return f(std::integral_constant<int, FMT_Q4_K>{});
    case FMT_Q5_K: return f(std::integral_constant<int, FMT_Q5_K>{});
    case FMT_Q6_K: return f(std::integral_constant<int, FMT_Q6_K>{});
    case FMT_Q8_0: return f(std::integral_constant<int, FMT_Q8_0>{});
    default: return SV_EINVAL;
  }
}

template <int FMT, bool RAW = false>
int dispatch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N,
                  int S, int c_bf16, int ldc, hipStream_t s) {
  switch (g_gemv_variant) {
    case 1: return launch_gemv<FMT, 1, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    case 2: return launch_gemv<FMT, 2, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    case 3: return launch_gemv<FMT, 4, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    case 4: return launch_gemv<FMT, 1, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    case 5: return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    case 6: return launch_gemv<FMT, 4, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    default: break;
  }
  const int tiles = N / TILE_N;
  // measured on MI355X (M = 9): wide outputs want 4 tiles x 8 waves, K >= 4096 narrow outputs
  // 1 x 8, K = 2048 2 x 8 when there are >= 2 tiles per CU, K = 4096 (prepared operands)
  // 2 x 8 from 3 tiles per CU (6144 x 4096: 9.7 -> 7.6 us)
  if (S >= 8) {
    // (Q8_0 keeps two tiles: four tiles of int8 quants exceed the register file)
    if (tiles >= 4 * 192 && FMT == FMT_Q4_K)
      return launch_gemv<FMT, 4, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    if (tiles >= 2 * 128 && S <= 8) return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    if (!RAW && FMT == FMT_Q4_K && tiles >= 3 * 128 && S <= 16)
      return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
    return launch_gemv<FMT, 1, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
  }
  if (tiles >= 2 * 256) return launch_gemv<FMT, 2, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
  return launch_gemv<FMT, 1, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, ldc, s);
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

SV_API int64_t snowllm_kquant_gguf_bytes(int fmt, int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  if (fmt == FMT_Q4_K) return K % 256 ? -1 : N * (K / 256) * 144;
  if (fmt == FMT_Q5_K) return K % 256 ? -1 : N * (K / 256) * 176;
  if (fmt == FMT_Q6_K) return K % 256 ? -1 : N * (K / 256) * 210;
  if (fmt == FMT_Q8_0) return K % 32 ? -1 : N * (K / 32) * 34;
  return -1;
}

// Repacked sizes: quant + meta - 4 = the GGUF bytes (the quant buffer keeps 4 bytes of slack).
SV_API int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  const int64_t blocks = N * (K / 256);
  switch (fmt) {
    case FMT_Q4_K: return blocks * 128 + 4;
    case FMT_Q5_K: return blocks * 160 + 4;
    case FMT_Q6_K: return blocks * 192 + 4;
    default: return N * K + 4;
  }
}

SV_API int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  return N * (K / 256) * (fmt == FMT_Q6_K ? 18 : 16);
}

SV_API int snowllm_kquant_supported(int fmt) { return fmt_ok(fmt) ? 1 : 0; }

// Extension (tuning knob, no counterpart in the reference): force a GEMV tile shape
// (0 = automatic, 1..6 = fixed (tiles per workgroup, waves) pairs). Process-global.
SV_API void snowverify_gemv_variant(int v) { g_gemv_variant = v; }

// Extension (no counterpart in the reference): repack two GGUF tensors of one format, `top`
// (rows 0 .. n_top - 1) and `bottom` (rows n_top .. N - 1), as one [N, K] matrix -- an
// expert's [gate; up] from its two stacks.
SV_API int snowverify_kquant_shuffle_split(int fmt, const uint8_t* top, const uint8_t* bottom,
                                           int64_t n_top, uint8_t* quant, uint8_t* meta,
                                           int64_t N, int64_t K, void* stream) {
  if (!fmt_ok(fmt) || N <= 0 || K <= 0 || K % 256 || N % TILE_N || n_top < 0 || n_top > N ||
      !top || (n_top < N && !bottom))
    return SV_EINVAL;
  const int64_t S = K / 256;
  const int64_t total = N * S;
  const int nt = 256;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((total + nt - 1) / nt));
  if (fmt == FMT_Q4_K)
    hipLaunchKernelGGL(shuffle_q4k, grid, dim3(nt), 0, s, top, bottom, n_top, quant, meta, N, S);
  else if (fmt == FMT_Q5_K)
    hipLaunchKernelGGL(shuffle_q5k, grid, dim3(nt), 0, s, top, bottom, n_top, quant, meta, N, S);
  else if (fmt == FMT_Q6_K)
    hipLaunchKernelGGL(shuffle_q6k, grid, dim3(nt), 0, s, top, bottom, n_top, quant, meta, N, S);
  else
    hipLaunchKernelGGL(shuffle_q80, grid, dim3(nt), 0, s, top, bottom, n_top, quant, meta, N, S);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

SV_API int snowllm_gemm_kquant_shuffle_b(int fmt, const uint8_t* gguf, uint8_t* quant,
                                         uint8_t* meta, int64_t N, int64_t K, void* stream) {
  return snowverify_kquant_shuffle_split(fmt, gguf, nullptr, N, quant, meta, N, K, stream);
}

SV_API int64_t snowllm_gemm_kquant_a_ws_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 256) return 0;
  const int64_t tiles = (M + TILE_M - 1) / TILE_M;
  return (int64_t)(tiles * xprep_tile_bytes(K / 256));
}

// Extension (no counterpart in the reference): convert activations once into the operand
// workspace so several weights that share an input (gate/up, Q/K/V) reuse it.
SV_API int snowverify_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws,
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

// Extension (no counterpart in the reference): the GEMV on a prepared operand workspace,
// writing row m of the result at c + m * ldc (ldc >= N elements), so that two weights of
// different formats fill the column ranges of one output (Q|K and V of a fused projection).
SV_API int snowverify_gemm_kquant_a_prepared_ld(int fmt, const uint8_t* quant,
                                                const uint8_t* meta, void* c, int64_t ldc,
                                                int64_t M, int64_t N, int64_t K, int c_is_bf16,
                                                const void* ws, void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N || ldc < N ||
      ldc > INT32_MAX)
    return SV_EINVAL;
  if (!weight_fits(fmt, N, K)) return SV_ENOTSUP;
  if (M == 0) return SV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t S = K / 256;
  const size_t tb = xprep_tile_bytes(S);
  const int64_t mt = (M + TILE_M - 1) / TILE_M;
  const size_t esz = c_is_bf16 ? 2 : 4;
  const int ld = (int)ldc;
  if (mt > 1 && g_gemv_variant == 0) {
    // wider than one row tile: one launch over every row tile (the waves split the
    // superblocks as the automatic 16-row launch does: the same bits)
    return by_format(fmt, [&](auto F) {
      constexpr int FM = decltype(F)::value;
      return S >= 8 ? launch_gemv_mt<FM, 8>(quant, meta, ws, c, (int)M, (int)N, (int)S, c_is_bf16, ld, s)
                    : launch_gemv_mt<FM, 4>(quant, meta, ws, c, (int)M, (int)N, (int)S, c_is_bf16, ld, s);
    });
  }
  for (int64_t t = 0; t < mt; ++t) {
    const int rows = (int)((M - t * TILE_M) < TILE_M ? (M - t * TILE_M) : TILE_M);
    void* ct = (char*)c + (size_t)t * TILE_M * ldc * esz;
    const void* wst = (const char*)ws + t * tb;
    int rc = by_format(fmt, [&](auto F) {
      return dispatch_gemv<decltype(F)::value>(quant, meta, wst, ct, rows, (int)N, (int)S,
                                               c_is_bf16, ld, s);
    });
    if (rc) return rc;
  }
  return SV_OK;
}

// Extension (no counterpart in the reference): the GEMV on a prepared operand workspace.
SV_API int snowverify_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta,
                                          void* c, int64_t M, int64_t N, int64_t K,
                                          int c_is_bf16, const void* ws, void* stream) {
  return snowverify_gemm_kquant_a_prepared_ld(fmt, quant, meta, c, N, M, N, K, c_is_bf16, ws,
                                              stream);
}

SV_API int snowllm_gemm_kquant_a(int fmt, const void* a, const uint8_t* quant, const uint8_t* meta,
                                 void* c, int64_t M, int64_t N, int64_t K, int c_is_bf16, void* ws,
                                 void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (!weight_fits(fmt, N, K)) return SV_ENOTSUP;
  if (M == 0) return SV_OK;
  if (M <= TILE_M && M * K * 2 <= INT32_MAX) {
    // one launch: the GEMV converts the bf16 activations itself (same operands as the
    // prepared path, so the same results); ws is not touched
    hipStream_t s = (hipStream_t)stream;
    return by_format(fmt, [&](auto F) {
      return dispatch_gemv<decltype(F)::value, true>(quant, meta, a, c, (int)M, (int)N,
                                                     (int)(K / 256), c_is_bf16, (int)N, s);
    });
  }
  int rc = snowverify_gemm_kquant_prepare_a(a, M, K, ws, stream);
  if (rc) return rc;
  return snowverify_gemm_kquant_a_prepared(fmt, quant, meta, c, M, N, K, c_is_bf16, ws, stream);
}

// ---------------------------------------------------------------------------------------
// The no-allocation form of snowllm_gemm_kquant_a, for callers that cannot allocate (code
// under HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc). Up to 16
// rows the GEMV converts the activations itself and needs no workspace; above that the
// operand workspace lives in `scratch`, a file-scope device array of a fixed size -- each GPU
// the library runs on holds its own copy until the process ends. Host code never passes the
// array's name to a kernel: its device address is read once per device with
// hipGetSymbolAddress, with that device current, and kept.
// ---------------------------------------------------------------------------------------
namespace {
constexpr int64_t NOALLOC_MAX_M = 64, NOALLOC_MAX_K = 16384;
constexpr size_t NOALLOC_WS_BYTES = 2244608;  // snowllm_gemm_kquant_a_ws_bytes(64, 16384)
static __device__ __align__(256) uint8_t scratch[NOALLOC_WS_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];

// The current device's address of `scratch`.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return SV_ENOTSUP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return SV_EINVAL;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SV_OK;
}
}  // namespace

SV_API int snowverify_gemm_kquant_a_noalloc(int fmt, const void* a, const uint8_t* quant,
                                            const uint8_t* meta, void* c, int64_t M, int64_t N,
                                            int64_t K, int c_is_bf16, void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (M > NOALLOC_MAX_M || K > NOALLOC_MAX_K) return SV_EINVAL;  // beyond the array
  if (M == 0) return SV_OK;
  if (M <= TILE_M)  // the one-launch form: no workspace
    return snowllm_gemm_kquant_a(fmt, a, quant, meta, c, M, N, K, c_is_bf16, nullptr, stream);
  if ((size_t)snowllm_gemm_kquant_a_ws_bytes(M, K) > NOALLOC_WS_BYTES) return SV_EINVAL;
  void* ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc) return rc;
  // the prep pass writes every byte of the workspace the GEMV reads (padding rows included),
  // so nothing needs clearing between calls
  rc = snowverify_gemm_kquant_prepare_a(a, M, K, ws, stream);
  if (rc) return rc;
  return snowverify_gemm_kquant_a_prepared(fmt, quant, meta, c, M, N, K, c_is_bf16, ws, stream);
}
