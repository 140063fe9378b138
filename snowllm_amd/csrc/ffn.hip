// Feed-forward side of the verify step on gfx950:
//   - residual update + RMSNorm fused with the fp16 operand conversion of the GEMVs;
//   - GEMV with fp16 weights (LM head) and bf16 weights (MoE router), MFMA, no dequant;
//   - gate/up Q4_K GEMV with SwiGLU in the epilogue (dense MLP and MoE experts);
//   - MoE: a device-side plan of the experts the block touches (no host round trip), expert
//     gate/up + SwiGLU and expert down GEMVs over that plan, and the weighted combine.
//
// Expert weights of one layer are stored back to back: gate/up of expert e is the packed
// [2F, H] k-quant matrix (gate rows 0..F-1, up rows F..2F-1) at e * gu_bytes, down of expert e
// the packed [H, F] matrix at e * dn_bytes (quant and meta kept in separate arrays, as the
// repack produces them). The shared expert has its own pair of matrices.
#include "kquant_core.h"

#include <mutex>
#include <type_traits>

namespace {
using namespace kq;

inline hipStream_t Sx(void* s) { return (hipStream_t)s; }

// ---------------------------------------------------------------------------------------
// residual + RMSNorm + operand conversion. One workgroup per row, one thread per 16-byte word
// of the row (thread t holds k = 8 t .. 8 t + 7), so the row is read with one load per thread:
//   v = bf16(x + res_in) (v = x without res_in) -> res_out
//   y = bf16(v * rsqrt(mean(v^2) + eps) * gamma) -> y_out (optional), fp16 operands -> ws
// The sum of squares meets over the waves in LDS in a fixed order. Word t is (superblock
// t / 32, sub-block (t / 4) % 8, k-group t % 4), so a superblock's 32 words lie in one half
// wave and a sub-block's 4 words in one quad: the conversion's per-(row, superblock) maximum
// and sub-block sums are cross-lane moves within the wave. The tile's rows past M write zero
// operands, as the conversion of a zero row would.
// ---------------------------------------------------------------------------------------
constexpr int NORM_MAX_THREADS = 1024;

__device__ __forceinline__ u32x4 add_bf16_words(const u32x4& xv, const u32x4& rv) {
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __uint_as_float(xw[i] << 16) + __uint_as_float(rw[i] << 16);
    const float b = __uint_as_float(xw[i] & 0xffff0000u) + __uint_as_float(rw[i] & 0xffff0000u);
    o[i] = pack_bf16x2(a, b);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// The MoE layer's output as the norm's input: x[r] = bf16(sum_k pairs[r * topk + k] +
// shared[r]) in that order (the combine of the experts' pre-weighted rows), optionally
// written to x_out.
struct MoeSource {
  const float* pairs;   // [M * topk, H] f32, or null: x is read as bf16
  const float* shared;  // [M, H] f32 or null
  uint16_t* x_out;      // [M, H] bf16 or null
  int topk;
};

constexpr int MOE_WORDS_INFLIGHT = 8;  // top-k rows whose loads are all issued before the sums

__device__ __forceinline__ u32x4 moe_words(const MoeSource& ms, int64_t row, int64_t H,
                                           int64_t col) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
  if (ms.shared) {
    const float4* src = (const float4*)(ms.shared + row * H + col);
    sa = src[0];
    sb = src[1];
  }
  if (ms.topk <= MOE_WORDS_INFLIGHT) {
    // every row's loads in flight first, then the sums in the same order as the loop below
    float4 a[MOE_WORDS_INFLIGHT], b[MOE_WORDS_INFLIGHT];
#pragma unroll
    for (int k = 0; k < MOE_WORDS_INFLIGHT; ++k) {
      if (k < ms.topk) {
        const float4* src = (const float4*)(ms.pairs + (row * ms.topk + k) * H + col);
        a[k] = src[0];
        b[k] = src[1];
      }
    }
#pragma unroll
    for (int k = 0; k < MOE_WORDS_INFLIGHT; ++k) {
      if (k < ms.topk) {
        acc[0] += a[k].x; acc[1] += a[k].y; acc[2] += a[k].z; acc[3] += a[k].w;
        acc[4] += b[k].x; acc[5] += b[k].y; acc[6] += b[k].z; acc[7] += b[k].w;
      }
    }
  } else {
    for (int k = 0; k < ms.topk; ++k) {
      const float4* src = (const float4*)(ms.pairs + (row * ms.topk + k) * H + col);
      const float4 a = src[0], b = src[1];
      acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
      acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
    }
  }
  if (ms.shared) {  // the shared expert's row last
    acc[0] += sa.x; acc[1] += sa.y; acc[2] += sa.z; acc[3] += sa.w;
    acc[4] += sb.x; acc[5] += sb.y; acc[6] += sb.z; acc[7] += sb.w;
  }
  return u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
               pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7])};
}

// (The arguments the loads need come first: the first 56 bytes arrive preloaded in SGPRs.)
__global__ void __launch_bounds__(NORM_MAX_THREADS) norm_prep_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ gamma, const float* __restrict__ src_pairs,
    const float* __restrict__ src_shared, int M32, int H32, int src_topk, float eps,
    uint16_t* __restrict__ x_out, uint16_t* __restrict__ res_out, uint16_t* __restrict__ y_out,
    void* __restrict__ ws, size_t tile_bytes) {
  const MoeSource ms{src_pairs, src_shared, x_out, src_topk};
  const int64_t M = M32, H = H32;
  __shared__ float part[NORM_MAX_THREADS / 64];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nwaves = (int)(blockDim.x >> 6);
  const int wpr = (int)(H >> 3);
  const bool act = t < wpr, live = act && row < M;
  const int64_t off = row * H + (int64_t)t * 8;
  u32x4 v = {0u, 0u, 0u, 0u}, gv = {0u, 0u, 0u, 0u};
  if (act) gv = *(const u32x4*)(gamma + (int64_t)t * 8);
  if (live) {
    u32x4 rv = {0u, 0u, 0u, 0u};
    if (residual) rv = *(const u32x4*)(residual + off);  // in flight with the row's loads
    if (ms.pairs) {
      v = moe_words(ms, row, H, (int64_t)t * 8);
      if (ms.x_out) *(u32x4*)(ms.x_out + off) = v;
    } else {
      v = *(const u32x4*)(x + off);
    }
    if (residual) v = add_bf16_words(v, rv);
  }
  const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __uint_as_float(vw[i] << 16), b = __uint_as_float(vw[i] & 0xffff0000u);
    ss = __builtin_fmaf(a, a, ss);
    ss = __builtin_fmaf(b, b, ss);
  }
  ss = wave_sum_dpp(ss);
  if (lane == 0) part[wv] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < nwaves; ++w) tot += part[w];
  const float inv = __frsqrt_rn(tot / (float)H + eps);
  float y[8];
  uint32_t yo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    yo[i] = pack_bf16x2(__uint_as_float(vw[i] << 16) * inv * __uint_as_float(gw[i] << 16),
                        __uint_as_float(vw[i] & 0xffff0000u) * inv *
                            __uint_as_float(gw[i] & 0xffff0000u));
    y[2 * i] = __uint_as_float(yo[i] << 16);
    y[2 * i + 1] = __uint_as_float(yo[i] & 0xffff0000u);
  }
  if (live) {
    if (res_out) *(u32x4*)(res_out + off) = v;
    if (y_out) *(u32x4*)(y_out + off) = u32x4{yo[0], yo[1], yo[2], yo[3]};
  }
  word_operand(y, t, row, ws, tile_bytes, H / QK, act);
}

// ---------------------------------------------------------------------------------------
// GEMV with 16-bit weights. Repacked layout: [tile][s][j][lane][8 halves] holding
// W[16 tile + (lane & 15)][256 s + 32 j + 8 (lane >> 4) + perm(e)] where perm is kperm for fp16
// weights (they meet the fp16 operand workspace) and the identity for bf16 weights (they
// meet bf16 activations read directly).
// ---------------------------------------------------------------------------------------
constexpr int WT_F16 = 1;
constexpr int WT_BF16 = 2;
constexpr int DENSE_MT = 4;        // row tiles per dense_gemv workgroup above two
constexpr int DENSE_MAX_M = 256;   // rows of one verify step

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// One launch covers up to MT 16-row tiles of the rows (blockIdx.y: the group of MT tiles):
// each superblock's weights are loaded once and multiplied against every tile's operands, so
// a wide verify block streams the weights once per MT tiles. Each row's arithmetic is the
// same whatever MT is (an MFMA row depends on its own operands only).
template <int WT, int NTILE, int NW, int MT>
__global__ void __launch_bounds__(NW * 64) dense_gemv(const u32x4* __restrict__ w,
                                                      const void* __restrict__ act,
                                                      void* __restrict__ c, int M, int N, int S,
                                                      int c_bf16, size_t tile_bytes) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4, r = lane & 15;
  const int tiles = (N + TILE_N - 1) / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  const int K = S * QK;
  const int m0 = blockIdx.y * MT;                       // first row tile of the group
  const int row_tiles = (M + TILE_M - 1) / TILE_M;
  const int mt = row_tiles - m0 < MT ? row_tiles - m0 : MT;
  // the block's own tiles as the buffer: offsets stay 32-bit whatever N * K is
  const int own = tiles - tile0 < NTILE ? tiles - tile0 : NTILE;
  __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)tile0 * S * 8 * 64), 0, own * S * 8 * 64 * 16, 0x00020000);
  __amdgpu_buffer_rsrc_t xr[MT], sr[MT];
  uint32_t vx[MT], vs[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int rows = M - (m0 + m) * TILE_M;  // valid rows of tile m0 + m (<= 0: none)
    if constexpr (WT == WT_F16) {
      XPrepView xv = xprep_view((char*)act + (size_t)(m0 + m) * tile_bytes, S);
      xr[m] = __builtin_amdgcn_make_buffer_rsrc((void*)xv.xop, 0, S * 8 * 64 * 16, 0x00020000);
      sr[m] = __builtin_amdgcn_make_buffer_rsrc((void*)xv.scale, 0, S * 16 * 4, 0x00020000);
      vx[m] = r < rows ? lane * 16 : 0x80000000u;
      vs[m] = kq * 16;
    } else {
      const int rv = rows < TILE_M ? (rows > 0 ? rows : 0) : TILE_M;
      xr[m] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)((const uint16_t*)act + (int64_t)(m0 + m) * TILE_M * K), 0, rv * K * 2,
          0x00020000);
      sr[m] = xr[m];
      vx[m] = r < rows ? (uint32_t)(r * K * 2 + kq * 16) : 0x80000000u;
      vs[m] = 0;
    }
  }
  floatx4 acc[MT][NTILE];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int t = 0; t < NTILE; ++t) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s = wv; s < S; s += NW) {
    u32x4 wb[NTILE][8];
#pragma unroll
    for (int t = 0; t < NTILE; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        wb[t][j] = bload4(wr, lane * 16, (uint32_t)(((t * S + s) * 8 + j) * 64 * 16));
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= mt) break;  // uniform
      u32x4 xa[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (WT == WT_F16) xa[j] = bload4(xr[m], vx[m], (uint32_t)((s * 8 + j) * 64 * 16));
        else xa[j] = bload4(xr[m], vx[m], (uint32_t)((s * QK + j * 32) * 2));
      }
      floatx4 scale = {1.f, 1.f, 1.f, 1.f};
      if constexpr (WT == WT_F16)
        scale = __builtin_bit_cast(floatx4, bload4(sr[m], vs[m], (uint32_t)(s * 16 * 4)));
#pragma unroll
      for (int t = 0; t < NTILE; ++t) {
        floatx4 sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if constexpr (WT == WT_F16)
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xa[j]),
                                                        __builtin_bit_cast(half8, wb[t][j]), sb, 0, 0, 0);
          else
            sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[j]),
                                                         __builtin_bit_cast(bf16x8, wb[t][j]), sb, 0, 0, 0);
        }
        acc[m][t] += sb * scale;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m >= mt) break;  // uniform
    if (m) __syncthreads();  // the previous tile's partials are read
    combine_waves<NTILE, NW>(part, acc[m], wv, lane);
    for (int idx = threadIdx.x; idx < NTILE * 64; idx += NW * 64) {
      const int t = idx >> 6, l = idx & 63;
      const int tile = tile0 + t;
      if (tile >= tiles) continue;
      floatx4 v = part[0][t][l];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) v += part[ww][t][l];
      const int n = tile * TILE_N + (l & 15);
      if (n >= N) continue;
      const int rb = (m0 + m) * TILE_M + 4 * (l >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rb + i;
        if (row >= M) break;
        if (c_bf16) ((uint16_t*)c)[(int64_t)row * N + n] = f32_to_bf16(v[i]);
        else ((float*)c)[(int64_t)row * N + n] = v[i];
      }
    }
  }
}

__global__ void dense_shuffle_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                     int64_t N, int64_t K, int wt) {
  // one thread per (tile, s, j, lane): 8 halves
  const int64_t S = K / QK, tiles = (N + TILE_N - 1) / TILE_N;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= tiles * S * 8 * 64) return;
  const int lane = (int)(id & 63);
  const int64_t rest = id >> 6;
  const int j = (int)(rest % 8);
  const int64_t s = (rest / 8) % S, tile = rest / 8 / S;
  const int64_t n = tile * TILE_N + (lane & 15);
  const int64_t k0 = s * QK + j * 32 + (lane >> 4) * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t k = k0 + (wt == WT_F16 ? kperm_c(e) : e);
    dst[id * 8 + e] = n < N ? src[n * K + k] : (uint16_t)0;
  }
}

// ---------------------------------------------------------------------------------------
// Gate/up (+ SwiGLU) over tile pairs (p, p + F/16) of a packed [2F, K] k-quant weight.
// `plan` selects the expert per grid.y slot (MoE) or is null (dense MLP, one weight).
// act_out: [slots, 16, F] bf16 (MoE; rows >= M zero) or [M, F] (dense).
// ---------------------------------------------------------------------------------------
// MoE plan: per slot (a routed expert the block touches, then the shared expert) the rows
// routed to it in ascending order, compacted, and each row's (row * topk + k) pair index. A
// block of up to MOE_MAX_M rows: an expert with more than 16 rows takes several consecutive
// slots of 16 (its rows in order), so that every slot fits one 16-row operand tile and each
// expert's weights are read once per 16 of its rows; the shared expert takes ceil(M / 16).
// ---------------------------------------------------------------------------------------
constexpr int MOE_MAX_M = 64;       // block rows per plan
constexpr int MOE_MAX_PICKS = 512;  // rows * topk per plan
// routed slots <= unique experts + picks / 16 (an expert of c rows takes <= 1 + c / 16; one
// slot each up to 16 rows), then the shared expert's ceil(M / 16)
constexpr int MOE_MAX_SLOTS = 256 + MOE_MAX_PICKS / 16 + MOE_MAX_M / 16;  // 292
struct MoePlan {
  int32_t n_slots;                         // routed slots + shared slots
  int32_t n_routed;                        // routed slots
  int32_t slot_expert[MOE_MAX_SLOTS];      // expert id per slot (E = shared)
  int32_t slot_rows[MOE_MAX_SLOTS];        // rows of the slot (<= 16)
  int32_t row_of[MOE_MAX_SLOTS][16];       // compact position -> block row
  int32_t pair_of[MOE_MAX_SLOTS][16];      // compact position -> pair index (-1: shared)
  uint32_t epoch;                          // nonzero, new for every plan written
};

// Slots a plan of M rows, topk picks each, can take (routed + shared).
inline int64_t moe_plan_slots(int64_t M, int64_t topk, int64_t E, bool shared) {
  const int64_t picks = M * topk;
  // up to 16 rows no expert takes a second slot
  return std::min(E, picks) + (M > 16 ? picks / 16 : 0) + (shared ? (M + 15) / 16 : 0);
}

// Plan generation counter: every plan kernel takes the next value (skipping 0) for its plan.
// Plan kernels are stream-ordered on one device, so one thread updates it without atomics.
__device__ uint32_t g_moe_epoch;

// Row gather for one wave: compact row r = lane & 15 of the slot reads block row row_of[r]
// from the operand workspace (row R in 16-row tile R / 16, tiles tile_bytes apart); rows past
// the slot's count read zeros (out-of-range offsets). The streams' ranges cover the block's
// `tiles` operand tiles.
__device__ __forceinline__ void gather_rows(GemvStreams& st, const int32_t* rows, int n_rows,
                                            int lane, const void* ws, int S, int tiles,
                                            uint32_t tile_bytes) {
  const int r = lane & 15, kq = lane >> 4;
  const int R = r < n_rows ? rows[r] : -1;
  const uint32_t tr = R >= 0 ? (uint32_t)(R >> 4) * tile_bytes : 0u;
  const int rr = R & 15;
  st.v_xop = R >= 0 ? tr + (uint32_t)((rr + 16 * kq) * 16) : 0x80000000u;
  st.v_sx = R >= 0 ? tr + (uint32_t)((rr + 16 * kq) * 4) : 0x80000000u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ci = 4 * kq + i;
    const int Ri = ci < n_rows ? rows[ci] : -1;
    st.v_scale_g[i] = Ri >= 0 ? (uint32_t)(Ri >> 4) * tile_bytes + (uint32_t)((Ri & 15) * 4)
                              : 0x80000000u;
  }
  if (tiles > 1) {
    const XPrepView xv = xprep_view((void*)ws, S);
    const uint32_t more = (uint32_t)(tiles - 1) * tile_bytes;
    st.xop = __builtin_amdgcn_make_buffer_rsrc((void*)xv.xop, 0, (int)(more + S * 8 * 64 * 16),
                                               0x00020000);
    st.sxop = __builtin_amdgcn_make_buffer_rsrc((void*)xv.sxop, 0, (int)(more + S * 2 * 64 * 4),
                                                0x00020000);
    st.scale = __builtin_amdgcn_make_buffer_rsrc((void*)xv.scale, 0, (int)(more + S * 16 * 4),
                                                 0x00020000);
  }
}

// ---------------------------------------------------------------------------------------
// Gate/up GEMV with SwiGLU in the epilogue: act[r, n] = silu(x Wg^T)[r, n] * (x Wu^T)[r, n],
// gate_up the packed [2F, K] k-quant weight (gate rows first). Block = PPB pairs (a gate tile
// and its up tile) x WS waves splitting the superblocks; blockIdx.y = MoE slot (plan mode:
// the slot's expert, rows gathered, act written compact at act_out + slot * 16 * F) or the
// whole block (plan == null: rows 0..M-1 of x, act [M, F]).
// ---------------------------------------------------------------------------------------
// bx: the block's pair group; slot: the plan slot (plan mode) or 0. DEVICE_SCOPE: the
// activations are stored with device-scope stores (visible to other workgroups of the same
// launch once the stores complete). SC: 0, or the superblock count S when the waves walk them
// with three weight buffers each (gemv_loop_deep). VW: with WS = 1, the number of waves the
// one wave stands for (it keeps their partial sums and adds them in their order: VW = 2 gives
// the bits of WS = 2).
template <int FMT, int WS, int PPB, bool DEVICE_SCOPE, int SC = 0, int VW = 1>
__device__ __forceinline__ void gate_up_body(
    int bx, int slot, const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta,
    int64_t gu_qbytes, int64_t gu_mbytes, const uint8_t* __restrict__ sh_quant,
    const uint8_t* __restrict__ sh_meta, const MoePlan* __restrict__ plan, int E,
    const void* __restrict__ ws, uint16_t* __restrict__ act_out, int M, int F, int S) {
  __shared__ floatx4 part[PPB][WS][2][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pl = wv / WS, sw = wv % WS;
  const int kq = lane >> 4;
  const int half_tiles = F / TILE_N;
  const int pair = bx * PPB + pl;
  const uint8_t* q = quant;
  const uint8_t* m = meta;
  int n_rows = M;
  if (plan) {
    if (slot >= plan->n_slots) return;
    const int e = plan->slot_expert[slot];
    if (e >= E) { q = sh_quant; m = sh_meta; }
    else { q = quant + e * gu_qbytes; m = meta + e * gu_mbytes; }
    n_rows = plan->slot_rows[slot];
  }
  GemvStreams st = make_streams<FMT>(q, m, ws, 2 * half_tiles, S, lane, M);
  const uint32_t Mv = decode_magic<FMT>();
  static_assert(VW == 1 || (WS == 1 && SC > 0), "virtual waves: one wave, the deep loop");
  floatx4 acc[2 * VW];
#pragma unroll
  for (int i = 0; i < 2 * VW; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (pair < half_tiles) {
    if (plan) {
      gather_rows(st, plan->row_of[slot], n_rows, lane, ws, S, (M + 15) >> 4,
                  (uint32_t)xprep_tile_bytes(S));
      if constexpr (SC > 0)
        gemv_loop_deep<FMT, 2, SC / WS, true, WS, VW>(st, sw, pair, half_tiles, kq, Mv, acc);
      else
        gemv_loop<FMT, 2, WS, true>(st, sw, S, pair, half_tiles, kq, Mv, acc);
    } else {
      if constexpr (SC > 0)
        gemv_loop_deep<FMT, 2, SC / WS, false, WS, VW>(st, sw, pair, half_tiles, kq, Mv, acc);
      else
        gemv_loop<FMT, 2, WS>(st, sw, S, pair, half_tiles, kq, Mv, acc);
    }
  }
  floatx4 g = acc[0], u = acc[1];
#pragma unroll
  for (int v = 1; v < VW; ++v) {  // the virtual waves' partials in the order WS waves add them
    g += acc[2 * v];
    u += acc[2 * v + 1];
  }
  if constexpr (WS > 1) {
    part[pl][sw][0][lane] = acc[0];
    part[pl][sw][1][lane] = acc[1];
    __syncthreads();
    if (sw != 0) return;
    g = part[pl][0][0][lane];
    u = part[pl][0][1][lane];
#pragma unroll
    for (int j = 1; j < WS; ++j) {
      g += part[pl][j][0][lane];
      u += part[pl][j][1][lane];
    }
  }
  if (pair >= half_tiles) return;
  const int n = pair * TILE_N + (lane & 15);
  const int rb = 4 * (lane >> 4);
  uint16_t* out = plan ? act_out + (int64_t)slot * 16 * F : act_out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = rb + i;
    if (row >= n_rows) break;
    const float gg = bf16_to_f32(f32_to_bf16(g[i]));  // projections are bf16 tensors
    const float uu = bf16_to_f32(f32_to_bf16(u[i]));
    const uint16_t a = f32_to_bf16(gg / (1.0f + __expf(-gg)) * uu);
    if constexpr (DEVICE_SCOPE)
      __hip_atomic_store(out + (int64_t)row * F + n, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      out[(int64_t)row * F + n] = a;
  }
}

// The deep form (SC > 0) at two waves per SIMD: with a budget for more waves the compiler moves
// the later superblocks' loads down to their use.
template <int FMT, int WS, int PPB, int SC = 0, int VW = 1>
__global__ void __launch_bounds__(WS * PPB * 64)
    __attribute__((amdgpu_waves_per_eu(SC > 0 ? 2 : 1, SC > 0 ? 2 : 10))) gate_up_kernel(
    const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta, int64_t gu_qbytes,
    int64_t gu_mbytes, const uint8_t* __restrict__ sh_quant, const uint8_t* __restrict__ sh_meta,
    const MoePlan* __restrict__ plan, int E, const void* __restrict__ ws,
    uint16_t* __restrict__ act_out, int M, int F, int S) {
  gate_up_body<FMT, WS, PPB, false, SC, VW>(blockIdx.x, blockIdx.y, quant, meta, gu_qbytes,
                                            gu_mbytes, sh_quant, sh_meta, plan, E, ws, act_out,
                                            M, F, S);
}

// The gate/up loop by superblock count S: at S = 8 or 16 (hidden 2048 or 4096) each of a pair's
// two waves walks its S / 2 superblocks with the weights of the next two in flight behind the
// one it multiplies (gemv_loop_deep, unrolled), otherwise gemv_loop's one. The same sums in the
// same order either way.
template <class Fn>
void with_gu_depth(int64_t S, Fn&& fn) {
  if (S == 8) fn(std::integral_constant<int, 8>{});
  else if (S == 16) fn(std::integral_constant<int, 16>{});
  else fn(std::integral_constant<int, 0>{});
}

// MoE gate/up item shape: fn(WS, PPB, SC, VW) as integral constants. A launch of 64 or more
// slots (a block of 8 or more rows) at hidden 2048 runs one wave per pair standing for the two
// (gemv_loop_deep with VW = 2, the same bits): 32 gate/up waves per slot instead of 64, so
// that up to 96 slots' gate/up items are all resident at once (three waves per SIMD) and none
// starts late. Smaller launches fit either way and keep two waves per pair, whose walk is half
// as long.
template <class Fn>
void with_gu_shape(int64_t S, int64_t max_slots, Fn&& fn) {
  using std::integral_constant;
  if (S == 8 && max_slots >= 64)
    fn(integral_constant<int, 1>{}, integral_constant<int, 4>{}, integral_constant<int, 8>{},
       integral_constant<int, 2>{});
  else
    with_gu_depth(S, [&](auto sc) {
      fn(integral_constant<int, 2>{}, integral_constant<int, 2>{}, sc,
         integral_constant<int, 1>{});
    });
}

// ---------------------------------------------------------------------------------------
// MoE routing (transformers qwen3_next semantics): softmax over the E routed logits in fp32,
// top-k (ties to the lower expert id), renormalised; the logit in column E is the shared
// expert's gate, applied as sigmoid. Wave m routes row m with the row's logits in registers
// (expert e = lane + 64 i), k rounds of a wave arg-max.
//
// MoE plan: the unique experts the block touches in ascending id (a ballot prefix count over
// the 256 expert flags), the (row, k) pair of each row routed to each, then the shared expert
// as the last slot. Routing and plan run in one block so the ids never leave LDS.
// ---------------------------------------------------------------------------------------
constexpr int ROUTE_THREADS = 1024;  // 16 waves: one per row (M <= 16), four for the plan

// Top-k of E <= 256 logits (expert e = lane + 64 i) in descending order with ties to the
// lower expert id, and the picks' renormalised softmax weights: lane k ends with the k-th
// pick's id and weight. Each lane sorts its four candidates once; a round takes the wave
// maximum of the lanes' heads (left in every lane), the lanes holding it (ballot; on a tie
// the lowest expert id among them) and the winning lane drops its head. The softmax order is
// the logits' order (exp is monotonic, so the picks are the same), and the renormalised
// weight of pick k is p_k / sum_j p_j = e^(v_k - v_0) / sum_j e^(v_j - v_0) (v_0 the largest
// logit): the full softmax sum cancels, so it is never formed.
__device__ __forceinline__ void route_row(const float* __restrict__ l, int E, int topk, int lane,
                                          float& my_w, int& my_id) {
  uint32_t key[4];  // ordered keys; 0 = past E
  uint32_t id[4];
  {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = l[lane + 64 * i < E ? lane + 64 * i : 0];  // all in flight
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      key[i] = e < E ? ord_key(v[i]) : 0u;
      id[i] = (uint32_t)e;
    }
  }
  // sort the lane's candidates: key descending, then id ascending (a five-comparator network
  // under that total order)
  auto cswap = [&](int a, int b) {
    // bitwise, not short-circuit: no branches
    const bool sw = (key[b] > key[a]) | ((key[b] == key[a]) & (id[b] < id[a]));
    const uint32_t ka = key[a], ia = id[a];
    key[a] = sw ? key[b] : key[a];
    id[a] = sw ? id[b] : id[a];
    key[b] = sw ? ka : key[b];
    id[b] = sw ? ia : id[b];
  };
  cswap(0, 1); cswap(2, 3); cswap(0, 2); cswap(1, 3); cswap(1, 2);
  my_id = -1;
  uint32_t my_key = 0u;  // lane k: the k-th pick's key
  for (int k = 0; k < topk; ++k) {
    const uint32_t km = wave_max_u32_all(key[0]);
    const uint64_t tied = __ballot(key[0] == km);
    int wl;  // the winning lane: the only one holding km, else the one with the lowest id
    if (__popcll(tied) == 1)
      wl = (int)__builtin_ctzll(tied);
    else
      wl = (int)(wave_min_u32_dpp(key[0] == km ? id[0] : 0xffffffffu) & 63u);
    const int e = __builtin_amdgcn_readlane((int)id[0], wl);
    const bool pop = lane == wl;
    key[0] = pop ? key[1] : key[0];
    id[0] = pop ? id[1] : id[0];
    key[1] = pop ? key[2] : key[1];
    id[1] = pop ? id[2] : id[1];
    key[2] = pop ? key[3] : key[2];
    id[2] = pop ? id[3] : id[2];
    key[3] = pop ? 0u : key[3];
    my_key = lane == k ? km : my_key;
    my_id = lane == k ? e : my_id;
  }
  // weights over the picks (lanes < topk <= 16, all in the first row of 16 lanes)
  const float v0 = ord_key_to_float((uint32_t)__builtin_amdgcn_readlane((int)my_key, 0));
  const float ek = lane < topk ? __expf(ord_key_to_float(my_key) - v0) : 0.f;
  float ks = ek;
  ks += __uint_as_float(dpp_u32<DPP_QUAD_XOR1>(__float_as_uint(ks)));
  ks += __uint_as_float(dpp_u32<DPP_QUAD_XOR2>(__float_as_uint(ks)));
  ks += __uint_as_float(dpp_u32<DPP_HALF_MIRROR>(__float_as_uint(ks)));
  ks += __uint_as_float(dpp_u32<DPP_MIRROR>(__float_as_uint(ks)));
  my_w = lane < topk ? ek / ks : 0.f;
}

// Inclusive sum over the wave's lanes (lane order).
__device__ __forceinline__ int wave_incl_sum(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    v += lane >= d ? o : 0;
  }
  return v;
}

// Plan from the expert row masks (mask[e] bit r: block row r is routed to expert e; complete
// and visible to every thread) and the picks ids_s[M * topk] in LDS; ep_prev = g_moe_epoch,
// loaded by the caller. Expert e of c rows takes ceil(c / 16) consecutive slots, experts in
// ascending id; every wave forms the slots' prefix over the 256 experts itself (four groups of
// 64, a wave sum each), so slots need no exchange between waves: waves 0-3 write the expert
// slots, waves 4-11 the (row, pick) lists, waves 12-13 the shared expert's rows, all at once.
// Needs ROUTE_THREADS threads.
__device__ __forceinline__ void plan_from_masks(const int32_t* ids_s, int M, int topk, int E,
                                               int shared, const uint64_t* mask, uint32_t ep_prev,
                                               MoePlan* __restrict__ plan) {
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint64_t below = (1ull << lane) - 1ull;
  uint64_t mk[4], bal[4];
  int cnt[4];
  bool multi = false;  // some expert routed more than 16 rows (uniform)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mk[i] = lane + 64 * i < E ? mask[lane + 64 * i] : 0ull;
    bal[i] = __ballot(mk[i] != 0ull);
    cnt[i] = __popcll(bal[i]);
    if (M > 16) multi |= __ballot(__popcll(mk[i]) > 16) != 0ull;
  }
  int base[4];  // first slot of expert lane + 64 i
  int n_routed = 0;
  if (!multi) {
    // one slot per used expert: the slot is the number of used experts below (ballots)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      base[i] = n_routed + __popcll(bal[i] & below);
      n_routed += cnt[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = (__popcll(mk[i]) + 15) >> 4;
      const int incl = wave_incl_sum(v, lane);
      base[i] = n_routed + incl - v;
      n_routed += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  const int n_shared = shared ? (M + 15) >> 4 : 0;
  if (w < 4) {
    // expert e = t: its slots, 16 of its rows each
    const uint64_t me = w == 0 ? mk[0] : w == 1 ? mk[1] : w == 2 ? mk[2] : mk[3];
    const int b = w == 0 ? base[0] : w == 1 ? base[1] : w == 2 ? base[2] : base[3];
    const int c = __popcll(me);
    for (int j = 0; 16 * j < c; ++j) {
      plan->slot_expert[b + j] = t;
      plan->slot_rows[b + j] = c - 16 * j < 16 ? c - 16 * j : 16;
    }
    if (t == 0) {
      const uint32_t ep = (ep_prev + 1u) != 0u ? ep_prev + 1u : 1u;  // skips 0
      g_moe_epoch = ep;
      plan->epoch = ep;
      plan->n_routed = n_routed;
      for (int j = 0; j < n_shared; ++j) {
        plan->slot_expert[n_routed + j] = E;
        plan->slot_rows[n_routed + j] = M - 16 * j < 16 ? M - 16 * j : 16;
      }
      plan->n_slots = n_routed + n_shared;
    }
  } else if (w < 12) {
    // pick p: its row's position among the rows routed to its expert, then that position's slot
    const int p = t - 256;
    const int e = p < M * topk ? ids_s[p] : -1;
    int b = 0;  // the first slot of expert e
    if (!multi) {
      if (e >= 0 && e < E) {
        const int g = e >> 6;
        const uint64_t bg = g == 0 ? bal[0] : g == 1 ? bal[1] : g == 2 ? bal[2] : bal[3];
        b = (g > 0 ? cnt[0] : 0) + (g > 1 ? cnt[1] : 0) + (g > 2 ? cnt[2] : 0) +
            __popcll(bg & ((1ull << (e & 63)) - 1ull));
      }
    } else {
      // every lane takes part in the exchanges: the base from lane e % 64 of group e / 64
      const int src = e >= 0 ? (e & 63) : 0;
      int bg[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bg[i] = __shfl(base[i], src, 64);
      const int g = e >= 0 ? e >> 6 : 0;
      b = g == 0 ? bg[0] : g == 1 ? bg[1] : g == 2 ? bg[2] : bg[3];
    }
    if (e >= 0 && e < E) {
      const int r = p / topk;
      const int pos = __popcll(mask[e] & ((1ull << r) - 1ull));
      const int sl = b + (pos >> 4);
      plan->row_of[sl][pos & 15] = r;
      plan->pair_of[sl][pos & 15] = p;
    }
  } else if (w < 14 && shared) {
    const int r = t - 768;
    if (r < M) {
      plan->row_of[n_routed + (r >> 4)][r & 15] = r;
      plan->pair_of[n_routed + (r >> 4)][r & 15] = -1;
    }
  }
}

__global__ void __launch_bounds__(ROUTE_THREADS) moe_route_plan_kernel(
    const float* __restrict__ logits, int64_t stride, int M, int E, int topk,
    float* __restrict__ weights, int32_t* __restrict__ ids, float* __restrict__ shared_w,
    MoePlan* __restrict__ plan) {
  __shared__ int32_t ids_s[MOE_MAX_PICKS];
  __shared__ uint64_t mask[256];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t ep_prev = plan ? g_moe_epoch : 0u;
  if (t < 256) mask[t] = 0ull;
  __syncthreads();
  for (int row = w; row < M; row += ROUTE_THREADS / 64) {  // wave w: rows w, w + 16, ...
    const float* l = logits + (int64_t)row * stride;
    const float gate = shared_w ? l[E] : 0.f;
    float my_w;
    int my_id;
    route_row(l, E, topk, lane, my_w, my_id);
    if (lane < topk) {
      weights[row * topk + lane] = my_w;
      ids[row * topk + lane] = my_id;
      ids_s[row * topk + lane] = my_id;
      if (my_id >= 0 && my_id < E)
        atomicOr((unsigned long long*)&mask[my_id], 1ull << row);
    }
    if (lane == 0 && shared_w) shared_w[row] = 1.0f / (1.0f + __expf(-gate));
  }
  if (!plan) return;
  __syncthreads();
  plan_from_masks(ids_s, M, topk, E, shared_w != nullptr, mask, ep_prev, plan);
}

__global__ void __launch_bounds__(ROUTE_THREADS) moe_plan_kernel(const int32_t* __restrict__ ids,
                                                                int M, int topk, int E, int shared,
                                                                MoePlan* __restrict__ plan) {
  __shared__ int32_t ids_s[MOE_MAX_PICKS];
  __shared__ uint64_t mask[256];
  const int t = threadIdx.x;
  const uint32_t ep_prev = g_moe_epoch;
  if (t < 256) mask[t] = 0ull;
  const int e = t < M * topk ? ids[t] : -1;
  if (t < M * topk) ids_s[t] = e;
  __syncthreads();
  if (e >= 0 && e < E) atomicOr((unsigned long long*)&mask[e], 1ull << (t / topk));
  __syncthreads();
  plan_from_masks(ids_s, M, topk, E, shared, mask, ep_prev, plan);
}

// ---------------------------------------------------------------------------------------
// The post-attention block of a MoE layer up to the experts in one launch: residual update +
// RMSNorm + the experts' operand conversion (norm_prep_kernel), the router GEMV over the
// normalised rows (dense_gemv, bf16 weights) and the routing + plan (moe_route_plan_kernel).
// One workgroup per 16 router columns; every workgroup normalises all M rows itself into LDS
// (the same sums in the same order as norm_prep_kernel: the thread of word t of a row is
// lane t % 64 of the row's wave t / 64), with its router weights in flight behind the rows, and
// workgroup j < 16 also writes row j of res_out, y_out and the operand workspace. The logits go out with
// device-scope stores; the last workgroup to count itself in (an atomic counter, no wait)
// reads them back with device-scope loads and routes and plans the block, then clears the
// counter for the next launch. Every result has the bits of the three separate launches.
// Launches on one device must be stream-ordered (library-owned counter).
// ---------------------------------------------------------------------------------------
constexpr int NR_THREADS = 1024;  // 16 waves: one per routed row; the GEMV takes dense_gemv's
constexpr int NR_MAXP = 8;        // row passes held in registers (M <= 8 * 8192 / H)
constexpr int NR_MAX_LDS = 128 * 1024;  // dynamic LDS beside the ~27 KiB of static arrays
__device__ uint32_t g_router_arrive;

// (The arguments the first loads need come first: they arrive preloaded in SGPRs.)
__global__ void __launch_bounds__(NR_THREADS) norm_router_plan_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ gamma, const u32x4* __restrict__ router, int M, int H, int E,
    int topk, float eps, uint16_t* __restrict__ res_out, uint16_t* __restrict__ y_out,
    void* __restrict__ ws, size_t tile_bytes, float* __restrict__ logits,
    float* __restrict__ weights, int32_t* __restrict__ ids, float* __restrict__ shared_w,
    MoePlan* __restrict__ plan) {
  // router rows: the E experts, then the shared expert's gate when shared_w is given
  extern __shared__ __attribute__((aligned(16))) uint8_t nr_lds[];  // y rows, H + 8 apart
  __shared__ float part_ss[NR_MAXP][NR_THREADS / 64];
  __shared__ floatx4 part[NR_THREADS / 64][64];
  __shared__ uint32_t last;
  __shared__ int32_t ids_s[MOE_MAX_PICKS];
  __shared__ uint64_t mask[256];
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int kq = lane >> 4, r = lane & 15;
  const int S = H / QK, N = E + (shared_w ? 1 : 0);
  const int ystride = H + 8;  // bf16 elements between the LDS rows (a row's 16 B reads spread)
  uint16_t* ylds = (uint16_t*)nr_lds;
  // this workgroup's router tile: dense_gemv's waves (8 from 8 superblocks, else 4) take
  // superblocks s = wave, wave + NWG, ...
  const int NWG = S >= 8 ? 8 : 4;
  const int tile = blockIdx.x;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(router + (int64_t)tile * S * 8 * 64), 0, S * 8 * 64 * 16, 0x00020000);
  u32x4 wb[8];

  // residual + RMSNorm of every row: RP rows per pass, wpr = H / 8 threads per row (whole
  // waves: H % 512 == 0); every pass's words are loaded before any sum (one round trip), the
  // passes' sums meet in one barrier. The four waves of a SIMD issue this prologue one after
  // another, so it is kept short: shifts when wpr is a power of two, bounds-checked buffer
  // loads (rows past M read as zero) at one vector offset per pass.
  const int wpr = H >> 3;
  int tr, rsub, RP;
  if ((wpr & (wpr - 1)) == 0) {  // uniform
    const int lg = __builtin_ctz(wpr);
    rsub = t >> lg, tr = t & (wpr - 1), RP = NR_THREADS >> lg;
  } else {
    rsub = t / wpr, tr = t - rsub * wpr, RP = NR_THREADS / wpr;
  }
  const int wpw = wpr >> 6;  // waves per row
  const uint32_t rbytes = (uint32_t)(M * H * 2), pstride = (uint32_t)(RP * H * 2);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, rbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)residual, 0, residual ? rbytes : 0u, 0x00020000);
  const uint32_t voff = (uint32_t)(rsub * H + tr * 8) * 2;
  // gamma: the first row group's waves load it and pass it on through LDS (every row group
  // needs the same words)
  __shared__ u32x4 gam_s[4096 / 8];
  u32x4 gv = {0u, 0u, 0u, 0u};
  if (rsub == 0) gv = *(const u32x4*)(gamma + (int64_t)tr * 8);  // wave-uniform
  u32x4 xv[NR_MAXP], rv[NR_MAXP];
#pragma unroll
  for (int p = 0; p < NR_MAXP; ++p) {
    if (p * RP >= M) break;  // uniform; passes <= NR_MAXP (host-checked)
    xv[p] = bload4(xr, voff + p * pstride, 0u);
    rv[p] = bload4(rr, voff + p * pstride, 0u);
  }
  // the router weights behind the rows (the norm needs only the rows); every wave issues the
  // same eight loads (out of the buffer's range, so reading nothing, in the waves without a
  // superblock) so that the rows' wait below is vmcnt(8) in every wave
  {
    const uint32_t wvo = wv < NWG && wv < S ? (uint32_t)lane * 16 : 0x80000000u;
#pragma unroll
    for (int j = 0; j < 8; ++j) wb[j] = bload4(wr, wvo, (uint32_t)((wv * 8 + j) * 64 * 16));
  }
  __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));  // vmcnt(8): the rows, not the weights
  if (rsub == 0) gam_s[tr] = gv;
#pragma unroll
  for (int p = 0; p < NR_MAXP; ++p) {
    if (p * RP >= M) break;  // uniform
    if (residual) xv[p] = add_bf16_words(xv[p], rv[p]);
    const uint32_t vw[4] = {xv[p].x, xv[p].y, xv[p].z, xv[p].w};
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __uint_as_float(vw[i] << 16), b = __uint_as_float(vw[i] & 0xffff0000u);
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) part_ss[p][wv] = ss;
  }
  __syncthreads();
  gv = gam_s[tr];
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
  auto normalise = [&](const u32x4& v, float inv, uint32_t (&yo)[4], float (&y)[8]) {
    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      yo[i] = pack_bf16x2(__uint_as_float(vw[i] << 16) * inv * __uint_as_float(gw[i] << 16),
                          __uint_as_float(vw[i] & 0xffff0000u) * inv *
                              __uint_as_float(gw[i] & 0xffff0000u));
      y[2 * i] = __uint_as_float(yo[i] << 16);
      y[2 * i + 1] = __uint_as_float(yo[i] & 0xffff0000u);
    }
  };
  // workgroup j writes row j's results (the 16 rows of the operand tile over 16 workgroups;
  // the first workgroup writes them all when there are fewer)
  auto owns = [&](int row) { return gridDim.x >= 16 ? row == (int)blockIdx.x : blockIdx.x == 0; };
#pragma unroll
  for (int p = 0; p < NR_MAXP; ++p) {
    if (p * RP >= M) break;  // uniform
    const int row = p * RP + rsub;
    if (row >= M) break;  // uniform: the last pass's row groups past M
    float tot = 0.f;
    for (int w = 0; w < wpw; ++w) tot += part_ss[p][rsub * wpw + w];
    const float inv = __frsqrt_rn(tot / (float)H + eps);
    float y[8];
    uint32_t yo[4];
    normalise(xv[p], inv, yo, y);
    *(u32x4*)(ylds + row * ystride + tr * 8) = u32x4{yo[0], yo[1], yo[2], yo[3]};
    if (owns(row)) {  // wave-uniform
      const int64_t off = (int64_t)row * H + (int64_t)tr * 8;
      if (res_out) *(u32x4*)(res_out + off) = xv[p];
      if (y_out) *(u32x4*)(y_out + off) = u32x4{yo[0], yo[1], yo[2], yo[3]};
      if (row < 16) word_operand(y, tr, row, ws, tile_bytes, H / QK, true);
    }
  }
  // the tile's rows past M get zero operands, as norm_prep_kernel writes them
  for (int row0 = 0; row0 < 16; row0 += RP) {  // uniform
    const int row = row0 + rsub;
    if (row >= M && row < 16 && owns(row)) {
      float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      word_operand(y, tr, row, ws, tile_bytes, H / QK, true);
    }
  }
  __syncthreads();  // the rows are in LDS

  // router GEMV from the LDS rows (dense_gemv's bf16 form: the same products and sums)
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = wv; wv < NWG && s < S; s += NWG) {
    if (s != wv)
#pragma unroll
      for (int j = 0; j < 8; ++j) wb[j] = bload4(wr, lane * 16, (uint32_t)((s * 8 + j) * 64 * 16));
    u32x4 xa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      xa[j] = r < M ? *(const u32x4*)(ylds + r * ystride + s * QK + j * 32 + kq * 8)
                    : u32x4{0u, 0u, 0u, 0u};
    floatx4 sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j)
      sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[j]),
                                                   __builtin_bit_cast(bf16x8, wb[j]), sb, 0, 0, 0);
    acc += sb * floatx4{1.f, 1.f, 1.f, 1.f};
  }
  if (wv < NWG) part[wv][lane] = acc;
  __syncthreads();
  if (wv == 0) {
    floatx4 v = part[0][lane];
    for (int ww = 1; ww < NWG; ++ww) v += part[ww][lane];
    const int n = tile * TILE_N + (lane & 15);
    const int rb = 4 * (lane >> 4);
    if (n < N)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rb + i < M)
          __hip_atomic_store(logits + (int64_t)(rb + i) * N + n, v[i], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  // count in once this workgroup's logits have been written; the last one routes and plans
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (t == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(&g_router_arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (!last) return;
  if (t == 0) __hip_atomic_store(&g_router_arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // every workgroup's logits, back through LDS (the y rows are no longer needed)
  float* lg = (float*)nr_lds;
  constexpr int LG_PER = (16 * 257 + NR_THREADS - 1) / NR_THREADS;  // all loads in flight
  float lv[LG_PER];
#pragma unroll
  for (int k = 0; k < LG_PER; ++k) {
    const int i = t + k * NR_THREADS;
    lv[k] = i < M * N ? __hip_atomic_load(logits + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0.f;
  }
#pragma unroll
  for (int k = 0; k < LG_PER; ++k)
    if (t + k * NR_THREADS < M * N) lg[t + k * NR_THREADS] = lv[k];
  if (t < 256) mask[t] = 0ull;
  const uint32_t ep_prev = g_moe_epoch;
  __syncthreads();
  // moe_route_plan_kernel's routing, wave w on row w
  for (int row = wv; row < M; row += NR_THREADS / 64) {
    const float* l = lg + row * N;
    const float gate = shared_w ? l[E] : 0.f;
    float my_w;
    int my_id;
    route_row(l, E, topk, lane, my_w, my_id);
    if (lane < topk) {
      weights[row * topk + lane] = my_w;
      ids[row * topk + lane] = my_id;
      ids_s[row * topk + lane] = my_id;
      if (my_id >= 0 && my_id < E)
        atomicOr((unsigned long long*)&mask[my_id], 1ull << row);
    }
    if (lane == 0 && shared_w) shared_w[row] = 1.0f / (1.0f + __expf(-gate));
  }
  __syncthreads();
  plan_from_masks(ids_s, M, topk, E, shared_w != nullptr, mask, ep_prev, plan);
}

// ---------------------------------------------------------------------------------------
// MoE down: per (tile group, slot) the down GEMV of the slot's expert over its compact
// activation rows [n_rows, F] (converted to fp16 operands in-kernel), with the weights of the
// next superblock in flight during the current one. Routed rows are written pre-weighted into
// pairs [M*topk, H] f32 at their pair index; the shared expert's rows, weighted by
// sigmoid(gate), into shared_out [M, H].
// ---------------------------------------------------------------------------------------
template <int FMT, int NTILE, bool DEVICE_SCOPE>
__device__ __forceinline__ void act_operands(SbOperands<FMT, NTILE>& o, const uint16_t* a, int F,
                                             int n_rows, int s, int lane) {
  XOperands xo;
  if constexpr (DEVICE_SCOPE) {
    // device-scope loads (sc1): rows another workgroup of this launch has just published
    const int r = lane & 15, kq = lane >> 4;
    const __amdgpu_buffer_rsrc_t ar =
        __builtin_amdgcn_make_buffer_rsrc((void*)a, 0, 16 * F * 2, 0x00020000);
    const uint32_t vo = r < n_rows ? (uint32_t)((r * F + kq * 8) * 2) : 0x80000000u;
    u32x4 raw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      raw[j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, vo, (uint32_t)((s * QK + j * 32) * 2),
                                                       16 /* sc1 */));
    convert_words(raw, lane, xo);
  } else {
    convert_superblock(a, F, n_rows, s, lane, xo);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) o.x[j] = xo.x[j];
  o.sx0 = xo.sx0;
  o.sx1 = xo.sx1;
  // per-row scales of rows 4 kq .. 4 kq + 3 live in lanes 4 kq + i (kq = 0 row group)
  const int kq = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) o.scale[i] = __shfl(xo.scale, 4 * kq + i, 64);
}

template <int FMT, int NTILE, int WS, bool DEVICE_SCOPE>
__device__ __forceinline__ void down_loop(const GemvStreams& st, const uint16_t* a, int F,
                                          int n_rows, int w, int S, int tile0, int lane,
                                          uint32_t Mv, floatx4* acc) {
  if (w >= S) return;
  const int kq = lane >> 4;
  SbOperands<FMT, NTILE> bufA, bufB;
  load_sb<FMT, NTILE, false>(bufA, st, w, S, tile0, 1);
  for (int s = w;;) {
    if (s + WS < S) load_sb<FMT, NTILE, false>(bufB, st, s + WS, S, tile0, 1);
    act_operands<FMT, NTILE, DEVICE_SCOPE>(bufA, a, F, n_rows, s, lane);
    gemv_superblock<FMT, NTILE>(bufA, acc, kq, Mv);
    s += WS;
    if (s >= S) break;
    if (s + WS < S) load_sb<FMT, NTILE, false>(bufA, st, s + WS, S, tile0, 1);
    act_operands<FMT, NTILE, DEVICE_SCOPE>(bufB, a, F, n_rows, s, lane);
    gemv_superblock<FMT, NTILE>(bufB, acc, kq, Mv);
    s += WS;
    if (s >= S) break;
  }
}

// bx: the block's tile-group index; slot: the plan slot. DEVICE_SCOPE: the activations are read
// with device-scope loads. ONE_SB: F / QK == WS, one superblock per wave (no second operand
// buffer, so fewer registers). wait(): called once by every wave before the activations are
// read (in the one-superblock form, with the wave's weights already in flight); it returns
// true (the same in every wave) when the activations were never published, and the item then
// writes NaN to every output it owns, so that a failed hand-off cannot pass as a result.
template <int FMT, int NTILE, int WS, int GPB, bool DEVICE_SCOPE, bool ONE_SB, class Wait>
__device__ __forceinline__ void moe_down_body(
    int bx, int slot, const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta,
    int64_t dn_qbytes, int64_t dn_mbytes, const uint8_t* __restrict__ sh_quant,
    const uint8_t* __restrict__ sh_meta, const MoePlan* __restrict__ plan, int E,
    const uint16_t* __restrict__ act, const float* __restrict__ weights,
    const float* __restrict__ shared_w, float* __restrict__ pairs,
    float* __restrict__ shared_out, int H, int F, Wait&& wait) {
  __shared__ floatx4 part[GPB][WS][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gl = wv / WS, sw = wv % WS;
  if (slot >= plan->n_slots) return;
  const int e = plan->slot_expert[slot];
  const int n_rows = plan->slot_rows[slot];
  const uint8_t* q = e >= E ? sh_quant : quant + e * dn_qbytes;
  const uint8_t* m = e >= E ? sh_meta : meta + e * dn_mbytes;
  const int S = F / QK;
  const int tiles = H / TILE_N;
  const int tile0 = (bx * GPB + gl) * NTILE;
  const GemvStreams st = make_streams<FMT>(q, m, nullptr, tiles, S, lane, 16);
  const uint32_t Mv = decode_magic<FMT>();
  // the epilogue's destinations and gates for this lane's compact rows, fetched up front
  const int rb = 4 * (lane >> 4);
  int dst[4];
  float gate[4];
  auto fetch_epilogue = [&]() {
    const int32_t* ids = e >= E ? plan->row_of[slot] : plan->pair_of[slot];
    const float* gsrc = e >= E ? shared_w : weights;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = rb + i < n_rows ? ids[rb + i] : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) gate[i] = rb + i < n_rows ? gsrc[dst[i]] : 0.f;
  };
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint16_t* slot_act = act + (int64_t)slot * 16 * F;
  bool poisoned = false;
  if constexpr (ONE_SB) {
    // one superblock per wave (S == WS): its weights go out first, then the epilogue's
    // operands, then the activations
    const bool live = tile0 < tiles && sw < S;
    SbOperands<FMT, NTILE> o;
    if (live) load_sb<FMT, NTILE, false>(o, st, sw, S, tile0, 1);
    fetch_epilogue();
    poisoned = wait();
    if (live) {
      act_operands<FMT, NTILE, DEVICE_SCOPE>(o, slot_act, F, n_rows, sw, lane);
      gemv_superblock<FMT, NTILE>(o, acc, lane >> 4, Mv);
    }
  } else {
    fetch_epilogue();
    poisoned = wait();
    if (tile0 < tiles)
      down_loop<FMT, NTILE, WS, DEVICE_SCOPE>(st, slot_act, F, n_rows, sw, S, tile0, lane, Mv,
                                              acc);
  }
  if constexpr (WS > 1) {
#pragma unroll
    for (int t = 0; t < NTILE; ++t) part[gl][sw][t][lane] = acc[t];
    __syncthreads();
    if (sw != 0) return;
#pragma unroll
    for (int t = 0; t < NTILE; ++t) {
      acc[t] = part[gl][0][t][lane];
#pragma unroll
      for (int j = 1; j < WS; ++j) acc[t] += part[gl][j][t][lane];
    }
  }
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const int tile = tile0 + t;
    if (tile >= tiles) break;
    const int n = tile * TILE_N + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (rb + i >= n_rows) break;  // compact row
      const float y = bf16_to_f32(f32_to_bf16(acc[t][i]));  // expert outputs are bf16 tensors
      float* out = e >= E ? shared_out : pairs;
      out[(int64_t)dst[i] * H + n] = poisoned ? __builtin_nanf("") : y * gate[i];
    }
  }
}

// Down item of the one-launch experts kernel with four tiles and all SD superblocks per wave
// (four waves: sixteen tiles of 16 output columns): each wave's weights, SD times those of a
// one-superblock item, go out before the wait, so that twice as many down weights stream
// while the gate/up items run, and the slot's activations are loaded once per workgroup: wave
// s < SD loads superblock s of the compact rows straight into LDS (device-scope loads) and
// converts it there, one chunk at a time, with convert_words' arithmetic. The superblocks'
// products are added in order, s = 0 first: each is an exact product by a power of two, so
// the sum is the one the two-wave item forms (the same bits). The meta words are loaded one
// dword per lane and gathered across the column's four lanes at multiply time.
typedef __attribute__((address_space(3))) void lds_void;
constexpr int DN_WIDE_TILES = 4;  // tiles per wave of a wide down item

template <int FMT, int SD, class Wait>
__device__ __forceinline__ void moe_down_wide_body(
    int bx, int slot, const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta,
    int64_t dn_qbytes, int64_t dn_mbytes, const uint8_t* __restrict__ sh_quant,
    const uint8_t* __restrict__ sh_meta, const MoePlan* __restrict__ plan, int E,
    const uint16_t* __restrict__ act, const float* __restrict__ weights,
    const float* __restrict__ shared_w, float* __restrict__ pairs,
    float* __restrict__ shared_out, int H, Wait&& wait) {
  constexpr int DT = DN_WIDE_TILES, F = SD * QK;
  constexpr int QV = QLayout<FMT>::kQuantVecs;
  __shared__ u32x4 xs[SD][8][64];  // fp16 A operands of the slot's activation superblocks
  __shared__ float xs_sum[SD][2][64];
  __shared__ floatx4 xs_scale[SD][64];
  __shared__ int32_t ep_dst[16];
  __shared__ float ep_gate[16];
  const int lane = threadIdx.x & 63, kq = lane >> 4, r = lane & 15;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (slot >= plan->n_slots) return;
  const int e = __builtin_amdgcn_readfirstlane(plan->slot_expert[slot]);
  const int n_rows = __builtin_amdgcn_readfirstlane(plan->slot_rows[slot]);
  const uint8_t* q = e >= E ? sh_quant : quant + e * dn_qbytes;
  const uint8_t* m = e >= E ? sh_meta : meta + e * dn_mbytes;
  const int tiles = H / TILE_N, tile0 = (bx * 4 + wv) * DT;
  const GemvStreams st = make_streams<FMT>(q, m, nullptr, tiles, SD, lane, 16);
  u32x4 wq[SD][DT][QV];
  uint32_t wm[SD][DT];
  uint32_t wd[SD][DT];
#pragma unroll
  for (int s = 0; s < SD; ++s) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const uint32_t ts = (uint32_t)((tile0 + t) * SD + s);
      constexpr uint32_t TB = QLayout<FMT>::kTsBytes;
      if constexpr (FMT == FMT_Q5_K) {
        wq[s][t][0] = bload4(st.quant, st.v_quant, ts * TB);
        wq[s][t][1] = bload4(st.quant, st.v_quant, ts * TB + 1024);
        const u32x2 h = bload2(st.quant, st.v_quant >> 1, ts * TB + 2048);
        wq[s][t][2] = u32x4{h.x, h.y, 0u, 0u};
      } else {
#pragma unroll
        for (int i = 0; i < QV; ++i) wq[s][t][i] = bload4(st.quant, st.v_quant, ts * TB + i * 1024);
      }
      wm[s][t] = bload1u(st.meta, st.v_meta + kq * 4, ts * 16 * 16);  // dword kq of column r
    }
    if constexpr (FMT == FMT_Q6_K) load_sb_d<DT>(wd[s], st, s, SD, tile0, 1);
  }
  // the epilogue's destinations and gates of the slot's compact rows
  if (wv == 1 && lane < 16) {
    const int32_t* ids = e >= E ? plan->row_of[slot] : plan->pair_of[slot];
    const float* gsrc = e >= E ? shared_w : weights;
    const int d = lane < n_rows ? ids[lane] : 0;
    ep_dst[lane] = d;
    ep_gate[lane] = lane < n_rows ? gsrc[d] : 0.f;
  }
  const bool poisoned = wait();  // ends with a workgroup barrier
  if (wv < SD) {
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(act + (int64_t)slot * 16 * F), 0, 16 * F * 2, 0x00020000);
    const uint32_t vo = r < n_rows ? (uint32_t)((r * F + kq * 8) * 2) : 0x80000000u;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void*)&xs[wv][j][0], 16, vo,
                                               (uint32_t)((wv * QK + j * 32) * 2), 0,
                                               16 /* sc1: device scope */);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    float sx0, sx1, sc;
    convert_chunks([&](int j) { return xs[wv][j][lane]; },
                   [&](int j, u32x4 v) { xs[wv][j][lane] = v; }, lane, sx0, sx1, sc);
    xs_sum[wv][0][lane] = sx0;
    xs_sum[wv][1][lane] = sx1;
    floatx4 rs;
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[i] = __shfl(sc, 4 * kq + i, 64);  // rows 4 kq + i
    xs_scale[wv][lane] = rs;
  }
  __syncthreads();
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < SD; ++s) {
    SbOperands<FMT, DT> o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o.x[j] = xs[s][j][lane];
    o.sx0 = xs_sum[s][0][lane];
    o.sx1 = xs_sum[s][1][lane];
    o.scale = xs_scale[s][lane];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int i = 0; i < QV; ++i) o.q[t][i] = wq[s][t][i];
      o.m[t] = u32x4{(uint32_t)__shfl((int)wm[s][t], r, 64),
                     (uint32_t)__shfl((int)wm[s][t], r + 16, 64),
                     (uint32_t)__shfl((int)wm[s][t], r + 32, 64),
                     (uint32_t)__shfl((int)wm[s][t], r + 48, 64)};
      o.dq[t] = wd[s][t];
    }
    gemv_superblock<FMT, DT>(o, acc, kq, Mv);
  }
  float* out = e >= E ? shared_out : pairs;
  const int rb = 4 * kq;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (rb + i >= n_rows) break;  // compact row
    const int64_t d = ep_dst[rb + i];
    const float gt = ep_gate[rb + i];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int n = (tile0 + t) * TILE_N + (lane & 15);
      const float y = bf16_to_f32(f32_to_bf16(acc[t][i]));  // expert outputs are bf16 tensors
      out[d * H + n] = poisoned ? __builtin_nanf("") : y * gt;
    }
  }
}

template <int FMT, int NTILE, int WS, int GPB, bool ONE_SB>
__global__ void __launch_bounds__(WS * GPB * 64) moe_down_kernel(
    const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta, int64_t dn_qbytes,
    int64_t dn_mbytes, const uint8_t* __restrict__ sh_quant, const uint8_t* __restrict__ sh_meta,
    const MoePlan* __restrict__ plan, int E, const uint16_t* __restrict__ act,
    const float* __restrict__ weights, const float* __restrict__ shared_w,
    float* __restrict__ pairs, float* __restrict__ shared_out, int H, int F) {
  moe_down_body<FMT, NTILE, WS, GPB, false, ONE_SB>(blockIdx.x, blockIdx.y, quant, meta, dn_qbytes,
                                            dn_mbytes, sh_quant, sh_meta, plan, E, act, weights,
                                            shared_w, pairs, shared_out, H, F,
                                            [] { return false; });
}

// ---------------------------------------------------------------------------------------
// Gate/up and down of every slot in one launch. Workgroups 0 .. GU-1 run gate/up items
// (slot-major), the rest down items (slot-major). A gate/up item stores its activations with
// device-scope stores and, once every wave's stores have completed, writes the plan's epoch
// into its flag in each of its slot's down items' flag lines; a down item waits until the
// flags of all of its slot's gate/up items hold the epoch in its own line, clears them and
// reads the activations with device-scope loads. Each line has one reader, so nothing is
// counted and no address is contended.
//
// Progress: every gate/up item has a lower workgroup index than every down item, and
// workgroups are dispatched in index order (per XCD, and so overall for the ones an XCD
// holds), so when a gate/up item waits for a CU slot, every workgroup holding one on its XCD
// has a lower index: a gate/up item, which waits for nothing. Every gate/up item therefore
// runs, and every wait ends. The wait is bounded all the same: on a time-out the down item
// records g_moe_error and writes NaN instead of its outputs.
//
// Ordering: the activation stores and loads are device-scope (sc1) and the flags are
// device-scope atomics; each gate/up wave waits for its stores' completion (vmcnt(0)) before
// the barrier that precedes the flag store, and a down item issues its activation loads only
// after its flag loads returned the epoch. The epoch comes from the plan, so a flag left set by
// a gate/up item that finished after its down item gave up never matches a later plan; the
// clear lets a plan be run twice. The flags are library-owned: launches of this kernel on one
// device must be stream-ordered.
// ---------------------------------------------------------------------------------------
constexpr int MOE_MAX_ITEMS = 32;  // gate/up or down items per slot
__device__ __align__(256) uint32_t g_moe_flags[MOE_MAX_SLOTS][MOE_MAX_ITEMS][MOE_MAX_ITEMS];
__device__ uint32_t g_moe_error;
constexpr uint32_t MOE_WAIT_POLLS = 1u << 20;  // ~0.1 s: far beyond any gate/up item

// Three waves per SIMD when the down items take one superblock per wave (the gate/up items then
// bound the registers at 168); two otherwise.
template <int FMT, int DN_FMT, int GU_WS, int GU_PPB, int GU_SC, int GU_VW, int DN_NTILE,
          int DN_WS, int DN_GPB, bool ONE_SB, int WAVES = (ONE_SB ? 3 : 2), bool DN_WIDE = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES))) moe_experts_kernel(
    // first the arguments of the plan read and the gate/up weight addresses: the first 56
    // bytes arrive preloaded in SGPRs
    const MoePlan* __restrict__ plan, const uint8_t* __restrict__ gu_quant,
    const uint8_t* __restrict__ gu_meta, int64_t gu_qbytes, int64_t gu_mbytes, int gu_per_slot,
    int dn_per_slot, int max_slots, int E, const uint8_t* __restrict__ sh_gu_quant,
    const uint8_t* __restrict__ sh_gu_meta, const uint8_t* __restrict__ dn_quant,
    const uint8_t* __restrict__ dn_meta, int64_t dn_qbytes, int64_t dn_mbytes,
    const uint8_t* __restrict__ sh_dn_quant, const uint8_t* __restrict__ sh_dn_meta,
    const void* __restrict__ ws, uint16_t* __restrict__ act, const float* __restrict__ weights,
    const float* __restrict__ shared_w, float* __restrict__ pairs,
    float* __restrict__ shared_out, int M, int H, int F) {
  static_assert(GU_WS * GU_PPB * 64 == 256 && DN_WS * DN_GPB * 64 == 256, "256-thread items");
  const int item = blockIdx.x;
  const int n_gu = gu_per_slot * max_slots;
  const int n_slots = plan->n_slots;
  const uint32_t epoch = plan->epoch;
  if (item < n_gu) {
    const int slot = item / gu_per_slot;
    if (slot >= n_slots) return;
    gate_up_body<FMT, GU_WS, GU_PPB, true, GU_SC, GU_VW>(item % gu_per_slot, slot, gu_quant, gu_meta,
                                           gu_qbytes, gu_mbytes, sh_gu_quant, sh_gu_meta, plan,
                                           E, ws, act, M, F, H / QK);
    // every wave waits for its own activation stores to complete (the barrier alone does not
    // wait for stores), then one count publishes the item
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if ((int)threadIdx.x < dn_per_slot)
      __hip_atomic_store(&g_moe_flags[slot][threadIdx.x][item % gu_per_slot], epoch,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // slot and item index are wave-uniform: keep them scalar so that the weight offsets derived
  // from them stay scalar through the divergent wait below
  const int d = item - n_gu;
  const int slot = __builtin_amdgcn_readfirstlane(d / dn_per_slot);
  const int didx = __builtin_amdgcn_readfirstlane(d % dn_per_slot);
  if (slot >= n_slots) return;
  // the wait for the slot's gate/up items, once the item's weights are in flight
  __shared__ uint32_t timed_out;
  auto wait = [&]() -> bool {
    if (threadIdx.x == 0) timed_out = 0u;  // wave 0 holds every polling lane
    if ((int)threadIdx.x < gu_per_slot) {  // one lane per gate/up item of the slot
      uint32_t* flag = &g_moe_flags[slot][didx][threadIdx.x];
      uint32_t polls = 0;
      while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) {
        if (++polls == MOE_WAIT_POLLS) {
          __hip_atomic_store(&g_moe_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          timed_out = 1u;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // sole reader
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(timed_out) != 0u;
  };
  if constexpr (DN_WIDE)
    moe_down_wide_body<DN_FMT, 2>(didx, slot, dn_quant, dn_meta, dn_qbytes, dn_mbytes,
                                  sh_dn_quant, sh_dn_meta, plan, E, act, weights, shared_w,
                                  pairs, shared_out, H, wait);
  else
    moe_down_body<DN_FMT, DN_NTILE, DN_WS, DN_GPB, true, ONE_SB>(
        didx, slot, dn_quant, dn_meta, dn_qbytes, dn_mbytes, sh_dn_quant, sh_dn_meta,
        plan, E, act, weights, shared_w, pairs, shared_out, H, F, wait);
}

// out[r, n] = bf16(sum_k pairs[r*topk + k, n] + shared_out[r, n]) in a fixed order
__global__ void moe_combine_kernel(const float* __restrict__ pairs,
                                   const float* __restrict__ shared_out, uint16_t* __restrict__ out,
                                   int M, int H, int topk) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * H) return;
  const int64_t r = i / H, n = i % H;
  float acc = 0.f;
  for (int k = 0; k < topk; ++k) acc += pairs[(r * topk + k) * H + n];
  if (shared_out) acc += shared_out[i];
  out[i] = f32_to_bf16(acc);
}

int launch_norm_prep(const void* x, MoeSource ms, const void* res_in, void* res_out,
                     const void* gamma, void* y_out, void* ws, int64_t M, int64_t H, float eps,
                     hipStream_t s) {
  const int64_t S = H / 256, mt = (M + 15) / 16;
  const int threads = (int)((H / 8 + 63) / 64 * 64);
  hipLaunchKernelGGL(norm_prep_kernel, dim3((unsigned)(mt * 16)), dim3(threads), 0, s,
                     (const uint16_t*)x, (const uint16_t*)res_in, (const uint16_t*)gamma,
                     ms.pairs, ms.shared, (int)M, (int)H, ms.topk, eps, ms.x_out,
                     (uint16_t*)res_out, (uint16_t*)y_out, ws, xprep_tile_bytes(S));
  SV_CHECK_LAUNCH();
  return SV_OK;
}

template <int WT, int NTILE, int NW>
int launch_dense(const void* w, const void* act, void* c, int M, int N, int S, int c_bf16,
                 hipStream_t s) {
  const int tiles = (N + TILE_N - 1) / TILE_N;
  const int row_tiles = (M + TILE_M - 1) / TILE_M;
  const size_t tb = xprep_tile_bytes(S);
  const int groups = (tiles + NTILE - 1) / NTILE;
  if (row_tiles == 1 || groups < 64)
    // one row tile per workgroup: a narrow output (the router's 17 tiles) then still has
    // workgroups for several CUs (the same sums per row tile)
    hipLaunchKernelGGL((dense_gemv<WT, NTILE, NW, 1>), dim3(groups, row_tiles), dim3(NW * 64), 0,
                       s, (const u32x4*)w, act, c, M, N, S, c_bf16, tb);
  else if (row_tiles == 2)
    hipLaunchKernelGGL((dense_gemv<WT, NTILE, NW, 2>), dim3((tiles + NTILE - 1) / NTILE),
                       dim3(NW * 64), 0, s, (const u32x4*)w, act, c, M, N, S, c_bf16, tb);
  else
    hipLaunchKernelGGL((dense_gemv<WT, NTILE, NW, DENSE_MT>),
                       dim3((tiles + NTILE - 1) / NTILE, (row_tiles + DENSE_MT - 1) / DENSE_MT),
                       dim3(NW * 64), 0, s, (const u32x4*)w, act, c, M, N, S, c_bf16, tb);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

}  // namespace

// =======================================================================================
// C ABI (extensions; the reference reaches these through its snowllm_inference_* entry
// points, snowllm/_capi.py:687-692, with internal workspaces)
// =======================================================================================

// Residual update + RMSNorm + operand conversion for the k-quant GEMVs: res_out = x + res_in
// (x alone when res_in is null), y = RMSNorm(res_out) * gamma. All bf16 [M, H], H <= 8192;
// res_in, res_out and y_out may be null. Each element is read and written by one thread, so
// res_out and y_out may alias x or res_in (in-place residual update). ws as for
// snowllm_gemm_kquant_a.
SV_API int snowverify_norm_prep(const void* x, const void* res_in, void* res_out,
                                const void* gamma, void* y_out, void* ws, int64_t M, int64_t H,
                                float eps, void* stream) {
  if (M <= 0 || H <= 0 || H % 256 || H > 8 * NORM_MAX_THREADS) return SV_EINVAL;
  return launch_norm_prep(x, MoeSource{nullptr, nullptr, nullptr, 0}, res_in, res_out, gamma,
                          y_out, ws, M, H, eps, Sx(stream));
}

// snowverify_norm_prep on the MoE layer's output without materialising it first: x =
// bf16(sum_k pairs[r * topk + k] + shared_out[r]) (as snowverify_moe_combine), written to
// x_out if given. pairs [M*topk, H] f32, shared_out [M, H] f32 or null.
SV_API int snowverify_norm_prep_moe(const float* pairs, const float* shared_out, int64_t topk,
                                    void* x_out, const void* res_in, void* res_out,
                                    const void* gamma, void* y_out, void* ws, int64_t M,
                                    int64_t H, float eps, void* stream) {
  if (!pairs || topk <= 0 || M <= 0 || H <= 0 || H % 256 || H > 8 * NORM_MAX_THREADS)
    return SV_EINVAL;
  if (x_out && (x_out == res_out || x_out == y_out)) return SV_EINVAL;
  return launch_norm_prep(nullptr, MoeSource{pairs, shared_out, (uint16_t*)x_out, (int)topk},
                          res_in, res_out, gamma, y_out, ws, M, H, eps, Sx(stream));
}

// snowverify_norm_prep (x + res_in -> res_out, RMSNorm * gamma -> y_out and the operand
// workspace ws) + snowverify_dense_gemv (bf16 router [E (+1), H] repacked, over the normalised
// rows, f32 logits [M, E (+1)]) + snowverify_moe_route with the plan, in one launch and with
// their bits. shared_w null: no shared expert (E router rows). M <= 16, H a multiple of 512 up
// to 4096 with M * (H + 8) * 2 <= 128 KiB, E <= 256, topk <= 16. Uses a library-owned
// counter: calls on one device must be stream-ordered.
SV_API int snowverify_norm_router_plan(const void* x, const void* res_in, void* res_out,
                                       const void* gamma, float eps, void* ws, void* y_out,
                                       const void* router, float* logits, int64_t M, int64_t H,
                                       int64_t E, int64_t topk, float* weights, int32_t* ids,
                                       float* shared_w, void* plan, void* stream) {
  if (!x || !gamma || !ws || !router || !logits || !weights || !ids || !plan || M <= 0 ||
      M > 16 || H <= 0 || H % 512 || H > 4096 || E <= 0 || E > 256 || topk <= 0 || topk > 16 ||
      topk > E)
    return SV_EINVAL;
  if (res_out && (res_out == x || res_out == res_in)) return SV_EINVAL;  // read by every block
  const int64_t N = E + (shared_w ? 1 : 0);
  const size_t lds = std::max((size_t)(M * (H + 8) * 2), (size_t)(M * N * 4));
  if (lds > NR_MAX_LDS || (M + 8192 / H - 1) / (8192 / H) > NR_MAXP) return SV_ENOTSUP;
  if (lds > 65536) {
    // beyond the default dynamic LDS limit (16 rows of H = 2048 with their padding): raise
    // the kernel's limit once, up to the CU's 160 KiB
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
      attr = hipFuncSetAttribute((const void*)norm_router_plan_kernel,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, NR_MAX_LDS);
    });
    if (attr != hipSuccess) return (int)attr;
  }
  hipLaunchKernelGGL(norm_router_plan_kernel, dim3((unsigned)((N + TILE_N - 1) / TILE_N)),
                     dim3(NR_THREADS), lds, Sx(stream), (const uint16_t*)x,
                     (const uint16_t*)res_in, (const uint16_t*)gamma, (const u32x4*)router,
                     (int)M, (int)H, (int)E, (int)topk, eps, (uint16_t*)res_out,
                     (uint16_t*)y_out, ws, xprep_tile_bytes(H / 256), logits, weights, ids,
                     shared_w, (MoePlan*)plan);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Bytes of a repacked 16-bit weight [N, K] (N padded to a multiple of 16).
SV_API int64_t snowverify_dense_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % 256) return -1;
  return ((N + 15) / 16) * 16 * K * 2;
}

// Repack a row-major 16-bit weight [N, K] (wt 1 = fp16, 2 = bf16) for snowverify_dense_gemv.
SV_API int snowverify_dense_shuffle(const void* src, void* dst, int64_t N, int64_t K, int wt,
                                    void* stream) {
  if (N <= 0 || K <= 0 || K % 256 || (wt != WT_F16 && wt != WT_BF16)) return SV_EINVAL;
  const int64_t total = ((N + 15) / 16) * (K / 256) * 8 * 64;
  hipLaunchKernelGGL(dense_shuffle_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     Sx(stream), (const uint16_t*)src, (uint16_t*)dst, N, K, wt);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// C[M, N] = A[M, K] W[N, K]^T, fp32 accumulate. wt 1: fp16 weights against the operand
// workspace `act` (snowverify_gemm_kquant_prepare_a / snowverify_norm_prep, one 16-row tile
// after the other); wt 2: bf16 weights against bf16 activations `act` [M, K]. M <= 256: a
// workgroup multiplies each weight tile against up to four row tiles.
SV_API int snowverify_dense_gemv(int wt, const void* w, const void* act, void* c, int64_t M,
                                 int64_t N, int64_t K, int c_is_bf16, void* stream) {
  if (M <= 0 || M > DENSE_MAX_M || N <= 0 || K <= 0 || K % 256) return SV_EINVAL;
  // 32-bit in-kernel offsets: one block's weights (<= 2 tiles) and the activations
  if (N > (int64_t)1 << 30 || K > 65536) return SV_ENOTSUP;
  const int S = (int)(K / 256);
  hipStream_t s = Sx(stream);
  if (wt == WT_F16) {
    if (S >= 8) return launch_dense<WT_F16, 2, 8>(w, act, c, (int)M, (int)N, S, c_is_bf16, s);
    return launch_dense<WT_F16, 2, 4>(w, act, c, (int)M, (int)N, S, c_is_bf16, s);
  }
  if (wt == WT_BF16) {
    if (S >= 8) return launch_dense<WT_BF16, 1, 8>(w, act, c, (int)M, (int)N, S, c_is_bf16, s);
    return launch_dense<WT_BF16, 1, 4>(w, act, c, (int)M, (int)N, S, c_is_bf16, s);
  }
  return SV_EINVAL;
}

// Dense SwiGLU MLP front half: act[M, F] = silu(x Wg^T) * (x Wu^T) with gate_up the packed
// [2F, K] k-quant weight (gate rows first) and ws the prepared operands of x. M <= 16.
SV_API int snowverify_gate_up_swiglu(int fmt, const void* quant, const void* meta, const void* ws,
                                     void* act, int64_t M, int64_t F, int64_t K, void* stream) {
  if ((fmt != 4 && fmt != 5 && fmt != 6 && fmt != 8) || M <= 0 || M > 16 || F <= 0 || F % 16 ||
      K % 256)
    return SV_EINVAL;
  const int S = (int)(K / 256);
  hipStream_t s = Sx(stream);
  // two pairs per workgroup, two waves per pair: at FFN 14336 the 448 workgroups are all
  // resident at once (two per CU at most), where one pair on four waves left 896 workgroups, a
  // round and three quarters (measured at BASELINE config 3: 22.4 -> 20.6 us per call, step
  // 3.266 -> 3.182 ms; eight waves per pair: 26.2 us)
  constexpr int WS = 2, PPB = 2;
  const dim3 grid((unsigned)((F / 16 + PPB - 1) / PPB), 1);
  with_gu_depth(S, [&](auto sc_c) {
    constexpr int SC = decltype(sc_c)::value;
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(64 * WS * PPB), 0, s, (const uint8_t*)quant,
                         (const uint8_t*)meta, 0, 0, nullptr, nullptr, nullptr, 0, ws,
                         (uint16_t*)act, (int)M, (int)F, S);
    };
    if (fmt == 4) go(gate_up_kernel<4, WS, PPB, SC>);
    else if (fmt == 5) go(gate_up_kernel<5, WS, PPB, SC>);
    else if (fmt == 6) go(gate_up_kernel<6, WS, PPB, SC>);
    else go(gate_up_kernel<8, WS, PPB, SC>);
  });
  SV_CHECK_LAUNCH();
  return SV_OK;
}

SV_API int64_t snowverify_moe_plan_bytes(void) { return (int64_t)sizeof(MoePlan); }

// The most slots a plan of M rows with topk picks each can take (an expert with more than 16
// rows takes one slot per 16; the shared expert ceil(M / 16)): the max_slots the expert
// launches need, and the slots of their activation scratch [slots, 16, F]. 0 past the limits.
SV_API int64_t snowverify_moe_max_slots(int64_t M, int64_t topk, int64_t E, int shared) {
  if (M <= 0 || M > MOE_MAX_M || topk <= 0 || M * topk > MOE_MAX_PICKS || E <= 0 || E > 256)
    return 0;
  return moe_plan_slots(M, topk, E, shared != 0);
}

// Plan the block's experts from top-k ids [M, topk] (i32). M <= 64, M * topk <= 512, E <= 256.
SV_API int snowverify_moe_plan(const int32_t* ids, int64_t M, int64_t topk, int64_t E, int shared,
                               void* plan, void* stream) {
  if (M <= 0 || M > MOE_MAX_M || topk <= 0 || M * topk > MOE_MAX_PICKS || E <= 0 || E > 256)
    return SV_EINVAL;
  hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(ROUTE_THREADS), 0, Sx(stream), ids, (int)M,
                     (int)topk, (int)E, shared, (MoePlan*)plan);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// MoE routing from router logits [M, stride] f32 (E routed columns, then the shared expert's
// gate in column E when shared_w is given): weights/ids [M, topk], shared_w [M].
SV_API int snowverify_moe_route(const float* logits, int64_t stride, int64_t M, int64_t E,
                                int64_t topk, float* weights, int32_t* ids, float* shared_w,
                                void* stream) {
  if (M < 0 || M > MOE_MAX_M || E <= 0 || E > 256 || topk <= 0 || topk > 16 || topk > E ||
      M * topk > MOE_MAX_PICKS || stride < E + (shared_w ? 1 : 0))
    return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipLaunchKernelGGL(moe_route_plan_kernel, dim3(1), dim3(ROUTE_THREADS), 0, Sx(stream), logits,
                     stride, (int)M, (int)E, (int)topk, weights, ids, shared_w, nullptr);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Routing and plan in one launch (the plan's shared slot exists when shared_w is given).
SV_API int snowverify_moe_route_plan(const float* logits, int64_t stride, int64_t M, int64_t E,
                                     int64_t topk, float* weights, int32_t* ids, float* shared_w,
                                     void* plan, void* stream) {
  if (M <= 0 || M > MOE_MAX_M || E <= 0 || E > 256 || topk <= 0 || topk > 16 || topk > E ||
      M * topk > MOE_MAX_PICKS || stride < E + (shared_w ? 1 : 0) || !plan)
    return SV_EINVAL;
  hipLaunchKernelGGL(moe_route_plan_kernel, dim3(1), dim3(ROUTE_THREADS), 0, Sx(stream), logits,
                     stride, (int)M, (int)E, (int)topk, weights, ids, shared_w, (MoePlan*)plan);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// MoE expert stages (Q4_K, Q5_K, Q6_K). act scratch [max_slots, 16, F] bf16 (compact rows
// per slot; max_slots from snowverify_moe_max_slots). M <= 64 block rows.
// Each tile pair (gate/up) or tile group (down) splits its superblocks over two waves: a launch
// then holds about twice the waves of one per pair, so the few workgroups that do not fit the
// first round over the CUs (more than 64 expert slots) finish in half the time (measured on
// MI355X: 30.0 -> 27.2 us gate/up, 25.1 -> 21.5 us down at 65 slots; +0.7 us at 57).
// Expert formats the MoE kernels take, and one packed expert matrix's bytes (the stacks hold
// expert e at e * these).
extern "C" int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K);
extern "C" int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K);
namespace {
bool expert_fmt(int f) { return f == 4 || f == 5 || f == 6; }
int64_t packed_quant(int f, int64_t N, int64_t K) { return snowllm_kquant_quant_bytes(f, N, K) - 4; }
int64_t packed_meta(int f, int64_t N, int64_t K) { return snowllm_kquant_meta_bytes(f, N, K); }
}  // namespace

constexpr int MOE_GU_WS = 2, MOE_GU_PPB = 2;             // gate/up: waves per pair, pairs per block
constexpr int MOE_DN_NTILE = 4, MOE_DN_WS = 2, MOE_DN_GPB = 2;  // down: tiles per group, waves
                                                                 // per group, groups per block

// Gate/up + SwiGLU of every slot of the plan; ws: prepared operands of the normalised hidden.
SV_API int snowverify_moe_gate_up(int fmt, const void* gu_quant, const void* gu_meta,
                                  const void* sh_gu_quant, const void* sh_gu_meta,
                                  const void* plan, const void* ws, void* act, int64_t M,
                                  int64_t max_slots, int64_t E, int64_t H, int64_t F,
                                  void* stream) {
  if (!expert_fmt(fmt) || M <= 0 || M > MOE_MAX_M || max_slots <= 0 ||
      max_slots > MOE_MAX_SLOTS || H % 256 || F % 256)
    return SV_EINVAL;
  const int64_t gu_q = packed_quant(fmt, 2 * F, H), gu_m = packed_meta(fmt, 2 * F, H);
  with_gu_shape(H / 256, max_slots, [&](auto ws_c, auto ppb_c, auto sc_c, auto vw_c) {
    constexpr int WS = decltype(ws_c)::value, PPB = decltype(ppb_c)::value,
                  SC = decltype(sc_c)::value, VW = decltype(vw_c)::value;
    const dim3 grid((unsigned)(F / 16 / PPB), (unsigned)max_slots);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(64 * WS * PPB), 0, Sx(stream),
                         (const uint8_t*)gu_quant, (const uint8_t*)gu_meta, gu_q, gu_m,
                         (const uint8_t*)sh_gu_quant, (const uint8_t*)sh_gu_meta,
                         (const MoePlan*)plan, (int)E, ws, (uint16_t*)act, (int)M, (int)F,
                         (int)(H / 256));
    };
    if (fmt == 4) go(gate_up_kernel<4, WS, PPB, SC, VW>);
    else if (fmt == 5) go(gate_up_kernel<5, WS, PPB, SC, VW>);
    else go(gate_up_kernel<6, WS, PPB, SC, VW>);
  });
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Down GEMV of every slot: routed rows pre-weighted into pairs [M*topk, H] f32, shared rows
// into shared_out [M, H] f32.
SV_API int snowverify_moe_down(int fmt, const void* dn_quant, const void* dn_meta,
                               const void* sh_dn_quant, const void* sh_dn_meta, const void* plan,
                               const void* act, const float* weights, const float* shared_w,
                               float* pairs, float* shared_out, int64_t max_slots, int64_t E,
                               int64_t H, int64_t F, void* stream) {
  if (!expert_fmt(fmt) || max_slots <= 0 || max_slots > MOE_MAX_SLOTS || H % 256 || F % 256)
    return SV_EINVAL;
  const int64_t dn_q = packed_quant(fmt, H, F), dn_m = packed_meta(fmt, H, F);
  const int groups = (int)(H / 16 / MOE_DN_NTILE);
  const dim3 grid((unsigned)((groups + MOE_DN_GPB - 1) / MOE_DN_GPB), (unsigned)max_slots);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64 * MOE_DN_WS * MOE_DN_GPB), 0, Sx(stream),
                       (const uint8_t*)dn_quant, (const uint8_t*)dn_meta, dn_q, dn_m,
                       (const uint8_t*)sh_dn_quant, (const uint8_t*)sh_dn_meta,
                       (const MoePlan*)plan, (int)E, (const uint16_t*)act, weights, shared_w,
                       pairs, shared_out, (int)H, (int)F);
  };
  auto by = [&](auto f) {
    constexpr int D = decltype(f)::value;
    if (F / QK == MOE_DN_WS) launch(moe_down_kernel<D, MOE_DN_NTILE, MOE_DN_WS, MOE_DN_GPB, true>);
    else launch(moe_down_kernel<D, MOE_DN_NTILE, MOE_DN_WS, MOE_DN_GPB, false>);
  };
  if (fmt == 4) by(std::integral_constant<int, 4>{});
  else if (fmt == 5) by(std::integral_constant<int, 5>{});
  else by(std::integral_constant<int, 6>{});
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// snowverify_moe_gate_up followed by snowverify_moe_down in one launch, with the same outputs
// and bits (max_slots = M * topk + shared). Uses library-owned flags: calls on one device
// must be stream-ordered.
SV_API int snowverify_moe_gate_up_down(int fmt, const void* gu_quant, const void* gu_meta,
                                       const void* dn_quant, const void* dn_meta,
                                       const void* sh_gu_quant, const void* sh_gu_meta,
                                       const void* sh_dn_quant, const void* sh_dn_meta,
                                       const void* plan, const void* ws, const float* weights,
                                       const float* shared_w, void* act, float* pairs,
                                       float* shared_out, int64_t M, int64_t max_slots,
                                       int64_t E, int64_t H, int64_t F, void* stream) {
  const int gu_fmt = fmt & 0xff, dn_fmt = (fmt >> 8) ? ((fmt >> 8) & 0xff) : gu_fmt;
  if (!expert_fmt(gu_fmt) || !expert_fmt(dn_fmt) || M <= 0 || M > MOE_MAX_M || max_slots <= 0 ||
      max_slots > MOE_MAX_SLOTS || H % 256 || F % 256 || (F / 16) % MOE_GU_PPB ||
      (H / 16 / MOE_DN_NTILE) % MOE_DN_GPB)
    return SV_EINVAL;
  const int64_t gu_q = packed_quant(gu_fmt, 2 * F, H), gu_m = packed_meta(gu_fmt, 2 * F, H);
  const int64_t dn_q = packed_quant(dn_fmt, H, F), dn_m = packed_meta(dn_fmt, H, F);
  const int dn_per_slot = (int)(H / 16 / MOE_DN_NTILE / MOE_DN_GPB);
  if (F / 16 / MOE_GU_PPB > MOE_MAX_ITEMS || dn_per_slot > MOE_MAX_ITEMS) return SV_ENOTSUP;
  // gu_per_slot: F / 16 pairs over the item shape's pairs per block (at most MOE_GU_PPB's)
  auto launch = [&](auto kern, int gu_per_slot, int dn_items = -1) {
    const int dn = dn_items >= 0 ? dn_items : dn_per_slot;
    const int64_t blocks = (int64_t)(gu_per_slot + dn) * max_slots;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, Sx(stream),
                       (const MoePlan*)plan, (const uint8_t*)gu_quant, (const uint8_t*)gu_meta,
                       gu_q, gu_m, gu_per_slot, dn, (int)max_slots, (int)E,
                       (const uint8_t*)sh_gu_quant, (const uint8_t*)sh_gu_meta,
                       (const uint8_t*)dn_quant, (const uint8_t*)dn_meta, dn_q, dn_m,
                       (const uint8_t*)sh_dn_quant, (const uint8_t*)sh_dn_meta, ws,
                       (uint16_t*)act, weights, shared_w, pairs, shared_out, (int)M, (int)H,
                       (int)F);
  };
  // Q4_K pairs: three waves per SIMD (168 registers); formats with wider weight operands
  // (Q5_K's qh, Q6_K's third vector) at two
  auto pick = [&](auto gu, auto dn) {
    constexpr int G = decltype(gu)::value, D = decltype(dn)::value;
    constexpr bool q4 = G == 4 && D == 4;
    with_gu_shape(H / QK, max_slots, [&](auto ws_c, auto ppb_c, auto sc_c, auto vw_c) {
      constexpr int WS = decltype(ws_c)::value, PPB = decltype(ppb_c)::value,
                    SC = decltype(sc_c)::value, VW = decltype(vw_c)::value;
      // launches of 128 or more slots (16 or more rows): wide down items, half as many,
      // twice the down weights in flight while the gate/up items run (measured at 180 slots:
      // 75.1 -> 70.9 us; at 53-83 slots one-superblock items are ahead by up to 2 us)
      if constexpr (D != 6) {
        if (max_slots >= 128 && F / QK == 2 && (H / TILE_N) % (4 * DN_WIDE_TILES) == 0) {
          launch(moe_experts_kernel<G, D, WS, PPB, SC, VW, DN_WIDE_TILES, 1, 4, true,
                                    q4 ? 3 : 2, true>,
                 (int)(F / 16 / PPB), (int)(H / TILE_N / (4 * DN_WIDE_TILES)));
          return;
        }
      }
      if (F / QK == MOE_DN_WS)
        launch(moe_experts_kernel<G, D, WS, PPB, SC, VW, MOE_DN_NTILE, MOE_DN_WS, MOE_DN_GPB,
                                  true, q4 ? 3 : 2>,
               (int)(F / 16 / PPB));
      else
        launch(moe_experts_kernel<G, D, WS, PPB, SC, VW, MOE_DN_NTILE, MOE_DN_WS, MOE_DN_GPB,
                                  false, 2>,
               (int)(F / 16 / PPB));
    });
    return SV_OK;
  };
  using I4 = std::integral_constant<int, 4>;
  using I5 = std::integral_constant<int, 5>;
  using I6 = std::integral_constant<int, 6>;
  if (gu_fmt == 4 && dn_fmt == 4) pick(I4{}, I4{});
  else if (gu_fmt == 4 && dn_fmt == 5) pick(I4{}, I5{});
  else if (gu_fmt == 4 && dn_fmt == 6) pick(I4{}, I6{});
  else if (gu_fmt == 5 && dn_fmt == 5) pick(I5{}, I5{});
  else if (gu_fmt == 5 && dn_fmt == 6) pick(I5{}, I6{});
  else if (gu_fmt == 6 && dn_fmt == 6) pick(I6{}, I6{});
  else return SV_ENOTSUP;  // down below gate/up precision: not a GGUF mix
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Non-zero if a launch of snowverify_moe_gate_up_down ever timed out waiting for its
// activations (a bug, never expected); reading it blocks on the device.
SV_API int snowverify_moe_sync_error(void) {
  uint32_t v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_moe_error), sizeof(v), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return -1;
  return (int)v;
}

// out [M, H] bf16 = sum_k pairs[r * topk + k] (+ shared_out[r]) in a fixed order.
SV_API int snowverify_moe_combine(const float* pairs, const float* shared_out, void* out,
                                  int64_t M, int64_t topk, int64_t H, void* stream) {
  if (M <= 0 || topk <= 0 || H <= 0) return SV_EINVAL;
  const int64_t n = M * H;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     Sx(stream), pairs, shared_out, (uint16_t*)out, (int)M, (int)H, (int)topk);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// MoE experts of one layer: gate/up, down and combine. ws: prepared operands of the normalised
// hidden [M, H] (M <= 64); act scratch [snowverify_moe_max_slots(M, topk, E, shared), 16, F]
// bf16; pairs [M*topk, H] f32;
// shared_out [M, H] f32; out [M, H] bf16 = sum_k w_k expert_k(x) + sigmoid(g) shared(x).
SV_API int snowverify_moe_experts(int fmt, const void* gu_quant, const void* gu_meta,
                                  const void* dn_quant, const void* dn_meta, const void* sh_gu_quant,
                                  const void* sh_gu_meta, const void* sh_dn_quant,
                                  const void* sh_dn_meta, const void* plan, const void* ws,
                                  const float* weights, const float* shared_w, void* act,
                                  float* pairs, float* shared_out, void* out, int64_t M,
                                  int64_t topk, int64_t E, int64_t H, int64_t F, void* stream) {
  const int64_t slots = snowverify_moe_max_slots(M, topk, E, sh_gu_quant != nullptr);
  if (slots <= 0) return SV_EINVAL;
  const int gu_fmt = fmt & 0xff, dn_fmt = (fmt >> 8) ? ((fmt >> 8) & 0xff) : gu_fmt;
  int rc = snowverify_moe_gate_up(gu_fmt, gu_quant, gu_meta, sh_gu_quant, sh_gu_meta, plan, ws, act,
                                  M, slots, E, H, F, stream);
  if (rc != SV_OK) return rc;
  rc = snowverify_moe_down(dn_fmt, dn_quant, dn_meta, sh_dn_quant, sh_dn_meta, plan, act, weights,
                           shared_w, pairs, shared_out, slots, E, H, F, stream);
  if (rc != SV_OK) return rc;
  return snowverify_moe_combine(pairs, sh_gu_quant ? shared_out : nullptr, out, M, topk, H, stream);
}
