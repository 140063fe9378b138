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

namespace {
using namespace kq;

inline hipStream_t Sx(void* s) { return (hipStream_t)s; }

// ---------------------------------------------------------------------------------------
// residual + RMSNorm + operand conversion. One wave per (row tile, superblock): every wave
// computes the row statistics over the full row (a few KiB from L2) and converts its own
// superblock. v = bf16(x + res_in) (v = x without res_in) is written to res_out by the wave
// owning those columns (res_out must not alias x or res_in: other waves still read them),
// y = bf16(v * inv * gamma), optional bf16 copy of y, fp16 operands of y into the workspace.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) norm_prep_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ res_out, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ y_out, void* __restrict__ ws, size_t tile_bytes, int64_t M, int64_t H,
    float eps) {
  const int s = blockIdx.x, tile = blockIdx.y;
  const int lane = threadIdx.x, r = lane & 15, kq = lane >> 4;
  const int64_t S = H / QK;
  const int64_t row = (int64_t)tile * TILE_M + r;
  const bool live = row < M;
  // 1) sum of squares of v = bf16(x + residual) over the row (this lane: k = 8 (4 i + kq) ..)
  float ss = 0.f;
  if (live) {
    for (int64_t k0 = kq * 8; k0 < H; k0 += 32) {
      const u32x4 xv = *(const u32x4*)(x + row * H + k0);
      u32x4 rv = {0u, 0u, 0u, 0u};
      if (residual) rv = *(const u32x4*)(residual + row * H + k0);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = __uint_as_float(xw[i] << 16), b = __uint_as_float(xw[i] & 0xffff0000u);
        if (residual) {
          a = bf16_to_f32(f32_to_bf16(a + __uint_as_float(rw[i] << 16)));
          b = bf16_to_f32(f32_to_bf16(b + __uint_as_float(rw[i] & 0xffff0000u)));
        }
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
      }
    }
  }
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  const float inv = __frsqrt_rn(ss / (float)H + eps);
  // 2) this superblock: update residual, normalise, stage bf16 y in LDS for the conversion
  __shared__ uint16_t ybuf[16][QK];
  if (live) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k0 = (int64_t)s * QK + j * 32 + kq * 8;
      const u32x4 xv = *(const u32x4*)(x + row * H + k0);
      u32x4 rv = {0u, 0u, 0u, 0u};
      if (residual) rv = *(const u32x4*)(residual + row * H + k0);
      const u32x4 gv = *(const u32x4*)(gamma + k0);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
      uint32_t nres[4], yw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = __uint_as_float(xw[i] << 16), b = __uint_as_float(xw[i] & 0xffff0000u);
        if (residual) {
          a = bf16_to_f32(f32_to_bf16(a + __uint_as_float(rw[i] << 16)));
          b = bf16_to_f32(f32_to_bf16(b + __uint_as_float(rw[i] & 0xffff0000u)));
        }
        nres[i] = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
        const uint16_t ya = f32_to_bf16(a * inv * __uint_as_float(gw[i] << 16));
        const uint16_t yb = f32_to_bf16(b * inv * __uint_as_float(gw[i] & 0xffff0000u));
        yw[i] = (uint32_t)ya | ((uint32_t)yb << 16);
      }
      if (res_out) *(u32x4*)(res_out + row * H + k0) = u32x4{nres[0], nres[1], nres[2], nres[3]};
      const u32x4 yv = {yw[0], yw[1], yw[2], yw[3]};
      if (y_out) *(u32x4*)(y_out + row * H + k0) = yv;
      *(u32x4*)&ybuf[r][j * 32 + kq * 8] = yv;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) *(u32x4*)&ybuf[r][j * 32 + kq * 8] = u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  // 3) fp16 operands of this superblock (src = ybuf, superblock 0 of a 256-wide row)
  XPrepView v = xprep_view((char*)ws + tile * tile_bytes, S);
  XOperands o;
  convert_superblock(&ybuf[0][0], QK, 16, 0, lane, o);
#pragma unroll
  for (int j = 0; j < 8; ++j) v.xop[((int64_t)s * 8 + j) * 64 + lane] = o.x[j];
  v.sxop[((int64_t)s * 2 + 0) * 64 + lane] = o.sx0;
  v.sxop[((int64_t)s * 2 + 1) * 64 + lane] = o.sx1;
  if (kq == 0) v.scale[(int64_t)s * 16 + r] = o.scale;
}

// ---------------------------------------------------------------------------------------
// GEMV with 16-bit weights. Repacked layout: [tile][s][j][lane][8 halves] holding
// W[16 tile + (lane & 15)][256 s + 32 j + 8 (lane >> 4) + perm(e)] where perm is kperm for fp16
// weights (they meet the fp16 operand workspace) and the identity for bf16 weights (they
// meet bf16 activations read directly).
// ---------------------------------------------------------------------------------------
constexpr int WT_F16 = 1;
constexpr int WT_BF16 = 2;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int WT, int NTILE, int NW>
__global__ void __launch_bounds__(NW * 64) dense_gemv(const u32x4* __restrict__ w,
                                                      const void* __restrict__ act,
                                                      void* __restrict__ c, int M, int N, int S,
                                                      int c_bf16) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4, r = lane & 15;
  const int tiles = (N + TILE_N - 1) / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  const int K = S * QK;
  __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, tiles * S * 8 * 64 * 16, 0x00020000);
  __amdgpu_buffer_rsrc_t xr, sr;
  uint32_t vx, vs;
  if constexpr (WT == WT_F16) {
    XPrepView xv = xprep_view((void*)act, S);
    xr = __builtin_amdgcn_make_buffer_rsrc((void*)xv.xop, 0, S * 8 * 64 * 16, 0x00020000);
    sr = __builtin_amdgcn_make_buffer_rsrc((void*)xv.scale, 0, S * 16 * 4, 0x00020000);
    vx = r < M ? lane * 16 : 0x80000000u;
    vs = kq * 16;
  } else {
    xr = __builtin_amdgcn_make_buffer_rsrc((void*)act, 0, M * K * 2, 0x00020000);
    sr = xr;
    vx = r < M ? (uint32_t)(r * K * 2 + kq * 16) : 0x80000000u;
    vs = 0;
  }
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s = wv; s < S; s += NW) {
    u32x4 xa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (WT == WT_F16) xa[j] = bload4(xr, vx, (uint32_t)((s * 8 + j) * 64 * 16));
      else xa[j] = bload4(xr, vx, (uint32_t)((s * QK + j * 32) * 2));
    }
    floatx4 scale = {1.f, 1.f, 1.f, 1.f};
    if constexpr (WT == WT_F16) scale = __builtin_bit_cast(floatx4, bload4(sr, vs, (uint32_t)(s * 16 * 4)));
    u32x4 wb[NTILE][8];
#pragma unroll
    for (int t = 0; t < NTILE; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        wb[t][j] = bload4(wr, lane * 16, (uint32_t)((((tile0 + t) * S + s) * 8 + j) * 64 * 16));
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
      acc[t] += sb * scale;
    }
  }
  combine_waves<NTILE, NW>(part, acc, wv, lane);
  for (int idx = threadIdx.x; idx < NTILE * 64; idx += NW * 64) {
    const int t = idx >> 6, l = idx & 63;
    const int tile = tile0 + t;
    if (tile >= tiles) continue;
    floatx4 v = part[0][t][l];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) v += part[ww][t][l];
    const int n = tile * TILE_N + (l & 15);
    if (n >= N) continue;
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
struct MoePlan {
  int32_t n_slots;             // routed unique experts + shared expert
  int32_t n_routed;
  int32_t slot_expert[136];    // expert id per slot (E = shared)
  int32_t pair_of[136][16];    // (row * topk + k) routed to the slot's expert, or -1
};

template <int FMT, int NW>
__global__ void __launch_bounds__(NW * 64) gate_up_kernel(
    const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta, int64_t gu_qbytes,
    int64_t gu_mbytes, const uint8_t* __restrict__ sh_quant, const uint8_t* __restrict__ sh_meta,
    const MoePlan* __restrict__ plan, int E, const void* __restrict__ ws,
    uint16_t* __restrict__ act_out, int M, int F, int S) {
  __shared__ floatx4 part[NW][2][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4;
  const int pair = blockIdx.x, slot = blockIdx.y;
  const uint8_t* q = quant;
  const uint8_t* m = meta;
  if (plan) {
    if (slot >= plan->n_slots) return;
    const int e = plan->slot_expert[slot];
    if (e >= E) { q = sh_quant; m = sh_meta; }
    else { q = quant + e * gu_qbytes; m = meta + e * gu_mbytes; }
  }
  const int half_tiles = F / TILE_N;
  const GemvStreams st = make_streams<FMT>(q, m, ws, 2 * half_tiles, S, lane, M);
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
  gemv_loop<FMT, 2, NW>(st, wv, S, pair, half_tiles, kq, Mv, acc);
  combine_waves<2, NW>(part, acc, wv, lane);
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    floatx4 g = part[0][0][l], u = part[0][1][l];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) {
      g += part[ww][0][l];
      u += part[ww][1][l];
    }
    const int n = pair * TILE_N + (l & 15);
    const int rb = 4 * (l >> 4);
    uint16_t* out = plan ? act_out + (int64_t)slot * 16 * F : act_out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rb + i;
      if (!plan && row >= M) break;
      const float gg = bf16_to_f32(f32_to_bf16(g[i]));  // projections are bf16 tensors
      const float uu = bf16_to_f32(f32_to_bf16(u[i]));
      const float a = (row < M) ? gg / (1.0f + __expf(-gg)) * uu : 0.f;
      out[(int64_t)row * F + n] = f32_to_bf16(a);
    }
  }
}

// ---------------------------------------------------------------------------------------
// MoE plan: unique experts touched by the block (ascending id), the (row, k) pair of each
// row routed to each, then the shared expert as the last slot. One block.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) moe_plan_kernel(const int32_t* __restrict__ ids, int M,
                                                       int topk, int E, int shared,
                                                       MoePlan* __restrict__ plan) {
  __shared__ uint32_t mask[256];
  __shared__ int32_t slot_of[256];
  const int t = threadIdx.x;
  for (int e = t; e < 256; e += 256) mask[e] = 0;
  __syncthreads();
  for (int p = t; p < M * topk; p += 256) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicOr(&mask[e], 1u << (p / topk));
  }
  __syncthreads();
  if (t == 0) {
    int n = 0;
    for (int e = 0; e < E; ++e) {
      slot_of[e] = mask[e] ? n : -1;
      if (mask[e]) plan->slot_expert[n++] = e;
    }
    plan->n_routed = n;
    if (shared) plan->slot_expert[n++] = E;
    plan->n_slots = n;
  }
  __syncthreads();
  for (int i = t; i < 136 * 16; i += 256) plan->pair_of[i / 16][i % 16] = -1;
  __syncthreads();
  for (int p = t; p < M * topk; p += 256) {
    const int e = ids[p];
    if (e >= 0 && e < E) plan->pair_of[slot_of[e]][p / topk] = p;
  }
}

// ---------------------------------------------------------------------------------------
// MoE down: per (tile group, slot): converts the slot's activations [16, F] in-kernel, runs the
// down GEMV of that expert and writes routed rows, pre-weighted, into pairs [M*topk, H] f32
// (or the shared expert's rows, weighted by sigmoid(gate), into shared_out [M, H]).
// ---------------------------------------------------------------------------------------
template <int FMT, int NTILE, int NW>
__global__ void __launch_bounds__(NW * 64) moe_down_kernel(
    const uint8_t* __restrict__ quant, const uint8_t* __restrict__ meta, int64_t dn_qbytes,
    int64_t dn_mbytes, const uint8_t* __restrict__ sh_quant, const uint8_t* __restrict__ sh_meta,
    const MoePlan* __restrict__ plan, int E, const uint16_t* __restrict__ act,
    const float* __restrict__ weights, const float* __restrict__ shared_w,
    float* __restrict__ pairs, float* __restrict__ shared_out, int M, int H, int F) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4;
  const int slot = blockIdx.y;
  if (slot >= plan->n_slots) return;
  const int e = plan->slot_expert[slot];
  const uint8_t* q = e >= E ? sh_quant : quant + e * dn_qbytes;
  const uint8_t* m = e >= E ? sh_meta : meta + e * dn_mbytes;
  const int S = F / QK;
  const int tiles = H / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  GemvStreams st = make_streams<FMT>(q, m, nullptr, tiles, S, lane, M);
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint16_t* a = act + (int64_t)slot * 16 * F;
  for (int s = wv; s < S; s += NW) {
    SbOperands<FMT, NTILE> o;
    load_sb<FMT, NTILE, false>(o, st, s, S, tile0, 1);
    XOperands xo;
    convert_superblock(a, F, 16, s, lane, xo);
#pragma unroll
    for (int j = 0; j < 8; ++j) o.x[j] = xo.x[j];
    o.sx0 = xo.sx0;
    o.sx1 = xo.sx1;
    // per-row scales of rows 4 kq .. 4 kq + 3 live in lanes 4 kq + i (kq = 0 row group)
#pragma unroll
    for (int i = 0; i < 4; ++i) o.scale[i] = __shfl(xo.scale, 4 * kq + i, 64);
    gemv_superblock<FMT, NTILE>(o, acc, kq, Mv);
  }
  combine_waves<NTILE, NW>(part, acc, wv, lane);
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
      const float y = bf16_to_f32(f32_to_bf16(v[i]));  // expert outputs are bf16 tensors
      if (e >= E) {
        shared_out[(int64_t)row * H + n] = y * shared_w[row];
      } else {
        const int p = plan->pair_of[slot][row];
        if (p >= 0) pairs[(int64_t)p * H + n] = y * weights[p];
      }
    }
  }
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

template <int WT, int NTILE, int NW>
int launch_dense(const void* w, const void* act, void* c, int M, int N, int S, int c_bf16,
                 hipStream_t s) {
  const int tiles = (N + TILE_N - 1) / TILE_N;
  hipLaunchKernelGGL((dense_gemv<WT, NTILE, NW>), dim3((tiles + NTILE - 1) / NTILE), dim3(NW * 64),
                     0, s, (const u32x4*)w, act, c, M, N, S, c_bf16);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

}  // namespace

// =======================================================================================
// C ABI (extensions; the reference reaches these through its snowllm_inference_* entry
// points, snowllm/_capi.py:687-692, with internal workspaces)
// =======================================================================================

// Residual update + RMSNorm + operand conversion for the k-quant GEMVs: res_out = x + res_in
// (x alone when res_in is null), y = RMSNorm(res_out) * gamma. All bf16 [M, H]; res_in,
// res_out and y_out may be null; res_out must not alias x or res_in. ws as for
// snowllm_gemm_kquant_a.
SV_API int snowverify_norm_prep(const void* x, const void* res_in, void* res_out,
                                const void* gamma, void* y_out, void* ws, int64_t M, int64_t H,
                                float eps, void* stream) {
  if (M <= 0 || H <= 0 || H % 256) return SV_EINVAL;
  if (res_out && (res_out == x || res_out == res_in)) return SV_EINVAL;
  const int64_t S = H / 256, mt = (M + 15) / 16;
  hipLaunchKernelGGL(norm_prep_kernel, dim3((unsigned)S, (unsigned)mt), dim3(64), 0, Sx(stream),
                     (const uint16_t*)x, (const uint16_t*)res_in, (uint16_t*)res_out,
                     (const uint16_t*)gamma, (uint16_t*)y_out, ws, xprep_tile_bytes(S), M, H, eps);
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
// workspace `act` (snowllm_gemm_kquant_prepare_a / snowverify_norm_prep); wt 2: bf16 weights
// against bf16 activations `act` [M, K]. M <= 16.
SV_API int snowverify_dense_gemv(int wt, const void* w, const void* act, void* c, int64_t M,
                                 int64_t N, int64_t K, int c_is_bf16, void* stream) {
  if (M <= 0 || M > 16 || N <= 0 || K <= 0 || K % 256) return SV_EINVAL;
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
  if ((fmt != 4 && fmt != 8) || M <= 0 || M > 16 || F <= 0 || F % 16 || K % 256) return SV_EINVAL;
  const int S = (int)(K / 256);
  hipStream_t s = Sx(stream);
  if (fmt == 4)
    hipLaunchKernelGGL((gate_up_kernel<4, 8>), dim3((unsigned)(F / 16), 1), dim3(512), 0, s,
                       (const uint8_t*)quant, (const uint8_t*)meta, 0, 0, nullptr, nullptr, nullptr,
                       0, ws, (uint16_t*)act, (int)M, (int)F, S);
  else
    hipLaunchKernelGGL((gate_up_kernel<8, 8>), dim3((unsigned)(F / 16), 1), dim3(512), 0, s,
                       (const uint8_t*)quant, (const uint8_t*)meta, 0, 0, nullptr, nullptr, nullptr,
                       0, ws, (uint16_t*)act, (int)M, (int)F, S);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

SV_API int64_t snowverify_moe_plan_bytes(void) { return (int64_t)sizeof(MoePlan); }

// Plan the block's experts from top-k ids [M, topk] (i32). M * topk <= 135, E <= 256, M <= 16.
SV_API int snowverify_moe_plan(const int32_t* ids, int64_t M, int64_t topk, int64_t E, int shared,
                               void* plan, void* stream) {
  if (M <= 0 || M > 16 || topk <= 0 || M * topk > 135 || E <= 0 || E > 256) return SV_EINVAL;
  hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, Sx(stream), ids, (int)M, (int)topk,
                     (int)E, shared, (MoePlan*)plan);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// MoE experts of one layer (Q4_K). ws: prepared operands of the normalised hidden [M, H];
// act scratch [M*topk + 1, 16, F] bf16; pairs [M*topk, H] f32; shared_out [M, H] f32;
// out [M, H] bf16 = sum_k w_k expert_k(x) + sigmoid(g) shared(x).
SV_API int snowverify_moe_experts(int fmt, const void* gu_quant, const void* gu_meta,
                                  const void* dn_quant, const void* dn_meta, const void* sh_gu_quant,
                                  const void* sh_gu_meta, const void* sh_dn_quant,
                                  const void* sh_dn_meta, const void* plan, const void* ws,
                                  const float* weights, const float* shared_w, void* act,
                                  float* pairs, float* shared_out, void* out, int64_t M,
                                  int64_t topk, int64_t E, int64_t H, int64_t F, void* stream) {
  if (fmt != 4 || M <= 0 || M > 16 || M * topk > 135 || H % 256 || F % 256) return SV_EINVAL;
  hipStream_t s = Sx(stream);
  const int64_t gu_q = 2 * F * H / 2, gu_m = 2 * F * (H / 256) * 16;
  const int64_t dn_q = H * F / 2, dn_m = H * (F / 256) * 16;
  const int slots = (int)(M * topk + (sh_gu_quant ? 1 : 0));
  hipLaunchKernelGGL((gate_up_kernel<4, 8>), dim3((unsigned)(F / 16), (unsigned)slots), dim3(512),
                     0, s, (const uint8_t*)gu_quant, (const uint8_t*)gu_meta, gu_q, gu_m,
                     (const uint8_t*)sh_gu_quant, (const uint8_t*)sh_gu_meta, (const MoePlan*)plan,
                     (int)E, ws, (uint16_t*)act, (int)M, (int)F, (int)(H / 256));
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL((moe_down_kernel<4, 4, 2>), dim3((unsigned)(H / 16 / 4), (unsigned)slots),
                     dim3(128), 0, s, (const uint8_t*)dn_quant, (const uint8_t*)dn_meta, dn_q, dn_m,
                     (const uint8_t*)sh_dn_quant, (const uint8_t*)sh_dn_meta, (const MoePlan*)plan,
                     (int)E, (const uint16_t*)act, weights, shared_w, pairs, shared_out, (int)M,
                     (int)H, (int)F);
  SV_CHECK_LAUNCH();
  const int64_t n = M * H;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, pairs,
                     sh_gu_quant ? shared_out : nullptr, (uint16_t*)out, (int)M, (int)H, (int)topk);
  SV_CHECK_LAUNCH();
  return SV_OK;
}
