// QK RMSNorm + rotate-half RoPE of 16 rows of one head, in the layout of an MFMA operand: lane
// (col = row, kq = lane >> 4) holds d = 32 ds + 8 kq + e (ds < D / 32, e < 8), as packed bf16
// words in and out (no fp32 copy of the row is kept). Shared by the
// standalone writer (layer.hip) and the attention kernel that normalises its own query rows and
// the block's keys (attention.hip), so both produce the same bits.
//
// Per row: y = v * rsqrt(mean(v^2) + eps) * gamma in fp32, then for d < 2 half the pair
// (d, d + half) rotates by the row's angle, then one rounding to bf16 (the reference's order,
// tests/test_lfm2_dspark_reference.py:22-27). The sum of squares is taken in a fixed order:
// each lane over its (ds, e) in sequence, then (kq 0 + kq 1) + (kq 2 + kq 3). half is a
// multiple of 32, so a dimension and its rotation partner sit in the same lane (ds and
// ds +- half / 32).
#pragma once
#include "common.h"

// This lane's words of a bf16 row (8 bf16 per sub-block ds, element e in word e / 2, low half
// first), fetched ahead of their use.
template <int D>
struct QkRaw {
  uint32_t w[D / 32][4];
};

// Zeros when !live.
template <int D>
__device__ __forceinline__ void qk_fetch(QkRaw<D>& x, const uint16_t* row, int kq, bool live) {
#pragma unroll
  for (int ds = 0; ds < D / 32; ++ds) {
    x.w[ds][0] = x.w[ds][1] = x.w[ds][2] = x.w[ds][3] = 0u;
    if (live) {
      const uint4 v = *(const uint4*)(row + ds * 32 + kq * 8);
      x.w[ds][0] = v.x; x.w[ds][1] = v.y; x.w[ds][2] = v.z; x.w[ds][3] = v.w;
    }
  }
}

// Element e of a sub-block's words, as fp32.
__device__ __forceinline__ float qk_elem(const uint32_t (&w)[4], int e) {
  return (e & 1) ? __uint_as_float(w[e >> 1] & 0xffff0000u) : __uint_as_float(w[e >> 1] << 16);
}

// The row-independent operands of one lane: gamma's words and the first sub-block's angles
// (used when half > 0), fetched ahead of their use.
template <int D>
struct QkAux {
  uint32_t g[D / 32][4];
  float c[8], s[8];
};

template <int D>
__device__ __forceinline__ void qk_fetch_aux(QkAux<D>& x, const uint16_t* __restrict__ gamma,
                                             const float* cosr, const float* sinr, int half,
                                             int kq) {
#pragma unroll
  for (int ds = 0; ds < D / 32; ++ds) {
    const uint4 g = *(const uint4*)(gamma + ds * 32 + kq * 8);
    x.g[ds][0] = g.x; x.g[ds][1] = g.y; x.g[ds][2] = g.z; x.g[ds][3] = g.w;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) x.c[e] = x.s[e] = 0.f;
  if (half > 0) {
    const float4* cp = (const float4*)(cosr + kq * 8);
    const float4* sp = (const float4*)(sinr + kq * 8);
    const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
    x.c[0] = c0.x; x.c[1] = c0.y; x.c[2] = c0.z; x.c[3] = c0.w;
    x.c[4] = c1.x; x.c[5] = c1.y; x.c[6] = c1.z; x.c[7] = c1.w;
    x.s[0] = s0.x; x.s[1] = s0.y; x.s[2] = s0.z; x.s[3] = s0.w;
    x.s[4] = s1.x; x.s[5] = s1.y; x.s[6] = s1.z; x.s[7] = s1.w;
  }
}

__device__ __forceinline__ uint4 qk_pack8(const float (&y)[8]) {
  uint4 o;
  o.x = pack_bf16x2(y[0], y[1]);
  o.y = pack_bf16x2(y[2], y[3]);
  o.z = pack_bf16x2(y[4], y[5]);
  o.w = pack_bf16x2(y[6], y[7]);
  return o;
}

// Normalise and rotate one row into out[ds] (8 bf16, RNE); cosr / sinr: this lane's row of the
// RoPE tables, HS = half / 32. The angles of sub-blocks 1 .. HS - 1 load where they are used.
template <int D, int HS>
__device__ __forceinline__ void qk_norm_rope_hs(const QkRaw<D>& x, const QkAux<D>& aux,
                                                const float* cosr, const float* sinr, float eps,
                                                int kq, uint4 (&out)[D / 32]) {
  constexpr int DS = D / 32;
  static_assert(2 * HS <= DS, "rotated dims exceed the head");
  float ss = 0.f;
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = qk_elem(x.w[ds], e);
      ss = __builtin_fmaf(v, v, ss);
    }
  ss = __fadd_rn(ss, __shfl_xor(ss, 16, 64));
  ss = __fadd_rn(ss, __shfl_xor(ss, 32, 64));
  const float inv = __frsqrt_rn(__fdiv_rn(ss, (float)D) + eps);
  auto scaled = [&](int ds, int e) {
    return __fmul_rn(__fmul_rn(qk_elem(x.w[ds], e), inv), qk_elem(aux.g[ds], e));
  };
  // rotate-half: d < half pairs with d + half (sub-block ds with ds + HS, same lane and slot)
#pragma unroll
  for (int ds = 0; ds < HS; ++ds) {
    float c[8], sn[8];
    if (ds == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) c[e] = aux.c[e], sn[e] = aux.s[e];
    } else {
      const float4* cp = (const float4*)(cosr + ds * 32 + kq * 8);
      const float4* sp = (const float4*)(sinr + ds * 32 + kq * 8);
      const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
      c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
      c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
      sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w;
      sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    }
    float ya[8], yb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ce = c[e], se = sn[e];
      const float a = scaled(ds, e), b = scaled(ds + HS, e);
      ya[e] = __fsub_rn(__fmul_rn(a, ce), __fmul_rn(b, se));
      yb[e] = __fadd_rn(__fmul_rn(b, ce), __fmul_rn(a, se));
    }
    out[ds] = qk_pack8(ya);
    out[ds + HS] = qk_pack8(yb);
  }
#pragma unroll
  for (int ds = 2 * HS; ds < DS; ++ds) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = scaled(ds, e);
    out[ds] = qk_pack8(y);
  }
}

// half a multiple of 32 with 2 half <= D and half <= 32 MAXHS (the entry points refuse any
// other; a kernel short of registers instantiates fewer rotation widths).
template <int D, int MAXHS = D / 64>
__device__ __forceinline__ void qk_norm_rope(const QkRaw<D>& x, const QkAux<D>& aux,
                                             const float* cosr, const float* sinr, int half,
                                             float eps, int kq, uint4 (&out)[D / 32]) {
  switch (half) {
    case 0: qk_norm_rope_hs<D, 0>(x, aux, cosr, sinr, eps, kq, out); break;
    case 32: qk_norm_rope_hs<D, 1>(x, aux, cosr, sinr, eps, kq, out); break;
    case 64:
      if constexpr (D >= 128 && MAXHS >= 2) qk_norm_rope_hs<D, 2>(x, aux, cosr, sinr, eps, kq, out);
      break;
    case 96:
      if constexpr (D >= 256 && MAXHS >= 3) qk_norm_rope_hs<D, 3>(x, aux, cosr, sinr, eps, kq, out);
      break;
    default:
      if constexpr (D >= 256 && MAXHS >= 4) qk_norm_rope_hs<D, 4>(x, aux, cosr, sinr, eps, kq, out);
      break;
  }
}

// Fetch, normalise and rotate one row where it is loaded.
template <int D, int MAXHS = D / 64>
__device__ __forceinline__ void qk_load_norm_rope(const uint16_t* row, bool live,
                                                  const uint16_t* __restrict__ gamma,
                                                  const float* cosr, const float* sinr, int half,
                                                  float eps, int kq, uint4 (&out)[D / 32]) {
  QkRaw<D> x;
  QkAux<D> aux;
  qk_fetch<D>(x, row, kq, live);
  qk_fetch_aux<D>(aux, gamma, cosr, sinr, half, kq);
  qk_norm_rope<D, MAXHS>(x, aux, cosr, sinr, half, eps, kq, out);
}

// Paged pool element offsets (layouts K [blocks, Hkv, D/16, page, 16], V [blocks, Hkv, page/4,
// D, 4]; tests/test_lfm2_dspark_reference.py:30-36): K of (slot, head h) at d .. d + 7 (d % 8 == 0)
// is one 16-byte run; V element (slot, h, d).
__device__ __forceinline__ int64_t k_pool_offset(int64_t blk, int off, int h, int Hkv, int D,
                                                 int page, int d) {
  return ((((int64_t)blk * Hkv + h) * (D / 16) + d / 16) * page + off) * 16 + d % 16;
}
__device__ __forceinline__ int64_t v_pool_offset(int64_t blk, int off, int h, int Hkv, int D,
                                                 int page, int d) {
  return ((((int64_t)blk * Hkv + h) * (page / 4) + off / 4) * D + d) * 4 + off % 4;
}

// Write this lane's part of a normalised K row (packed, slot >= 0) and copy its V row into the
// pools.
template <int D>
__device__ __forceinline__ void qk_store_kv(const uint4 (&k)[D / 32],
                                            const uint16_t* __restrict__ vrow,
                                            uint16_t* __restrict__ k_pool,
                                            uint16_t* __restrict__ v_pool, int slot, int h,
                                            int Hkv, int page, int kq) {
  if (slot < 0) return;
  const int64_t blk = slot / page;
  const int off = slot % page;
#pragma unroll
  for (int ds = 0; ds < D / 32; ++ds) {
    const int d = ds * 32 + kq * 8;
    *(uint4*)(k_pool + k_pool_offset(blk, off, h, Hkv, D, page, d)) = k[ds];
    const uint4 x = *(const uint4*)(vrow + d);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v_pool[v_pool_offset(blk, off, h, Hkv, D, page, d + 2 * i)] = (uint16_t)(w[i] & 0xffffu);
      v_pool[v_pool_offset(blk, off, h, Hkv, D, page, d + 2 * i + 1)] = (uint16_t)(w[i] >> 16);
    }
  }
}
