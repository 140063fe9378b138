// Shared device helpers for the gfx950 verify-step kernels.
//
// Everything here is wave64 / CDNA4 specific: reductions use 64-lane butterflies, bf16 and
// fp16 are handled as raw 16-bit patterns, and the canonical arithmetic used by the
// acceptance kernels (exp, fixed-point sums) is written with explicit IEEE operations so
// that a plain C restatement on the host reproduces it bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SV_API extern "C" __attribute__((visibility("default")))

// Status codes are HIP statuses so that snowllm_error_string can defer to the runtime.
#define SV_OK 0
#define SV_EINVAL ((int)hipErrorInvalidValue)
#define SV_ENOTSUP ((int)hipErrorNotSupported)

#define SV_CHECK_LAUNCH()                                   \
  do {                                                      \
    hipError_t _e = hipGetLastError();                      \
    if (_e != hipSuccess) return (int)_e;                   \
  } while (0)

static constexpr int WAVE = 64;

// ---------------------------------------------------------------------------------------
// 16-bit float patterns
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
// Round to nearest even (NaN stays NaN): the gfx950 v_cvt_pk_bf16_f32 conversion.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats -> packed bf16 pair (a in the low half), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){a, b}, b2_t));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}

// ---------------------------------------------------------------------------------------
// Wave64 reductions (butterfly; every lane ends with the result)
// ---------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    T o = __shfl_xor(v, s, WAVE);
    v = o > v ? o : v;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, WAVE);
  return v;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int s) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, s, WAVE);
  hi = __shfl_xor(hi, s, WAVE);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v += shfl_xor_u64(v, s);
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    uint64_t o = shfl_xor_u64(v, s);
    v = o > v ? o : v;
  }
  return v;
}

// Cross-lane moves on the VALU (DPP) instead of the LDS crossbar: quad xor 1 / xor 2, then
// mirrors within 8 and 16 lanes leave every lane of a 16-lane row with the row's result; the
// four rows meet through readlane. Each step is symmetric, so all lanes end with one value.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141,
              DPP_MIRROR = 0x140;

__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  uint32_t o;
  o = dpp_u32<DPP_QUAD_XOR1>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_QUAD_XOR2>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_HALF_MIRROR>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_MIRROR>(v); v = o > v ? o : v;
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
  return ab > cd ? ab : cd;
}

// Wave maximum left in every lane (no scalar round trip): the row maxima by DPP, then the
// gfx950 row-pair and half-wave swaps (v_permlane16_swap: rows 0<->1 and 2<->3;
// v_permlane32_swap: lanes 0-31 <-> 32-63).
__device__ __forceinline__ uint32_t wave_max_u32_all(uint32_t v) {
  uint32_t o;
  o = dpp_u32<DPP_QUAD_XOR1>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_QUAD_XOR2>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_HALF_MIRROR>(v); v = o > v ? o : v;
  o = dpp_u32<DPP_MIRROR>(v); v = o > v ? o : v;
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = r[0] > r[1] ? r[0] : r[1];
  const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return q[0] > q[1] ? q[0] : q[1];
}

__device__ __forceinline__ uint32_t wave_min_u32_dpp(uint32_t v) {
  uint32_t o;
  o = dpp_u32<DPP_QUAD_XOR1>(v); v = o < v ? o : v;
  o = dpp_u32<DPP_QUAD_XOR2>(v); v = o < v ? o : v;
  o = dpp_u32<DPP_HALF_MIRROR>(v); v = o < v ? o : v;
  o = dpp_u32<DPP_MIRROR>(v); v = o < v ? o : v;
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  const uint32_t ab = a < b ? a : b, cd = c < d ? c : d;
  return ab < cd ? ab : cd;
}

// Sum in a fixed order (pairs, quads, 8s, 16s, then rows 0 + 1 + 2 + 3).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __uint_as_float(dpp_u32<DPP_QUAD_XOR1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<DPP_QUAD_XOR2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<DPP_HALF_MIRROR>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<DPP_MIRROR>(__float_as_uint(v)));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ uint32_t wave_sum_u32_dpp(uint32_t v) {
  v += dpp_u32<DPP_QUAD_XOR1>(v);
  v += dpp_u32<DPP_QUAD_XOR2>(v);
  v += dpp_u32<DPP_HALF_MIRROR>(v);
  v += dpp_u32<DPP_MIRROR>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 0) + (uint32_t)__builtin_amdgcn_readlane((int)v, 16) +
         (uint32_t)__builtin_amdgcn_readlane((int)v, 32) + (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
}

// Inclusive prefix sum within each 16-lane row (row_shr by 1, 2, 4, 8; lanes shifted in
// from outside the row read 0).
__device__ __forceinline__ uint32_t row_scan_u32_dpp(uint32_t v) {
  v += dpp_u32<0x111>(v);
  v += dpp_u32<0x112>(v);
  v += dpp_u32<0x114>(v);
  v += dpp_u32<0x118>(v);
  return v;
}

// Block-wide reductions for blockDim.x == NT (a multiple of 64). `red` must hold NT/64 slots.
template <int NT>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
  v = wave_sum_u64(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) t += red[i];
  __syncthreads();
  return t;
}

template <int NT>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) t = red[i] > t ? red[i] : t;
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------------------
// Ordered float keys. NaN is treated as -inf (the argmax and top-k rules of the reference
// sampler). ord(a) > ord(b) <=> a > b for non-NaN floats, and -0.0 == +0.0.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ord_key(float f) {
  if (f != f) f = -__builtin_huge_valf();
  if (f == 0.0f) f = 0.0f;  // fold -0 into +0 so that ties compare equal
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float ord_key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// (value, index) packed so that the maximum key is the largest value with the lowest index.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  return ((uint64_t)ord_key(v) << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(uint64_t k) {
  return 0xffffffffu - (uint32_t)(k & 0xffffffffu);
}

// ---------------------------------------------------------------------------------------
// Canonical arithmetic shared (by restatement) with the host oracle.
//
// canon_exp: e^x for x <= 0 by Cody & Waite argument reduction (x = n ln2 + r, ln2 split
// into a high part with trailing zero bits and a low correction) followed by the degree-7
// Taylor polynomial of e^r evaluated by Horner's rule with fused multiply-adds, then
// scaled by 2^n. Inputs below -86 return 0 so that no subnormal result is ever produced.
// Every step is a single IEEE-754 binary32 operation, so the result is reproducible on any
// IEEE host with a correctly rounded fmaf.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float canon_exp(float x) {
#pragma clang fp contract(off)
  if (!(x >= -86.0f)) return 0.0f;  // also maps NaN and -inf to 0
  const float kLog2e = 1.44269502162933349609375f;   // log2(e) rounded to binary32
  const float kLn2Hi = 0.693145751953125f;           // ln 2 high part (12 trailing zero bits)
  const float kLn2Lo = 1.428606765330187045037746429443359375e-06f;  // ln 2 - kLn2Hi
  float t = __fmul_rn(x, kLog2e);
  float n = __builtin_rintf(t);
  float r = __builtin_fmaf(-n, kLn2Hi, x);
  r = __builtin_fmaf(-n, kLn2Lo, r);
  float p = 1.98412698412698412698e-4f;              // 1/7!
  p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);  // 1/6!
  p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);  // 1/5!
  p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);  // 1/4!
  p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);  // 1/3!
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// Probabilities below the smallest normal binary32 are flushed to zero explicitly, so the
// result never depends on a device's denormal mode.
__device__ __forceinline__ float canon_div(float a, float b) {
#pragma clang fp contract(off)
  float q = __fdiv_rn(a, b);
  return (__builtin_fabsf(q) < 1.17549435082228750797e-38f) ? 0.0f : q;
}

// Fixed-point weight: floor(w * 2^44) for w in [0, 1]. Sums of up to 2^19 such terms fit in
// 63 bits exactly, so any reduction order gives the same integer.
#define SV_FIX_BITS 44
__device__ __forceinline__ uint64_t canon_fix(float w) {
#pragma clang fp contract(off)
  if (!(w > 0.0f)) return 0;
  float s = __builtin_ldexpf(w, SV_FIX_BITS);
  return (uint64_t)__builtin_floorf(s);
}

// Round-to-nearest-even conversion of an unsigned 64-bit integer to binary32, written out
// with integer operations so that host and device agree without relying on library code.
__device__ __forceinline__ float canon_u64_to_f32(uint64_t v) {
  if (v == 0) return 0.0f;
  int lz = __builtin_clzll(v);
  int msb = 63 - lz;
  if (msb <= 23) return (float)(uint32_t)v;  // exact
  int shift = msb - 23;
  uint64_t mant = v >> shift;
  uint64_t rem = v & ((1ull << shift) - 1);
  uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (mant & 1))) {
    mant += 1;
    if (mant == (1ull << 24)) { mant >>= 1; shift += 1; }
  }
  return __builtin_ldexpf((float)(uint32_t)mant, shift);
}

// Sum of fixed-point weights back to a binary32 value: round(v) * 2^-44.
__device__ __forceinline__ float canon_unfix(uint64_t v) {
#pragma clang fp contract(off)
  return __builtin_ldexpf(canon_u64_to_f32(v), -SV_FIX_BITS);
}

// floor(u * R) for u in [0, 1) a binary32 value and R a 63-bit integer, exactly.
__device__ __forceinline__ uint64_t canon_scale_floor(float u, uint64_t R) {
  if (!(u > 0.0f)) return 0;
  uint32_t bits = __float_as_uint(u);
  int e = (int)((bits >> 23) & 0xff);
  uint64_t m = (e == 0) ? (bits & 0x7fffffu) : ((bits & 0x7fffffu) | 0x800000u);
  int exp2 = (e == 0 ? 1 : e) - 127 - 23;  // u = m * 2^exp2, exp2 <= -24 for u < 1
  unsigned __int128 prod = (unsigned __int128)m * (unsigned __int128)R;
  int sh = -exp2;
  if (sh >= 128) return 0;
  return (uint64_t)(prod >> sh);
}
