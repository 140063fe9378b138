// Per-layer plumbing of the verify step around the GEMVs and attention: model geometry,
// embedding gather, RMSNorm (+ residual), RoPE tables, QK-norm + RoPE + paged KV write, slot
// resolution, SwiGLU, MoE routing and residual adds.
//
// The reference compiles its model shapes into the library and selects one with
// snowllm_select_geometry (snowllm/_capi.py:44-113). Here shapes are run-time data: the same
// selection call works for the shapes this build is measured on, and snowverify_define_geometry
// installs any other. Entry points with the reference's signatures read the current geometry;
// the snowverify_* forms take every shape explicitly.
#include "common.h"

#include <string.h>

#include "geometry.h"
#include "qknorm.h"

namespace {

constexpr int GEO_QWEN36_35B_A3B = 0;  // reference id; BASELINE configs 4 and 5
constexpr int GEO_DENSE_8B = 100;      // this build's id for BASELINE config 3
constexpr int GEO_CUSTOM = 1000;       // installed by snowverify_define_geometry

BuildGeometry make_moe_35b() {
  BuildGeometry g;
  memset(&g, 0, sizeof g);
  g.hidden = 2048; g.num_heads = 16; g.num_kv_heads = 2; g.head_size = 256; g.block_size = 16;
  g.vocab_size = 151936;
  g.qkv_proj_n = (16 + 2 + 2) * 256; g.qkv_q_head_stride = 256;
  g.qkv_off_k = 16 * 256; g.qkv_off_v = 18 * 256;
  g.moe_num_experts = 256; g.moe_shared_expert = 1; g.moe_topk = 8; g.moe_topk_all = 9;
  g.moe_inter = 512; g.sampling_max_k = 1 << 19; g.lm_head_decode_max_m = 256;
  return g;
}

BuildGeometry make_dense_8b() {
  BuildGeometry g;
  memset(&g, 0, sizeof g);
  g.hidden = 4096; g.num_heads = 32; g.num_kv_heads = 8; g.head_size = 128; g.block_size = 16;
  g.vocab_size = 151936;
  g.qkv_proj_n = (32 + 8 + 8) * 128; g.qkv_q_head_stride = 128;
  g.qkv_off_k = 32 * 128; g.qkv_off_v = 40 * 128;
  g.sampling_max_k = 1 << 19; g.lm_head_decode_max_m = 256;
  g.mlp_inter = 14336; g.mlp_gate_up_n = 2 * 14336;
  return g;
}

BuildGeometry g_geo = make_moe_35b();
int g_geo_id = GEO_QWEN36_35B_A3B;

inline hipStream_t S(void* s) { return (hipStream_t)s; }

// ---------------------------------------------------------------------------------------
// embedding gather: out[m, :] = table[ids[m], :] (fp16 or bf16 table) -> bf16
// ---------------------------------------------------------------------------------------
__global__ void gather_embedding_kernel(const int64_t* __restrict__ ids,
                                        const uint16_t* __restrict__ table,
                                        uint16_t* __restrict__ out, int64_t V, int64_t H,
                                        int table_f16) {
  const int64_t m = blockIdx.x;
  int64_t id = ids[m];
  if (id < 0 || id >= V) id = 0;
  const uint16_t* row = table + id * H;
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
    const uint16_t v = row[i];
    out[m * H + i] = table_f16 ? f32_to_bf16(f16_to_f32(v)) : v;
  }
}

// Embedding gather from a Q4_K table [V, H] (H / 256 blocks of 144 bytes per row): one
// 256-thread block per row, thread t decodes element t of every block. A block is fp16 d at 0,
// fp16 dmin at 2, twelve bytes of 6-bit scales/mins at 4 and 128 nibble bytes at 16; element
// 64 g + 32 h + l is the low (h = 0) or high (h = 1) nibble of byte 16 + 32 g + l and uses
// scale/min j = 2 g + h, where j < 4 takes sc = s[j] & 63, m = s[j + 4] & 63 and j >= 4 takes
// sc = (s[j + 4] & 15) | (s[j - 4] >> 6) << 4, m = (s[j + 4] >> 4) | (s[j] >> 6) << 4. The
// value is fp32(d sc) q - fp32(dmin m), two roundings (no fused multiply-add), then bf16.
__global__ void __launch_bounds__(256) gather_embedding_q4k_kernel(
    const int64_t* __restrict__ ids, const uint8_t* __restrict__ table, uint16_t* __restrict__ out,
    int64_t V, int64_t H) {
#pragma clang fp contract(off)
  const int64_t m = blockIdx.x;
  int64_t id = ids[m];
  if (id < 0 || id >= V) id = 0;
  const int64_t nb = H / 256;
  const uint8_t* row = table + id * nb * 144;
  const int t = threadIdx.x, g = t >> 6, h = (t >> 5) & 1, l = t & 31, j = 2 * g + h;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + b * 144;
    const float d = f16_to_f32((uint16_t)(blk[0] | blk[1] << 8));
    const float dmin = f16_to_f32((uint16_t)(blk[2] | blk[3] << 8));
    const uint8_t* s = blk + 4;
    int sc, mn;
    if (j < 4) {
      sc = s[j] & 63;
      mn = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
      mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const uint8_t byte = blk[16 + 32 * g + l];
    const float q = (float)(h ? byte >> 4 : byte & 15);
    const float dsc = d * (float)sc;
    const float dmn = dmin * (float)mn;
    const float prod = dsc * q;
    out[m * H + b * 256 + t] = f32_to_bf16(prod - dmn);
  }
}

// ---------------------------------------------------------------------------------------
// RMSNorm: y = x * rsqrt(mean(x^2) + eps) * gamma, fp32 math, bf16 out. With a residual,
// the residual stream is updated first (residual = x + residual, rounded to bf16) and
// normalised. One 256-thread block per row.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ residual,
                                                      const uint16_t* __restrict__ gamma,
                                                      uint16_t* __restrict__ out, int64_t H,
                                                      float eps) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const uint16_t* xr = x + m * H;
  uint16_t* rr = residual ? residual + m * H : nullptr;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += 256) {
    float v = bf16_to_f32(xr[i]);
    if (rr) {
      v = bf16_to_f32(f32_to_bf16(v + bf16_to_f32(rr[i])));
      rr[i] = f32_to_bf16(v);
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = __frsqrt_rn(tot / (float)H + eps);
  const uint16_t* src = rr ? rr : xr;
  for (int64_t i = threadIdx.x; i < H; i += 256)
    out[m * H + i] = f32_to_bf16(bf16_to_f32(src[i]) * inv * bf16_to_f32(gamma[i]));
}

// ---------------------------------------------------------------------------------------
// RoPE tables: cos/sin[m, i] = cos/sin(pos[m] * inv_freq[i]), i < half (f32)
// ---------------------------------------------------------------------------------------
// Rows are `width` apart; width = 2 half repeats the half in columns half .. 2 half - 1.
__global__ void rope_cos_sin_kernel(const int64_t* __restrict__ pos,
                                    const float* __restrict__ inv_freq, float* __restrict__ c,
                                    float* __restrict__ s, int64_t M, int half, int width) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * half) return;
  const int64_t m = idx / half;
  const int i = (int)(idx % half);
  const float a = (float)pos[m] * inv_freq[i];
  const float cv = cosf(a), sv = sinf(a);
  c[m * width + i] = cv;
  s[m * width + i] = sv;
  if (width >= 2 * half) {
    c[m * width + half + i] = cv;
    s[m * width + half + i] = sv;
  }
}

// ---------------------------------------------------------------------------------------
// QK-norm + RoPE + paged KV write. Per head: RMSNorm over D with its gamma (fp32), rotate the
// first 2*half dims (pairs (i, i + half)), round once to bf16 (qknorm.h). q goes to q_out
// [M, Hq, D]; k and v go to the pools at slots[m] in the layouts K [blocks, Hkv, D/16, page, 16]
// and V [blocks, Hkv, page/4, D, 4]. One wave per (16 rows, head); a kv head's wave writes both
// its K and V rows.
// ---------------------------------------------------------------------------------------
// Sources of one row's heads: q head h at q + m * q_stride + h * q_head_stride, k head h at
// k + m * k_stride + h * D, v head h at v + m * v_stride + h * D; cos/sin rows cs_stride apart
// (the first `half` entries of a row are used).
struct QkvSources {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, q_head_stride, k_stride, v_stride, cs_stride;
};

template <int D>
__global__ void __launch_bounds__(64) qk_norm_rope_cache_kernel(
    QkvSources src, const uint16_t* __restrict__ q_gamma, const uint16_t* __restrict__ k_gamma,
    const float* __restrict__ cosv, const float* __restrict__ sinv, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ slots, int64_t M, int Hq, int Hkv, int half, int page, float eps) {
  const int head = blockIdx.x;
  const int lane = threadIdx.x, col = lane & 15, kq = lane >> 4;
  const int64_t m = (int64_t)blockIdx.y * 16 + col;
  const bool live = m < M;
  const int64_t mr = live ? m : 0;
  const float* cr = cosv + mr * src.cs_stride;
  const float* sr = sinv + mr * src.cs_stride;
  uint4 o[D / 32];
  if (head < Hq) {
    qk_load_norm_rope<D>(src.q + mr * src.q_stride + (int64_t)head * src.q_head_stride, live,
                         q_gamma, cr, sr, half, eps, kq, o);
    if (live)
#pragma unroll
      for (int ds = 0; ds < D / 32; ++ds)
        *(uint4*)(q_out + (m * Hq + head) * D + ds * 32 + kq * 8) = o[ds];
    return;
  }
  const int h = head - Hq;
  qk_load_norm_rope<D>(src.k + mr * src.k_stride + (int64_t)h * D, live, k_gamma, cr, sr, half,
                       eps, kq, o);
  if (live)
    qk_store_kv<D>(o, src.v + m * src.v_stride + (int64_t)h * D, k_pool, v_pool, slots[m], h, Hkv,
                   page, kq);
}

// The reference's rotary geometry: rotary dimension 64 (head_size x partial_rotary_factor,
// checked at snowllm/models/qwen3_5/qwen3_5_weights.py:444), so 32 frequencies.
constexpr int REF_ROPE_HALF = 32;

int launch_qk_norm_rope_cache(const QkvSources& src, const void* q_gamma, const void* k_gamma,
                              const float* cosv, const float* sinv, void* q_out, void* k_pool,
                              void* v_pool, const int32_t* slots, int64_t M, int64_t Hq,
                              int64_t Hkv, int64_t D, int64_t half, int64_t page, float eps,
                              hipStream_t s) {
  if (half < 0 || half % 32 || 2 * half > D) return SV_EINVAL;
  const dim3 grid((unsigned)(Hq + Hkv), (unsigned)((M + 15) / 16));
  auto kern = D == 64 ? qk_norm_rope_cache_kernel<64>
            : D == 128 ? qk_norm_rope_cache_kernel<128> : qk_norm_rope_cache_kernel<256>;
  if (D != 64 && D != 128 && D != 256) return SV_EINVAL;
  hipLaunchKernelGGL(kern, grid, dim3(64), 0, s, src, (const uint16_t*)q_gamma,
                     (const uint16_t*)k_gamma, cosv, sinv, (uint16_t*)q_out, (uint16_t*)k_pool,
                     (uint16_t*)v_pool, slots, M, (int)Hq, (int)Hkv, (int)half, (int)page, eps);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// slot = table[row_seq, pos / page] * page + pos % page (snowllm/engine/spec_decode.py:183).
// A row whose sequence or position is negative, whose page lies past the table's width, or
// whose table entry is negative (padding) gets slot -1, which the cache writers skip.
__global__ void resolve_slots_kernel(const int32_t* __restrict__ table, int64_t stride,
                                     const int32_t* __restrict__ seq, const int32_t* __restrict__ pos,
                                     int32_t* __restrict__ out, int64_t M, int64_t page) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  const int64_t p = pos[m], b = seq[m];
  if (p < 0 || b < 0) {
    out[m] = -1;
    return;
  }
  const int64_t col = p / page;
  const int64_t blk = col < stride ? (int64_t)table[b * stride + col] : -1;
  out[m] = blk >= 0 ? (int32_t)(blk * page + p % page) : -1;
}

// SwiGLU: out[m, i] = silu(gu[m, i]) * gu[m, F + i] (bf16)
__global__ void swiglu_kernel(const uint16_t* __restrict__ gu, int64_t stride,
                              uint16_t* __restrict__ out, int64_t M, int64_t F) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * F) return;
  const int64_t m = idx / F, i = idx % F;
  const float g = bf16_to_f32(gu[m * stride + i]);
  const float u = bf16_to_f32(gu[m * stride + F + i]);
  const float s = g / (1.0f + __expf(-g));
  out[idx] = f32_to_bf16(s * u);
}

// out = a + b (bf16, fp32 add, one rounding)
__global__ void add_bf16_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                uint16_t* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

}  // namespace

// =======================================================================================
// geometry
// =======================================================================================

SV_API void snowllm_model_config(BuildGeometry* out) {
  if (out) *out = g_geo;
}

SV_API int snowllm_select_geometry(int geo) {
  if (geo == GEO_QWEN36_35B_A3B) g_geo = make_moe_35b();
  else if (geo == GEO_DENSE_8B) g_geo = make_dense_8b();
  else return SV_EINVAL;
  g_geo_id = geo;
  return SV_OK;
}

SV_API int snowllm_active_geometry(void) { return g_geo_id; }

SV_API int64_t snowllm_geometry_name(int geo, char* buf, int64_t n) {
  const char* name = geo == GEO_QWEN36_35B_A3B ? "qwen3.6-35b-a3b"
                     : geo == GEO_DENSE_8B     ? "dense-8b"
                     : geo == GEO_CUSTOM       ? "custom"
                                               : "";
  const int64_t len = (int64_t)strlen(name);
  if (buf && n > 0) {
    const int64_t c = len < n - 1 ? len : n - 1;
    memcpy(buf, name, (size_t)c);
    buf[c] = 0;
  }
  return len;
}

// Extension: install arbitrary shapes as the current geometry (id 1000).
SV_API int snowverify_define_geometry(const BuildGeometry* g) {
  if (!g || g->hidden <= 0 || g->num_heads <= 0 || g->num_kv_heads <= 0 ||
      g->num_heads % g->num_kv_heads || g->head_size <= 0)
    return SV_EINVAL;
  g_geo = *g;
  g_geo_id = GEO_CUSTOM;
  return SV_OK;
}

// =======================================================================================
// layer ops
// =======================================================================================

// Extension: embedding gather from an fp16 (table_f16 = 1) or bf16 table [V, H] -> bf16.
SV_API int snowverify_gather_embedding(const int64_t* ids, const void* table, void* out, int64_t M,
                                       int64_t V, int64_t H, int table_f16, void* stream) {
  if (M < 0 || V <= 0 || H <= 0) return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipLaunchKernelGGL(gather_embedding_kernel, dim3((unsigned)M), dim3(256), 0, S(stream), ids,
                     (const uint16_t*)table, (uint16_t*)out, V, H, table_f16);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Reference signature (snowllm/_capi.py:375; snowllm/ops/embedding.py:18-25): bf16 table
// [vocab, hidden] of the current geometry.
SV_API int snowllm_gather_embedding(const int64_t* ids, const void* table, void* out, int64_t M,
                                    void* stream) {
  return snowverify_gather_embedding(ids, table, out, M, g_geo.vocab_size, g_geo.hidden, 0, stream);
}

// Reference signature (snowllm/_capi.py:726; snowllm/ops/embedding.py:27-41): gather from a
// Q4_K table [vocab, hidden / 256 * 144 bytes] -> bf16 [rows, hidden]; hidden % 256 == 0.
// Ids outside [0, vocab) read row 0, as the 16-bit gather does.
SV_API int snowllm_gather_embedding_q4_k(const int64_t* ids, const void* weight, void* out,
                                         int64_t rows, int64_t vocab, int64_t hidden,
                                         void* stream) {
  if (rows < 0 || vocab <= 0 || hidden <= 0 || hidden % 256 || !weight || !out) return SV_EINVAL;
  if (rows == 0) return SV_OK;
  if (!ids) return SV_EINVAL;
  hipLaunchKernelGGL(gather_embedding_q4k_kernel, dim3((unsigned)rows), dim3(256), 0, S(stream),
                     ids, (const uint8_t*)weight, (uint16_t*)out, vocab, hidden);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension: RMSNorm with explicit width; residual may be null.
SV_API int snowverify_rmsnorm(const void* x, void* residual, const void* gamma, void* out,
                              int64_t M, int64_t H, float eps, void* stream) {
  if (M < 0 || H <= 0) return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)M), dim3(256), 0, S(stream),
                     (const uint16_t*)x, (uint16_t*)residual, (const uint16_t*)gamma,
                     (uint16_t*)out, H, eps);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Reference signatures (snowllm/_capi.py:376, 381; snowllm/ops/norm.py:66-97).
SV_API int snowllm_rmsnorm(const void* x, const void* gamma, void* out, int64_t M, float eps,
                           void* stream) {
  return snowverify_rmsnorm(x, nullptr, gamma, out, M, g_geo.hidden, eps, stream);
}

SV_API int snowllm_rmsnorm_residual(const void* x, void* residual, const void* gamma, void* out,
                                    int64_t M, float eps, void* stream) {
  return snowverify_rmsnorm(x, residual, gamma, out, M, g_geo.hidden, eps, stream);
}

// Extension: RoPE tables [M, half] for positions and inverse frequencies.
SV_API int snowverify_rope_cos_sin(const int64_t* pos, const float* inv_freq, float* cosv,
                                   float* sinv, int64_t M, int64_t half, void* stream) {
  if (M < 0 || half <= 0) return SV_EINVAL;
  if (M == 0) return SV_OK;
  const int64_t n = M * half;
  hipLaunchKernelGGL(rope_cos_sin_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     S(stream), pos, inv_freq, cosv, sinv, M, (int)half, (int)half);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Reference signature (snowllm/_capi.py; wrapper snowllm/ops/rope.py:11-24, the plain form):
// cos/sin [M, 64] f32 for the reference's rotary dimension 64, the 32 frequencies' values in
// columns 0..31 repeated in 32..63 (the rotate-half convention); inv_freq f32 [32].
SV_API int snowllm_rope_cos_sin(const int64_t* pos, const float* inv_freq, float* cosv,
                                float* sinv, int64_t M, void* stream) {
  if (M < 0) return SV_EINVAL;
  if (M == 0) return SV_OK;
  const int64_t n = M * REF_ROPE_HALF;
  hipLaunchKernelGGL(rope_cos_sin_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     S(stream), pos, inv_freq, cosv, sinv, M, REF_ROPE_HALF, 2 * REF_ROPE_HALF);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension: QK-norm + RoPE + paged KV write with explicit shapes (the reference's
// snowllm_qk_norm_rope_cache, snowllm/_capi.py:397-399 and ops/attention_full.py:736-784,
// takes them from the geometry). proj [M, stride] bf16 = [q | k | v]; q_out [M, Hq, D];
// cos/sin [M, half]; slots [M] (negative: do not cache). D in {64, 128, 256}; half a multiple
// of 32 with 2 half <= D.
SV_API int snowverify_qk_norm_rope_cache(const void* proj, int64_t stride, const void* q_gamma,
                                         const void* k_gamma, const float* cosv, const float* sinv,
                                         void* q_out, void* k_pool, void* v_pool,
                                         const int32_t* slots, int64_t M, int64_t Hq, int64_t Hkv,
                                         int64_t D, int64_t half, int64_t page, float eps,
                                         void* stream) {
  if (M < 0 || Hq <= 0 || Hkv <= 0 || (D != 64 && D != 128 && D != 256) || half % 32 ||
      2 * half > D || half < 0 || page != 16)
    return SV_EINVAL;
  if (M == 0) return SV_OK;
  const uint16_t* p = (const uint16_t*)proj;
  const QkvSources src{p, p + Hq * D, p + (Hq + Hkv) * D, stride, D, stride, stride, half};
  return launch_qk_norm_rope_cache(src, q_gamma, k_gamma, cosv, sinv, q_out, k_pool, v_pool,
                                   slots, M, Hq, Hkv, D, half, page, eps, S(stream));
}

// Reference signature (snowllm/_capi.py:397-399; wrapper snowllm/ops/attention_full.py:736-
// 784): shapes from the active geometry (num_heads, num_kv_heads, head_size, q head stride),
// K and V read from their own rows (kp/ks, v/vs), cos/sin [m, 64] (rotary dim 64: the first 32
// columns hold the frequencies' cos and sin, as rope_cos_sin writes them). bf16 KV pools only:
// k_scale and v_scale must be null (the int8 KV variant is not part of this build).
SV_API int snowllm_qk_norm_rope_cache(const void* proj, int64_t n, const void* kp, int64_t ks,
                                      const void* v, int64_t vs, const void* q_gamma,
                                      const void* k_gamma, const float* cosv, const float* sinv,
                                      void* q, void* k_cache, void* v_cache, const void* k_scale,
                                      const void* v_scale, const int32_t* slots, int64_t m,
                                      float eps, int64_t block_size, void* stream) {
  if (k_scale || v_scale) return SV_ENOTSUP;
  const BuildGeometry& g = g_geo;
  if (block_size != g.block_size) return SV_EINVAL;
  const int64_t D = g.head_size, Hq = g.num_heads, Hkv = g.num_kv_heads;
  if (m < 0 || (D != 64 && D != 128 && D != 256) || block_size != 16) return SV_EINVAL;
  if (m == 0) return SV_OK;
  const QkvSources src{(const uint16_t*)proj, (const uint16_t*)kp, (const uint16_t*)v, n,
                       g.qkv_q_head_stride, ks, vs, 2 * REF_ROPE_HALF};
  return launch_qk_norm_rope_cache(src, q_gamma, k_gamma, cosv, sinv, q, k_cache, v_cache, slots,
                                   m, Hq, Hkv, D, REF_ROPE_HALF, block_size, eps, S(stream));
}

// Reference signature (snowllm/_capi.py:361; snowllm/ops/cache.py:40-53).
SV_API int snowllm_resolve_slots(const int32_t* table, int64_t stride, const int32_t* seq,
                                 const int32_t* pos, int32_t* out, int64_t M, int64_t page,
                                 void* stream) {
  if (M < 0 || stride <= 0 || page <= 0) return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipLaunchKernelGGL(resolve_slots_kernel, dim3((unsigned)((M + 255) / 256)), dim3(256), 0,
                     S(stream), table, stride, seq, pos, out, M, page);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Reference signature (snowllm/_capi.py:359; snowllm/ops/attention_full.py:521-528): bytes of
// the K and V pools for num_blocks pages of the current geometry (bf16 only).
SV_API void snowllm_kv_pool_bytes(int64_t num_blocks, int64_t block_size, int kv_int8, int64_t* k,
                                  int64_t* v) {
  const int64_t n = kv_int8 ? 0 : num_blocks * block_size * g_geo.num_kv_heads * g_geo.head_size * 2;
  if (k) *k = n;
  if (v) *v = n;
}

// Extension: SwiGLU over a [M, 2F] gate|up block (row stride in elements) -> [M, F].
SV_API int snowverify_swiglu(const void* gate_up, int64_t stride, void* out, int64_t M, int64_t F,
                             void* stream) {
  if (M < 0 || F <= 0 || stride < 2 * F) return SV_EINVAL;
  if (M == 0) return SV_OK;
  const int64_t n = M * F;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, S(stream),
                     (const uint16_t*)gate_up, stride, (uint16_t*)out, M, F);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension: out = a + b over n bf16 values.
SV_API int snowverify_add_bf16(const void* a, const void* b, void* out, int64_t n, void* stream) {
  if (n < 0) return SV_EINVAL;
  if (n == 0) return SV_OK;
  hipLaunchKernelGGL(add_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, S(stream),
                     (const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

const BuildGeometry& active_geometry() { return g_geo; }
