// The DSpark Markov head (snowllm/ops/dspark.py:10-16, 53-77; snowllm/_capi.py:567-573): a
// greedy walk over a draft block in which every row's logits get a low-rank bias from the
// previous token,
//
//   latent = W1[prev]                       (prev = the anchor, then the previous row's pick)
//   bias   = W2 latent                      (one value per vocabulary row)
//   pick   = argmax fp32(base + bias)        confidence = sigmoid([hidden, latent] . w + b)
//
// (the reference's PyTorch restatement: tests/test_lfm2_dspark_reference.py:143-152).
//
// Each row streams all of W2 ([V, rank] bf16, 78 MB at V = 151936, rank 256) once for every
// request of the batch together: the walk is HBM-bound, one launch per block row. W2 is packed
// so that one wave load of 1 KB gives each of 64 lanes a 16-byte chunk of its own vocabulary
// row; each lane sums its row's products in fp64 -- exact for products of two bf16 values --
// and rounds the sum once, so the bias does not depend on the summation order. Every
// workgroup reduces its rows to one (value, index) key per request; the last workgroup of a
// two-level arrival reduces the keys, writes the pick and the confidence, and the next row's
// launch reads the pick as its latent index.
#include "common.h"

namespace {

constexpr int DSP_WAVES = 4;               // waves per 64-row tile (they split the rank)
constexpr int DSP_NT = DSP_WAVES * WAVE;
constexpr int DSP_MAX_B = 16;              // requests per call
constexpr int DSP_MAX_RANK = 512;
constexpr uint64_t DSP_QUANTUM = 1ull << 20;  // > workgroups of a launch
constexpr int64_t DSP_MAX_V = (int64_t)1 << 31;

// Arrivals of the last launch (library-owned; calls on one device are stream-ordered). Each
// launch adds exactly one quantum, so the count stays a multiple of it between launches and
// captured replays need no reset.
__device__ uint64_t g_dsp_cnt;

// Packed W2: tile t holds rows [64 t, 64 t + rows_t), rows_t = min(64, n - 64 t), and stores
// chunk c (elements 8c .. 8c + 7) of its rows at elements 64 t k + (c rows_t + lane) 8. The
// packed matrix has exactly the n k elements of the source.
__global__ void dsp_pack_kernel(const uint16_t* __restrict__ raw, uint16_t* __restrict__ packed,
                                int64_t n, int64_t k) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // 16-byte chunk of the source
  const int64_t chunks = k / 8;
  if (i >= n * chunks) return;
  const int64_t row = i / chunks, c = i % chunks;
  const int64_t t = row / 64, lane = row % 64;
  const int64_t rows_t = n - 64 * t < 64 ? n - 64 * t : 64;
  const uint4 v = *(const uint4*)(raw + row * k + c * 8);
  *(uint4*)(packed + 64 * t * k + (c * rows_t + lane) * 8) = v;
}

// fp64 -> the nearest bf16 value, rounded once: round to odd at fp32 (16 spare bits), then to
// nearest-even at bf16.
__device__ __forceinline__ float bf16_from_f64(double d) {
  const float t = (float)d;
  uint32_t u = __float_as_uint(t);
  if ((double)t != d && d == d) {
    if (fabs((double)t) > fabs(d)) u -= 1;  // the fp32 rounding went away from zero: step back
    u |= 1;
  }
  return bf16_to_f32(f32_to_bf16(__uint_as_float(u)));
}

struct DspArgs {
  const float* base;        // [b * block, base_stride] f32
  const uint16_t* w1;       // [v, rank] bf16
  const uint16_t* w2;       // packed [v, rank] bf16
  const int64_t* anchor;    // [b]
  const uint16_t* pre_head; // [b * block, ps] bf16 or null
  const float* conf_w;      // [h + rank]
  const float* conf_b;      // scalar or null
  int64_t* out;             // [b, block]
  float* confidence;        // [b, block] or null
  uint64_t* partial;        // [b, nwg]
  int64_t v, base_stride, ps;
  int b, rank, block, h, nwg, fp32_bias, j;
};

// Grid: G <= 1024 workgroups of 4 waves; wave k of workgroup g takes the 64-row tiles
// 4 g + k, 4 g + k + 4 G, ... and keeps its best (value, index) key per request. Each lane sums
// its row's products in fp64 with 8 chunk loads (128 bytes of the row) in flight.
// Arrival is two-level so that no counter sees more than 32 arrivals: the workgroups of a
// group of 32 count on the group's counter; the group's last arrival reduces the group's keys
// and counts on the top counter, whose last arrival reduces the groups' keys and writes the
// pick (and the confidence).
constexpr int DSP_GRID = 1024, DSP_GROUP = 32, DSP_GROUPS = DSP_GRID / DSP_GROUP;
__device__ uint64_t g_dsp_group[DSP_GROUPS];

__device__ __forceinline__ bool dsp_arrive(uint64_t* cnt, int n, bool lead, uint32_t* s_flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint64_t inc = lead ? DSP_QUANTUM - (uint64_t)n + 1 : 1;
    const uint64_t old = __hip_atomic_fetch_add(cnt, inc, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = ((old + inc) & (DSP_QUANTUM - 1)) == 0;
  }
  __syncthreads();
  return *s_flag != 0;
}

__device__ __forceinline__ uint64_t dsp_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// MB: a compile-time bound on the requests (1, 4 or 16), which sizes the registers.
template <int MB>
__global__ void __launch_bounds__(DSP_NT) dsp_markov_kernel(DspArgs a) {
  __shared__ float s_lat[4096];                  // latents f32 [b][rank], b rank <= 4096
  __shared__ uint64_t s_key[DSP_WAVES][DSP_MAX_B];
  __shared__ uint32_t s_flag;
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int B = a.b, R = a.rank, j = a.j, G = a.nwg;
  for (int i = t; i < B * R; i += DSP_NT) {
    const int r = i / R, e = i % R;
    const int64_t prev = j == 0 ? a.anchor[r] : a.out[(int64_t)r * a.block + j - 1];
    s_lat[i] = (prev >= 0 && prev < a.v) ? bf16_to_f32(a.w1[prev * R + e]) : 0.f;
  }
  __syncthreads();

  const int64_t tiles = (a.v + WAVE - 1) / WAVE;
  const int chunks = R / 8;
  uint64_t best[MB];
#pragma unroll
  for (int r = 0; r < MB; ++r) best[r] = 0;
  for (int64_t tile = (int64_t)blockIdx.x * DSP_WAVES + w; tile < tiles;
       tile += (int64_t)G * DSP_WAVES) {
    const int64_t rows_t = a.v - tile * WAVE < WAVE ? a.v - tile * WAVE : WAVE;
    const int64_t row = tile * WAVE + lane;
    const bool live = lane < rows_t;
    const uint4* src = (const uint4*)(a.w2 + tile * WAVE * (int64_t)R) + lane;
    double acc[MB];
#pragma unroll
    for (int r = 0; r < MB; ++r) acc[r] = 0.0;
    for (int cb = 0; cb < chunks; cb += 8) {
      uint4 q[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        q[u] = {0u, 0u, 0u, 0u};
        if (live && cb + u < chunks) q[u] = src[(cb + u) * rows_t];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (cb + u < chunks) {
          const uint32_t qw[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
          float wv[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wv[2 * e] = __uint_as_float(qw[e] << 16);
            wv[2 * e + 1] = __uint_as_float(qw[e] & 0xffff0000u);
          }
#pragma unroll
          for (int r = 0; r < MB; ++r) {
            if (r < B) {
              const float* L = s_lat + r * R + (cb + u) * 8;
              double s0 = 0.0, s1 = 0.0;   // two chains; the sum stays exact
#pragma unroll
              for (int e = 0; e < 8; e += 2) {
                s0 += (double)(wv[e] * L[e]);        // exact bf16 x bf16
                s1 += (double)(wv[e + 1] * L[e + 1]);
              }
              acc[r] += s0 + s1;
            }
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < MB; ++r) {
      if (r < B && live) {
        const float bias = a.fp32_bias ? (float)acc[r] : bf16_from_f64(acc[r]);
        const float x = a.base[((int64_t)r * a.block + j) * a.base_stride + row] + bias;
        const uint64_t key = argmax_key(x, (uint32_t)row);
        best[r] = key > best[r] ? key : best[r];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < MB; ++r) {
    if (r < B) {
      const uint64_t k = wave_max_u64(best[r]);
      if (lane == 0) s_key[w][r] = k;
    }
  }
  __syncthreads();
  uint64_t* wg_keys = a.partial;                          // [b][G]
  uint64_t* group_keys = a.partial + (int64_t)B * G;      // [b][groups]
  if (t < B) {
    uint64_t m = s_key[0][t];
    for (int i = 1; i < DSP_WAVES; ++i) m = s_key[i][t] > m ? s_key[i][t] : m;
    __hip_atomic_store(&wg_keys[(int64_t)t * G + blockIdx.x], m, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  const int group = blockIdx.x / DSP_GROUP, groups = (G + DSP_GROUP - 1) / DSP_GROUP;
  const int g0 = group * DSP_GROUP, gn = G - g0 < DSP_GROUP ? G - g0 : DSP_GROUP;
  if (!dsp_arrive(&g_dsp_group[group], gn, blockIdx.x == g0, &s_flag)) return;
  // the group's last workgroup: its group's keys, one load per lane
  for (int r = w; r < B; r += DSP_WAVES) {
    uint64_t m = lane < gn ? dsp_load(&wg_keys[(int64_t)r * G + g0 + lane]) : 0;
    m = wave_max_u64(m);
    if (lane == 0)
      __hip_atomic_store(&group_keys[r * groups + group], m, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!dsp_arrive(&g_dsp_cnt, groups, group == 0, &s_flag)) return;
  // the last group: the pick and the confidence, one wave per request
  for (int r = w; r < B; r += DSP_WAVES) {
    uint64_t m = lane < groups ? dsp_load(&group_keys[r * groups + lane]) : 0;
    m = wave_max_u64(m);
    const int64_t at = (int64_t)r * a.block + j;
    if (lane == 0) a.out[at] = (int64_t)argmax_key_index(m);
    if (a.confidence) {
      float z = 0.f;
      const uint16_t* hid = a.pre_head + at * a.ps;
      for (int i = lane; i < a.h; i += WAVE) z += bf16_to_f32(hid[i]) * a.conf_w[i];
      for (int i = lane; i < R; i += WAVE) z += s_lat[r * R + i] * a.conf_w[a.h + i];
      z = wave_sum(z);
      if (lane == 0) {
        if (a.conf_b) z += *a.conf_b;
        a.confidence[at] = 1.f / (1.f + expf(-z));
      }
    }
  }
}

int64_t dsp_nwg(int64_t v) {
  const int64_t tiles = (v + WAVE - 1) / WAVE;
  const int64_t g = (tiles + DSP_WAVES - 1) / DSP_WAVES;
  return g < DSP_GRID ? g : DSP_GRID;
}

}  // namespace

// Bytes of a packed [n, k] bf16 weight: the same as the source, so the reference can view the
// buffer as [n, k] (snowllm/ops/dspark.py:11-14). k % 8 == 0.
SV_API int64_t snowllm_dspark_weight_bytes(int64_t n, int64_t k) {
  if (n <= 0 || k <= 0 || k % 8) return 0;
  return n * k * 2;
}

SV_API int snowllm_dspark_pack_weight(const void* raw, void* packed, int64_t n, int64_t k,
                                      void* stream) {
  if (!raw || !packed || n <= 0 || k <= 0 || k % 8 || raw == packed) return SV_EINVAL;
  const int64_t chunks = n * (k / 8);
  hipLaunchKernelGGL(dsp_pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)raw, (uint16_t*)packed, n, k);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Workspace of snowllm_dspark_markov: 8-byte keys per request for every workgroup and
// every group of workgroups.
SV_API int64_t snowllm_dspark_markov_workspace_bytes(int64_t b, int64_t v, int64_t rank,
                                                     int64_t block) {
  (void)rank;
  (void)block;
  if (b <= 0 || v <= 0) return 0;
  const int64_t g = dsp_nwg(v);
  return ((b * (g + (g + DSP_GROUP - 1) / DSP_GROUP) * 8 + 255) / 256) * 256;
}

// base f32 [b * block, >= v] (row stride base_stride), w1 bf16 [v, rank], w2 packed by
// snowllm_dspark_pack_weight, anchor i64 [b] -> out i64 [b, block]; with confidence (f32
// [b, block]) also pre_head bf16 [b * block, >= h] (row stride ps), conf_weight f32
// [h + rank] and an optional scalar conf_bias. fp32_bias keeps the bias in fp32 instead of
// bf16. b <= 16, rank % 8 == 0, rank <= 512, b rank <= 4096. Calls on one device must be
// stream-ordered.
SV_API int snowllm_dspark_markov(const void* base, const void* w1, const void* w2,
                                 const int64_t* anchor, const void* pre_head,
                                 const float* conf_weight, const float* conf_bias, int64_t* out,
                                 float* confidence, void* workspace, int64_t b, int64_t v,
                                 int64_t rank, int64_t block, int64_t base_stride, int64_t h,
                                 int64_t ps, int64_t workspace_bytes, int fp32_bias,
                                 void* stream) {
  if (!base || !w1 || !w2 || !anchor || !out || !workspace) return SV_EINVAL;
  if (b <= 0 || b > DSP_MAX_B || v <= 0 || v > DSP_MAX_V || rank <= 0 || rank % 8 ||
      rank > DSP_MAX_RANK || b * rank > 4096 || block <= 0 || block > 1024 || base_stride < v)
    return SV_EINVAL;
  if (confidence && (!pre_head || !conf_weight || h <= 0 || ps < h)) return SV_EINVAL;
  if (workspace_bytes < snowllm_dspark_markov_workspace_bytes(b, v, rank, block)) return SV_EINVAL;
  DspArgs a{(const float*)base, (const uint16_t*)w1, (const uint16_t*)w2, anchor,
            (const uint16_t*)pre_head, conf_weight, conf_bias, out, confidence,
            (uint64_t*)workspace, v, base_stride, ps, (int)b, (int)rank, (int)block,
            confidence ? (int)h : 0, (int)dsp_nwg(v), fp32_bias != 0, 0};
  for (int j = 0; j < block; ++j) {
    a.j = j;
    if (b == 1)
      hipLaunchKernelGGL(dsp_markov_kernel<1>, dim3((unsigned)a.nwg), dim3(DSP_NT), 0,
                         (hipStream_t)stream, a);
    else if (b <= 4)
      hipLaunchKernelGGL(dsp_markov_kernel<4>, dim3((unsigned)a.nwg), dim3(DSP_NT), 0,
                         (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL(dsp_markov_kernel<DSP_MAX_B>, dim3((unsigned)a.nwg), dim3(DSP_NT), 0,
                         (hipStream_t)stream, a);
    SV_CHECK_LAUNCH();
  }
  return SV_OK;
}
