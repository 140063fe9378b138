// DFlash 2 candidate selector on gfx950: the walk that turns a draft's logits into the
// proposed path (and, when sampling, the candidate lists and probabilities that the
// rejection step reads back by request slot).
//
// Semantics (snowllm/ops/dflash.py:164-198; checked by tests/test_dflash_sampling.py:44-75
// and tests/test_dflash_selector_topk.py:42-61): for batch row b and position j, with
// row = b * ell + j and prev the token picked at j - 1 (anchor[b] at j = 0),
//   (values, cand) = the 16 largest logits of the row, stable descending (NaN as -inf,
//                    ties to the lower id, -0 == +0);
//   corr[c]  = sum_r pred[prev, r] * hp[row, r] * succ[cand[c], r]            (greedy rows)
//            = bf16(sum_r bf16(pred[prev, r] * hp[row, r]) * succ[cand[c], r]) (sampling)
//   scores   = values + corr;
//   greedy (temperature <= 0 or no temperature): pick = first argmax, q = one-hot;
//   sampling: q = softmax(scores / T), pick = #(u[b, j] >= cumsum(q)) clamped to 15;
//   path[b, j] = cand[pick]; candidate_ids[slot, j] = cand; probabilities[slot, j] = q.
//
// Three launches, none of them with a cross-workgroup wait:
//   1. select_chunks: each (row, 4096-logit chunk) finds its top 16 (threshold = the 16th
//      largest of the 256 per-thread maxima, so at most 256 survivors, ranked exactly);
//   2. select_table: per row, merge the chunk lists of the row and of the row before it;
//      then, one wave per previous pick p (the previous row's candidate p, or the anchor at
//      j = 0), the 16 corrections of the row given p and the whole step (scores, q, pick):
//      every position is solved for all 16 possible predecessors at once;
//   3. select_walk: one wave per batch row follows the tabulated picks from the anchor.
//
// Arithmetic is canonical so that the host oracle reproduces it bit for bit: the products
// are exact in binary32 (bf16 x bf16 x bf16 fits 24 bits), each lane sums its R/64 terms in
// order and the 64 lane sums meet in a balanced binary tree in lane order; the softmax uses
// canon_exp, fixed-point sums and canon_div as the acceptance kernels do.
#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int SEL_K = 16;            // candidates per position (selector_top_k)
constexpr int SEL_RANK = 256;        // selector_rank of the DFlash 2 draft geometry
constexpr int SEL_CHUNK = 4096;
constexpr int SEL_NT = 256;
constexpr int SEL_RUN = SEL_CHUNK / SEL_NT;
constexpr int SEL_CHUNKS_MAX = 64;   // vocab <= 262144: the chunk lists merge in one wave
constexpr int SEL_ELL_MAX = 32;

struct SelectScratch {
  uint64_t* chunk_keys;  // [n][SEL_CHUNKS_MAX][16]
  uint64_t* top_keys;    // [n][16]
  float* q;              // [n][16 prev][16 cand]: the probabilities given previous pick p
  int32_t* pick;         // [n][16 prev]: the pick given previous pick p
};

inline size_t sel_align(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline SelectScratch select_scratch(void* base, int64_t n) {
  SelectScratch s;
  char* p = (char*)base;
  s.chunk_keys = (uint64_t*)p;
  p += sel_align((size_t)n * SEL_CHUNKS_MAX * SEL_K * 8);
  s.top_keys = (uint64_t*)p;
  p += sel_align((size_t)n * SEL_K * 8);
  s.q = (float*)p;
  p += sel_align((size_t)n * SEL_K * SEL_K * 4);
  s.pick = (int32_t*)p;
  return s;
}

inline int64_t select_scratch_size(int64_t n) {
  return (int64_t)(sel_align((size_t)n * SEL_CHUNKS_MAX * SEL_K * 8) +
                   sel_align((size_t)n * SEL_K * 8) + sel_align((size_t)n * SEL_K * SEL_K * 4) +
                   sel_align((size_t)n * SEL_K * 4));
}

// key = ord(value) << 32 | (2^32 - 1 - id): larger key = larger value, then lower id. Every
// key of a real logit is nonzero (ord(-inf) = 0x007fffff), so 0 marks an empty slot.
__device__ __forceinline__ uint64_t sel_key(float v, uint32_t id) {
  return ((uint64_t)ord_key(v) << 32) | (uint64_t)(0xffffffffu - id);
}
__device__ __forceinline__ uint32_t key_id(uint64_t k) { return 0xffffffffu - (uint32_t)k; }
__device__ __forceinline__ float key_value(uint64_t k) { return ord_key_to_float((uint32_t)(k >> 32)); }

__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  const uint32_t hi = wave_max_u32_dpp((uint32_t)(k >> 32));
  const uint32_t lo = wave_max_u32_dpp((uint32_t)(k >> 32) == hi ? (uint32_t)k : 0u);
  return ((uint64_t)hi << 32) | lo;
}

// ---------------------------------------------------------------------------------------
// 1. chunk top-16. Thread t holds logits c * 4096 + 256 i + t, i < 16 (coalesced loads).
// The 16 largest keys of the chunk are among the keys >= T, T = the 16th largest per-thread
// maximum: only the (at most 16) threads whose maximum is >= T hold such keys.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(SEL_NT) select_chunks(const float* __restrict__ logits,
                                                        int64_t V, SelectScratch sc) {
  __shared__ uint64_t s_max[SEL_NT];
  __shared__ uint64_t s_cand[SEL_NT];
  __shared__ uint64_t s_thr;
  __shared__ uint32_t s_count;
  const int c = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int t = threadIdx.x;
  const float* x = logits + row * V;
  uint64_t keys[SEL_RUN];
  uint64_t mine = 0;
  float xv[SEL_RUN];
#pragma unroll
  for (int i = 0; i < SEL_RUN; ++i) {  // every load in flight before the first key
    const int64_t id = (int64_t)c * SEL_CHUNK + i * SEL_NT + t;
    xv[i] = x[id < V ? id : V - 1];
  }
#pragma unroll
  for (int i = 0; i < SEL_RUN; ++i) {
    const int64_t id = (int64_t)c * SEL_CHUNK + i * SEL_NT + t;
    keys[i] = id < V ? sel_key(xv[i], (uint32_t)id) : 0ull;
    mine = keys[i] > mine ? keys[i] : mine;
  }
  s_max[t] = mine;
  if (t == 0) {
    s_thr = 1ull;  // fewer than 16 live threads: every live key survives
    s_count = 0u;
  }
  __syncthreads();
  int above = 0;
#pragma unroll 32
  for (int u = 0; u < SEL_NT; ++u) above += s_max[u] > mine;
  if (above == SEL_K - 1 && mine != 0ull) s_thr = mine;
  __syncthreads();
  const uint64_t thr = s_thr;
  if (mine >= thr) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < SEL_RUN; ++i) n += keys[i] >= thr;
    uint32_t pos = atomicAdd(&s_count, (uint32_t)n);
#pragma unroll
    for (int i = 0; i < SEL_RUN; ++i)
      if (keys[i] >= thr) s_cand[pos++] = keys[i];
  }
  __syncthreads();
  const int n_cand = (int)s_count;
  uint64_t* out = sc.chunk_keys + (row * SEL_CHUNKS_MAX + c) * SEL_K;
  if (t < n_cand) {
    const uint64_t k = s_cand[t];
    int rank = 0;
#pragma unroll 8
    for (int u = 0; u < n_cand; ++u) rank += s_cand[u] > k;
    if (rank < SEL_K) out[rank] = k;
  } else if (t < SEL_K) {
    out[t] = 0ull;
  }
}

// Merge the C sorted chunk lists of a row (lane = chunk) into the row's top 16, in order.
__device__ __forceinline__ void merge_row(const SelectScratch& sc, int64_t row, int C, int lane,
                                         uint64_t* dst) {
  uint64_t list[SEL_K];
  const uint64_t* src = sc.chunk_keys + (row * SEL_CHUNKS_MAX + lane) * SEL_K;
#pragma unroll
  for (int i = 0; i < SEL_K; ++i) list[i] = lane < C ? src[i] : 0ull;
  int h = 0;
  uint64_t head = list[0];
  for (int k = 0; k < SEL_K; ++k) {
    const uint64_t m = wave_max_key(head);
    if (lane == 0) dst[k] = m;
    if (head == m && m != 0ull) {
      ++h;
      uint64_t nx = 0ull;
#pragma unroll
      for (int i = 1; i < SEL_K; ++i) nx = h == i ? list[i] : nx;
      head = nx;
    }
  }
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(__builtin_bit_cast(uint16_t, (__bf16)f));
}

// ---------------------------------------------------------------------------------------
// 2. per row: its top 16 (wave 0), the previous row's (wave 1), then wave p tabulates
// corr[p][c] for previous token p (the previous row's candidate p, or the anchor at j = 0).
// ---------------------------------------------------------------------------------------
template <int E>  // terms per lane: r = lane * E + i, R = 64 E
// (The merge's inputs come first: they arrive preloaded in SGPRs; grid (ell, b), no division.)
__global__ void __launch_bounds__(SEL_K * 64) select_table(
    uint64_t* __restrict__ h_chunk_keys, uint64_t* __restrict__ h_top_keys, int C, int ell32,
    const uint16_t* __restrict__ hp, const uint16_t* __restrict__ pred,
    const uint16_t* __restrict__ succ, const int64_t* __restrict__ anchor,
    const float* __restrict__ temperature, const float* __restrict__ uniform,
    SelectScratch sc) {
  constexpr int R = 64 * E;
  __shared__ uint64_t s_top[SEL_K];
  __shared__ uint64_t s_prev[SEL_K];
  sc.chunk_keys = h_chunk_keys, sc.top_keys = h_top_keys;
  const int64_t ell = ell32, j = blockIdx.x, b = blockIdx.y;
  const int64_t row = b * ell + j;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w == 0) merge_row(sc, row, C, lane, s_top);
  if (w == 1 && j > 0) merge_row(sc, row - 1, C, lane, s_prev);
  __syncthreads();
  if (w == 0 && lane < SEL_K) sc.top_keys[row * SEL_K + lane] = s_top[lane];
  if (j == 0 && w > 0) return;
  const bool sampling = temperature != nullptr && temperature[b] > 0.0f;
  const int64_t prev = j == 0 ? anchor[b] : (int64_t)key_id(s_prev[w]);
  uint16_t pv[E], hv[E], sv[SEL_K][E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    pv[i] = pred[prev * R + lane * E + i];
    hv[i] = hp[row * R + lane * E + i];
  }
#pragma unroll
  for (int c = 0; c < SEL_K; ++c) {
    const uint16_t* sr = succ + (int64_t)key_id(s_top[c]) * R + lane * E;
#pragma unroll
    for (int i = 0; i < E; ++i) sv[c][i] = sr[i];
  }
  float a[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float prod = bf16_to_f32(pv[i]) * bf16_to_f32(hv[i]);
    a[i] = sampling ? round_bf16(prod) : prod;
  }
  float mine = 0.f;  // lane c: corr[c]
#pragma unroll
  for (int c = 0; c < SEL_K; ++c) {
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) part = part + a[i] * bf16_to_f32(sv[c][i]);
    float dot = wave_sum_dpp(part);
    if (sampling) dot = round_bf16(dot);
    mine = lane == c ? dot : mine;
  }
  // the step itself for previous pick p = w: lane c holds candidate c
  const bool live = lane < SEL_K;
  const float score = key_value(s_top[lane & (SEL_K - 1)]) + mine;
  float q;
  int pick;
  if (!sampling) {
    // first maximum: largest ordered score, then the lowest slot
    const uint32_t k = live ? ord_key(score) : 0u;
    const uint32_t best = wave_max_u32_dpp(k);
    pick = (int)__builtin_ctzll(__ballot(live && k == best));
    q = lane == pick ? 1.0f : 0.0f;
  } else {
    const float x = __fdiv_rn(score, temperature[b]);
    const float M = ord_key_to_float(wave_max_u32_dpp(live ? ord_key(x) : 0u));
    const float e = live ? canon_exp(x - M) : 0.0f;
    // fixed-point terms are < 2^45: 22-bit halves sum exactly in 32 bits over 16 lanes
    const uint64_t fe = canon_fix(e);
    const uint64_t Z = ((uint64_t)wave_sum_u32_dpp((uint32_t)(fe >> 22)) << 22) +
                       wave_sum_u32_dpp((uint32_t)(fe & 0x3fffffu));
    const float Zf = canon_unfix(Z);
    q = (live && Zf > 0.0f) ? canon_div(e, Zf) : 0.0f;
    // pick = #{c : fixed-point prefix_incl(c) <= floor(u * 2^44)}, clamped to 15
    const uint64_t fq = canon_fix(q);
    const uint64_t pre = ((uint64_t)row_scan_u32_dpp((uint32_t)(fq >> 22)) << 22) +
                         row_scan_u32_dpp((uint32_t)(fq & 0x3fffffu));
    const uint64_t target = canon_scale_floor(uniform[row], 1ull << SV_FIX_BITS);
    const int n = (int)__popcll(__ballot(live && pre <= target));
    pick = n < SEL_K - 1 ? n : SEL_K - 1;
  }
  if (live) sc.q[(row * SEL_K + w) * SEL_K + lane] = q;
  if (lane == 0) sc.pick[row * SEL_K + w] = pick;
}

// ---------------------------------------------------------------------------------------
// 3. the walk: follow the tabulated picks from p = 0 (the anchor) and emit the lists.
// ---------------------------------------------------------------------------------------
// (The tables' pointers come first: they arrive preloaded in SGPRs.)
__global__ void __launch_bounds__(64) select_walk(int32_t* __restrict__ h_pick,
                                                  uint64_t* __restrict__ h_top_keys,
                                                  float* __restrict__ h_q, int64_t ell,
                                                  const int32_t* __restrict__ slots,
                                                  int64_t* __restrict__ path,
                                                  int64_t* __restrict__ cand_out,
                                                  float* __restrict__ q_out, SelectScratch sc) {
  sc.pick = h_pick, sc.top_keys = h_top_keys, sc.q = h_q;
  __shared__ int32_t s_pick[SEL_ELL_MAX][SEL_K];
  __shared__ __attribute__((aligned(16))) uint64_t s_top[SEL_ELL_MAX][SEL_K];
  __shared__ __attribute__((aligned(16))) float s_q[SEL_ELL_MAX][SEL_K][SEL_K];
  const int64_t b = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t row0 = b * ell;
  const bool lists = cand_out != nullptr;
  // the batch row's tables in 16-byte words, all loads in flight together
  const float4* psrc = (const float4*)(sc.pick + row0 * SEL_K);
#pragma unroll 2
  for (int i = lane; i < ell * SEL_K / 4; i += 64) ((float4*)&s_pick[0][0])[i] = psrc[i];
  const float4* ksrc = (const float4*)(sc.top_keys + row0 * SEL_K);
#pragma unroll 2
  for (int i = lane; i < ell * SEL_K / 2; i += 64) ((float4*)&s_top[0][0])[i] = ksrc[i];
  if (lists) {
    const float4* qsrc = (const float4*)(sc.q + row0 * SEL_K * SEL_K);
#pragma unroll 8
    for (int i = lane; i < ell * SEL_K * SEL_K / 4; i += 64) ((float4*)&s_q[0][0][0])[i] = qsrc[i];
  }
  __syncthreads();
  const int64_t slot = lists ? (int64_t)slots[b] : 0;
  int p = 0;
  for (int64_t j = 0; j < ell; ++j) {
    const int pick = s_pick[j][p];
    if (lane == 0) path[row0 + j] = (int64_t)key_id(s_top[j][pick]);
    if (lists && lane < SEL_K) {
      cand_out[(slot * ell + j) * SEL_K + lane] = (int64_t)key_id(s_top[j][lane]);
      q_out[(slot * ell + j) * SEL_K + lane] = s_q[j][p][lane];
    }
    p = pick;
  }
}

int launch_select(const void* hp, const float* logits, const void* pred, const void* succ,
                  const int64_t* anchor, const float* temperature, const float* uniform,
                  const int32_t* slots, int64_t* path, int64_t* cand, float* q, void* scratch,
                  int64_t b, int64_t ell, int64_t V, int64_t R, hipStream_t s) {
  if (b <= 0 || ell <= 0 || ell > SEL_ELL_MAX || V < SEL_K ||
      V > (int64_t)SEL_CHUNK * SEL_CHUNKS_MAX || (R != 64 && R != 128 && R != 256 && R != 512) ||
      b * ell > 65535 || !scratch)
    return SV_EINVAL;
  const int64_t n = b * ell;
  const int C = (int)((V + SEL_CHUNK - 1) / SEL_CHUNK);
  const SelectScratch sc = select_scratch(scratch, n);
  hipLaunchKernelGGL(select_chunks, dim3((unsigned)C, (unsigned)n), dim3(SEL_NT), 0, s, logits,
                     V, sc);
  SV_CHECK_LAUNCH();
  auto table = R == 64 ? select_table<1> : R == 128 ? select_table<2>
             : R == 256 ? select_table<4> : select_table<8>;
  hipLaunchKernelGGL(table, dim3((unsigned)ell, (unsigned)b), dim3(SEL_K * 64), 0, s,
                     sc.chunk_keys, sc.top_keys, C, (int)ell, (const uint16_t*)hp,
                     (const uint16_t*)pred, (const uint16_t*)succ, anchor, temperature, uniform,
                     sc);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(select_walk, dim3((unsigned)b), dim3(64), 0, s, sc.pick, sc.top_keys, sc.q,
                     ell, slots, path, cand, q, sc);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

// snowllm/_capi.py:285 -- scratch of snowllm_draft_select / _sample for n = b * ell rows.
SV_API int64_t snowllm_draft_select_scratch_bytes(int64_t n) {
  if (n <= 0) return 0;
  return select_scratch_size(n);
}

// snowllm/_capi.py:286-287 (ops.dflash.select_path without temperature): greedy walk,
// path only. hp bf16 [b*ell, 256], logits f32 [b*ell, v], pred/succ bf16 [v, 256].
SV_API int snowllm_draft_select(const void* hp, const float* logits, const void* pred,
                                const void* succ, const int64_t* anchor, int64_t* path,
                                void* scratch, int64_t b, int64_t ell, int64_t v, void* stream) {
  return launch_select(hp, logits, pred, succ, anchor, nullptr, nullptr, nullptr, path, nullptr,
                       nullptr, scratch, b, ell, v, SEL_RANK, (hipStream_t)stream);
}

// snowllm/_capi.py:288 (ops.dflash.select_path with temperature): per-row greedy or
// sampling walk; candidate ids i64 and probabilities f32 [slots, ell, 16] at slots[b].
SV_API int snowllm_draft_sample(const void* hp, const float* logits, const void* pred,
                                const void* succ, const int64_t* anchor, const float* temperature,
                                const float* uniform, const int32_t* slots, int64_t* path,
                                int64_t* candidate_ids, float* probabilities, void* scratch,
                                int64_t b, int64_t ell, int64_t v, int64_t top_k, void* stream) {
  if (top_k != SEL_K || !temperature || !uniform || !slots || !candidate_ids || !probabilities)
    return SV_EINVAL;
  return launch_select(hp, logits, pred, succ, anchor, temperature, uniform, slots, path,
                       candidate_ids, probabilities, scratch, b, ell, v, SEL_RANK,
                       (hipStream_t)stream);
}

// Extension (no counterpart in the reference): the selector at another codebook rank R
// (64, 128, 256 or 512); temperature == NULL gives the greedy walk without lists.
SV_API int snowverify_draft_select(const void* hp, const float* logits, const void* pred,
                                   const void* succ, const int64_t* anchor,
                                   const float* temperature, const float* uniform,
                                   const int32_t* slots, int64_t* path, int64_t* candidate_ids,
                                   float* probabilities, void* scratch, int64_t b, int64_t ell,
                                   int64_t v, int64_t rank, void* stream) {
  if (temperature && (!uniform || !slots || !candidate_ids || !probabilities)) return SV_EINVAL;
  return launch_select(hp, logits, pred, succ, anchor, temperature, uniform, slots, path,
                       temperature ? candidate_ids : nullptr, temperature ? probabilities : nullptr,
                       scratch, b, ell, v, rank, (hipStream_t)stream);
}
