// Acceptance-side kernels of the verify step: argmax, greedy prefix acceptance, temperature
// softmax, top-k/top-p candidate lists, rejection sampling with residual resample, and
// ordinary top-k/top-p sampling.
//
// Vocabulary-wide work is split into 4096-element chunks so that a handful of rows still
// spreads over hundreds of workgroups. Every sum that feeds a sampling decision is taken in
// 44-bit fixed point (canon_fix), which makes the result independent of how the chunks and
// lanes are combined; maxima are exact in any order. The host oracle restates exactly this
// arithmetic, so accept lengths, emitted ids and probabilities agree bit for bit.
#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int CHUNK = 4096;
constexpr int NT = 256;                // threads per chunk workgroup
constexpr int RUN = CHUNK / NT;        // contiguous elements per thread in scan kernels
constexpr int ROWS_MAX = 2048;         // rows per argmax / reject launch
constexpr int CHUNKS_MAX = 128;        // vocab < 2^19 (fixed-point headroom)
constexpr int64_t VOCAB_MAX = (int64_t)CHUNK * CHUNKS_MAX;

// Library-owned scratch for the entry points whose reference signature carries no
// workspace (argmax, draft_reject). Calls on one device must be stream-ordered.
__device__ uint64_t g_chunk_keys[ROWS_MAX * CHUNKS_MAX];
__device__ uint64_t g_chunk_sums[ROWS_MAX * CHUNKS_MAX * 2];
__device__ int32_t g_first[ROWS_MAX];

inline int chunks_of(int64_t n) { return (int)((n + CHUNK - 1) / CHUNK); }

// ---------------------------------------------------------------------------------------
// argmax
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(NT) argmax_chunks(const float* __restrict__ logits,
                                                    int64_t V, int C) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  const float* x = logits + (int64_t)row * V;
  const int64_t base = (int64_t)c * CHUNK;
  uint64_t best = 0;
#pragma unroll 4
  for (int k = 0; k < RUN; ++k) {
    int64_t i = base + threadIdx.x + (int64_t)k * NT;
    if (i < V) {
      uint64_t key = argmax_key(x[i], (uint32_t)i);
      best = key > best ? key : best;
    }
  }
  best = block_max_u64<NT>(best, red);
  if (threadIdx.x == 0) g_chunk_keys[row * CHUNKS_MAX + c] = best;
}

__global__ void __launch_bounds__(WAVE) argmax_final(int64_t* __restrict__ out, int C) {
  const int row = blockIdx.x;
  uint64_t best = 0;
  for (int c = threadIdx.x; c < C; c += WAVE) {
    uint64_t k = g_chunk_keys[row * CHUNKS_MAX + c];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if (threadIdx.x == 0) out[row] = (int64_t)argmax_key_index(best);
}

// ---------------------------------------------------------------------------------------
// greedy acceptance: accepted = 1 + number of leading positions where the verified token
// equals the draft token.
// ---------------------------------------------------------------------------------------
__global__ void spec_accept_kernel(const int64_t* __restrict__ tokens,
                                   const int64_t* __restrict__ drafts, int64_t* __restrict__ acc,
                                   int64_t b, int64_t t, int64_t ts, int64_t ds) {
  int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= b) return;
  int64_t a = 1;
  for (int64_t j = 0; j + 1 < t; ++j) {
    if (tokens[r * ts + j] != drafts[r * ds + j]) break;
    ++a;
  }
  acc[r] = a;
}

// ---------------------------------------------------------------------------------------
// temperature softmax into a dense [rows, vocab] buffer. Row statistics live in the tail of
// the sampling workspace: per-chunk maxima (u32 keys) and per-chunk fixed-point sums.
// ---------------------------------------------------------------------------------------
struct SoftmaxTail {
  uint32_t* max_keys;  // [rows, C]
  uint64_t* sums;      // [rows, C]
};

__device__ __forceinline__ float row_temperature(const float* temperature, int row) {
  float t = temperature ? temperature[row] : 1.0f;
  return (t > 0.0f) ? t : 1.0f;
}

// A thread's RUN elements base + k NT of a row of V, every load issued before the first use
// (indices past the row read its last element; callers skip them).
__device__ __forceinline__ void load_run(const float* __restrict__ x, int64_t base, int64_t V,
                                         float (&v)[RUN]) {
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    const int64_t i = base + (int64_t)k * NT;
    v[k] = x[i < V ? i : V - 1];
  }
}

__global__ void __launch_bounds__(NT) softmax_max(const float* __restrict__ logits, int64_t V,
                                                  const float* __restrict__ temperature,
                                                  SoftmaxTail tail, int C) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  const float* x = logits + (int64_t)row * V;
  const float T = row_temperature(temperature, row);
  uint64_t best = 0;
  const int64_t base = (int64_t)c * CHUNK + threadIdx.x;
  float xv[RUN];
  load_run(x, base, V, xv);
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    if (base + (int64_t)k * NT < V) {
      uint32_t key = ord_key(__fdiv_rn(xv[k], T));
      best = key > best ? key : best;
    }
  }
  best = block_max_u64<NT>(best, red);
  if (threadIdx.x == 0) tail.max_keys[row * C + c] = (uint32_t)best;
}

__device__ __forceinline__ float row_max_from_keys(const uint32_t* keys, int C) {
  uint32_t m = 0;
  for (int c = 0; c < C; ++c) m = keys[c] > m ? keys[c] : m;
  return ord_key_to_float(m);
}

__global__ void __launch_bounds__(NT) softmax_exp(const float* __restrict__ logits, int64_t V,
                                                  const float* __restrict__ temperature,
                                                  float* __restrict__ dense, SoftmaxTail tail,
                                                  int C) {
  __shared__ uint64_t red[NT / WAVE];
  __shared__ float s_max;
  const int c = blockIdx.x, row = blockIdx.y;
  if (threadIdx.x < WAVE) {  // chunk maxima, one wave (exact in any order)
    const uint32_t* keys = tail.max_keys + row * C;
    uint32_t m = 0;
    for (int i = threadIdx.x; i < C; i += WAVE) m = keys[i] > m ? keys[i] : m;
    m = wave_max(m);
    if (threadIdx.x == 0) s_max = ord_key_to_float(m);
  }
  __syncthreads();
  const float M = s_max;
  const float* x = logits + (int64_t)row * V;
  float* e = dense + (int64_t)row * V;
  const float T = row_temperature(temperature, row);
  uint64_t sum = 0;
  const int64_t base = (int64_t)c * CHUNK + threadIdx.x;
  float xv[RUN];
  load_run(x, base, V, xv);
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    const int64_t i = base + (int64_t)k * NT;
    if (i < V) {
      float v = canon_exp(__fsub_rn(__fdiv_rn(xv[k], T), M));
      e[i] = v;
      sum += canon_fix(v);
    }
  }
  sum = block_sum_u64<NT>(sum, red);
  if (threadIdx.x == 0) tail.sums[row * C + c] = sum;
}

__global__ void __launch_bounds__(NT) softmax_norm(float* __restrict__ dense, int64_t V,
                                                   SoftmaxTail tail, int C) {
  __shared__ float s_z;
  const int c = blockIdx.x, row = blockIdx.y;
  if (threadIdx.x < WAVE) {  // fixed-point chunk sums, one wave (exact in any order)
    uint64_t z = 0;
    for (int i = threadIdx.x; i < C; i += WAVE) z += tail.sums[row * C + i];
    z = wave_sum_u64(z);
    if (threadIdx.x == 0) s_z = canon_unfix(z);
  }
  __syncthreads();
  const float Z = s_z;
  float* e = dense + (int64_t)row * V;
  const int64_t base = (int64_t)c * CHUNK + threadIdx.x;
  float ev[RUN];
  load_run(e, base, V, ev);
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    const int64_t i = base + (int64_t)k * NT;
    if (i < V) e[i] = (Z > 0.0f) ? canon_div(ev[k], Z) : 0.0f;
  }
}

// ---------------------------------------------------------------------------------------
// top-k / top-p candidate lists.
//
// Rows that keep the whole vocabulary without nucleus truncation are written in vocabulary
// order (ids 0..V-1) with the dense probabilities unchanged. Rows with k <= TOPK_MAX are
// selected by a four-pass radix select on the ordered probability keys (ties resolved to the
// lower vocabulary index), sorted by (probability desc, index asc), renormalised over the
// k survivors, truncated by top-p on the exclusive fixed-point prefix, and renormalised
// again. Unused slots of the width are (0, -1).
// ---------------------------------------------------------------------------------------
constexpr int TOPK_NT = 1024;
constexpr int TOPK_MAX = 1024;

struct TopkShared {
  uint32_t hist[256];
  uint64_t red[TOPK_NT / WAVE];
  uint64_t sel_key[TOPK_MAX];  // (ord key << 32) | ~index : descending order == wanted order
  uint64_t fix[TOPK_MAX];
  int32_t n_sel;
};

// Radix select: returns the ordered key tau of the k-th largest element of x[0..n) and the
// number of elements strictly above it.
__device__ void radix_threshold(const float* x, int64_t n, int k, TopkShared& sh,
                                uint32_t* tau_out, int* above_out) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;  // rank still to find among elements matching the prefix
  int above = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = threadIdx.x; i < 256; i += TOPK_NT) sh.hist[i] = 0;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += TOPK_NT) {
      uint32_t key = ord_key(x[i]);
      if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 0xff], 1u);
    }
    __syncthreads();
    // walk the digits from the top until the remaining rank falls inside one bucket
    __shared__ uint32_t s_digit;
    __shared__ int s_before;
    if (threadIdx.x == 0) {
      int acc = 0;
      int d = 255;
      for (; d >= 0; --d) {
        int h = (int)sh.hist[d];
        if (acc + h >= remaining) break;
        acc += h;
      }
      if (d < 0) d = 0;
      s_digit = (uint32_t)d;
      s_before = acc;
    }
    __syncthreads();
    above += s_before;
    remaining -= s_before;
    prefix |= s_digit << shift;
    mask |= 0xffu << shift;
    __syncthreads();
  }
  *tau_out = prefix;
  *above_out = above;
}

__global__ void __launch_bounds__(TOPK_NT) topk_topp_rows(
    const float* __restrict__ dense, float* __restrict__ values, int64_t* __restrict__ ids,
    int64_t V, int64_t width, const int32_t* __restrict__ top_k,
    const float* __restrict__ top_p) {
  __shared__ TopkShared sh;
  const int row = blockIdx.x;
  const int chunk = blockIdx.y;  // identity rows are copied chunk by chunk; selection uses chunk 0
  const float* p = dense + (int64_t)row * V;
  float* out_v = values + (int64_t)row * width;
  int64_t* out_i = ids + (int64_t)row * width;
  int64_t k64 = top_k ? (int64_t)top_k[row] : V;
  if (k64 <= 0 || k64 > V) k64 = V;
  const float tp = top_p ? top_p[row] : 1.0f;
  const bool nucleus = tp < 1.0f;

  if (k64 >= V && !nucleus) {
    const int64_t end = ((int64_t)chunk + 1) * CHUNK < width ? ((int64_t)chunk + 1) * CHUNK : width;
    for (int64_t i = (int64_t)chunk * CHUNK + threadIdx.x; i < end; i += TOPK_NT) {
      bool in = i < V;
      out_v[i] = in ? p[i] : 0.0f;
      out_i[i] = in ? i : -1;
    }
    return;
  }
  if (chunk != 0) return;
  if (k64 > width) {
    // a top-k wider than the list cannot be written: the row is marked with id -2 and NaN
    // values (callers size the width as the batch's largest top-k, as the reference's do)
    for (int64_t i = threadIdx.x; i < width; i += TOPK_NT) {
      out_v[i] = __builtin_nanf("");
      out_i[i] = -2;
    }
    return;
  }
  if (k64 > TOPK_MAX) return;  // the wide-list kernels below write the row
  const int k = (int)k64;
  uint32_t tau;
  int above;
  radix_threshold(p, V, k, sh, &tau, &above);
  const int ties_needed = k - above;

  // Compaction in vocabulary order: thread t owns a contiguous run so that the exclusive scan
  // of tie counts yields the lowest-index ties.
  const int64_t run = (V + TOPK_NT - 1) / TOPK_NT;
  const int64_t lo = (int64_t)threadIdx.x * run;
  const int64_t hi = lo + run < V ? lo + run : V;
  uint32_t my_gt = 0, my_eq = 0;
  for (int64_t i = lo; i < hi; ++i) {
    uint32_t key = ord_key(p[i]);
    my_gt += key > tau;
    my_eq += key == tau;
  }
  // exclusive scans of (gt, eq) counts over threads
  __shared__ uint32_t sgt[TOPK_NT];
  __shared__ uint32_t seq[TOPK_NT];
  sgt[threadIdx.x] = my_gt;
  seq[threadIdx.x] = my_eq;
  __syncthreads();
  for (int off = 1; off < TOPK_NT; off <<= 1) {
    uint32_t a = threadIdx.x >= (unsigned)off ? sgt[threadIdx.x - off] : 0;
    uint32_t b = threadIdx.x >= (unsigned)off ? seq[threadIdx.x - off] : 0;
    __syncthreads();
    sgt[threadIdx.x] += a;
    seq[threadIdx.x] += b;
    __syncthreads();
  }
  uint32_t gt_before = sgt[threadIdx.x] - my_gt;
  uint32_t eq_before = seq[threadIdx.x] - my_eq;
  uint32_t slot = gt_before + (eq_before < (uint32_t)ties_needed ? eq_before : ties_needed);
  uint32_t eq_seen = eq_before;
  for (int64_t i = lo; i < hi; ++i) {
    uint32_t key = ord_key(p[i]);
    bool take = key > tau;
    if (key == tau) {
      take = eq_seen < (uint32_t)ties_needed;
      ++eq_seen;
    }
    if (take) {
      sh.sel_key[slot] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
      ++slot;
    }
  }
  __syncthreads();
  // bitonic sort (descending) over the next power of two
  int n2 = 1;
  while (n2 < k) n2 <<= 1;
  for (int i = k + threadIdx.x; i < n2; i += TOPK_NT) sh.sel_key[i] = 0;
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < n2; i += TOPK_NT) {
        int j = i ^ stride;
        if (j > i) {
          bool desc = (i & size) == 0;
          uint64_t a = sh.sel_key[i], b = sh.sel_key[j];
          if (desc ? (a < b) : (a > b)) {
            sh.sel_key[i] = b;
            sh.sel_key[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // renormalise over the k survivors
  uint64_t part = 0;
  for (int i = threadIdx.x; i < k; i += TOPK_NT)
    part += canon_fix(p[0xffffffffu - (uint32_t)(sh.sel_key[i] & 0xffffffffu)]);
  uint64_t S = block_sum_u64<TOPK_NT>(part, sh.red);
  const float Sf = canon_unfix(S);
  for (int i = threadIdx.x; i < k; i += TOPK_NT) {
    uint32_t idx = 0xffffffffu - (uint32_t)(sh.sel_key[i] & 0xffffffffu);
    float v = Sf > 0.0f ? canon_div(p[idx], Sf) : 0.0f;
    out_v[i] = v;
    out_i[i] = idx;
    sh.fix[i] = canon_fix(v);
  }
  for (int64_t i = k + threadIdx.x; i < width; i += TOPK_NT) {
    out_v[i] = 0.0f;
    out_i[i] = -1;
  }
  if (!nucleus) return;
  __syncthreads();
  // nucleus: keep i iff the exclusive prefix (sorted order) is below top_p
  __shared__ uint64_t s_kept;
  if (threadIdx.x == 0) {
    const double limit = (double)tp * (double)(1ull << SV_FIX_BITS);
    uint64_t pre = 0, kept = 0;
    for (int i = 0; i < k; ++i) {
      bool keep = (double)pre < limit;
      pre += sh.fix[i];
      if (keep) kept += sh.fix[i]; else sh.fix[i] = ~0ull;  // mark dropped
    }
    s_kept = kept;
  }
  __syncthreads();
  const float Kf = canon_unfix(s_kept);
  for (int i = threadIdx.x; i < k; i += TOPK_NT) {
    float v = out_v[i];
    out_v[i] = (sh.fix[i] == ~0ull || !(Kf > 0.0f)) ? 0.0f : canon_div(v, Kf);
  }
}

// ---------------------------------------------------------------------------------------
// Picking an index from non-negative weights: pick = #{k : prefix_incl(k) <= floor(u * R)}
// with prefix sums and R taken in fixed point, clamped to n - 1.
// ---------------------------------------------------------------------------------------

// Weight sources
struct ValuesRow {  // plain probabilities row
  const float* v;
  __device__ float operator()(int64_t k) const { return v[k]; }
};

// Exclusive block scan of u64 run sums for blockDim == NT; returns the exclusive prefix.
template <int N>
__device__ uint64_t block_exclusive_scan_u64(uint64_t v, uint64_t* buf) {
  buf[threadIdx.x] = v;
  __syncthreads();
  for (int off = 1; off < N; off <<= 1) {
    uint64_t a = threadIdx.x >= (unsigned)off ? buf[threadIdx.x - off] : 0;
    __syncthreads();
    buf[threadIdx.x] += a;
    __syncthreads();
  }
  uint64_t incl = buf[threadIdx.x];
  __syncthreads();
  return incl - v;
}

// Count, within chunk c of a weight row of length n, the elements whose inclusive fixed-point
// prefix (starting from `base`) does not exceed `target`.
template <typename W>
__device__ uint32_t count_in_chunk(const W& w, int64_t n, int c, uint64_t base, uint64_t target,
                                   uint64_t* buf, uint64_t* red) {
  const int64_t lo = (int64_t)c * CHUNK + (int64_t)threadIdx.x * RUN;
  // every weight of the run first (clamped indices keep the loads unconditional, so they are
  // all in flight together), then the two passes over registers
  uint64_t f[RUN];
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    const int64_t k = lo + j;
    f[j] = canon_fix(w(k < n ? k : n - 1));
  }
  uint64_t run_sum = 0;
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    if (lo + j >= n) f[j] = 0;
    run_sum += f[j];
  }
  uint64_t pre = base + block_exclusive_scan_u64<NT>(run_sum, buf);
  uint32_t cnt = 0;
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    if (lo + j < n) {
      pre += f[j];
      cnt += pre <= target;
    }
  }
  return (uint32_t)block_sum_u64<NT>(cnt, red);
}

// ---------------------------------------------------------------------------------------
// Wide candidate lists: rows whose top-k exceeds TOPK_MAX (up to the whole vocabulary, with
// or without top-p). The whole row is sorted -- probability descending, ties to the lower id,
// the order of the short lists above -- by a stable least-significant-digit radix sort of
// (~ord_key(p), index) items over the 32 key bits, 8 bits per pass; each pass is a chunk
// histogram, a per-row scan of (digit, chunk) counts and a stable scatter. The lists then get
// the short lists' arithmetic on the sorted order: S = sum of the top k in fixed point,
// v = p / S, the top-p cut at the first exclusive fixed-point prefix >= top_p * 2^44 (found
// chunk by chunk), v / K over the kept prefix and 0 past it. The sorted items live in the
// sampling workspace behind the candidate lists (snowllm_sampling_workspace_bytes reserves
// them when width > TOPK_MAX).
// ---------------------------------------------------------------------------------------
constexpr int MODE_IDENT = 0, MODE_SMALL = 1, MODE_WIDE = 2, MODE_BAD = 3;

__device__ __forceinline__ int list_mode(const int32_t* top_k, const float* top_p, int row,
                                         int64_t V, int64_t width, int64_t* k_out,
                                         bool* nucleus_out) {
  int64_t k = top_k ? (int64_t)top_k[row] : V;
  if (k <= 0 || k > V) k = V;
  const float tp = top_p ? top_p[row] : 1.0f;
  const bool nucleus = tp < 1.0f;
  *k_out = k;
  *nucleus_out = nucleus;
  if (k >= V && !nucleus) return MODE_IDENT;
  if (k > width) return MODE_BAD;
  return k <= TOPK_MAX ? MODE_SMALL : MODE_WIDE;
}

struct WideArgs {
  const float* dense;
  const int32_t* top_k;
  const float* top_p;
  uint64_t* items[2];   // [rows, V] ping-pong
  uint32_t* hist;       // [rows, 256, C]
  uint64_t* part_s;     // [rows, C] fixed-point sums of the top k
  uint64_t* part_v;     // [rows, C] fixed-point sums of v = p / S
  uint64_t* cut;        // [rows, 2] first dropped position, kept sum K
  int64_t V, width;
  int C;
};

__device__ __forceinline__ uint64_t wide_item(float p, int64_t i) {
  return ((uint64_t)(~ord_key(p)) << 32) | (uint64_t)(uint32_t)i;
}

__device__ __forceinline__ bool wide_row(const WideArgs& a, int row, int64_t* k, bool* nuc) {
  return list_mode(a.top_k, a.top_p, row, a.V, a.width, k, nuc) == MODE_WIDE;
}

// Item e of the pass's input: pass 0 reads the probabilities themselves (index order).
__device__ __forceinline__ uint64_t wide_load(const WideArgs& a, int pass, int row, int64_t e) {
  if (pass == 0) return wide_item(a.dense[(int64_t)row * a.V + e], e);
  return a.items[(pass - 1) & 1][(int64_t)row * a.V + e];
}

__global__ void __launch_bounds__(NT) wide_hist(WideArgs a, int pass) {
  __shared__ uint32_t h[256];
  const int c = blockIdx.x, row = blockIdx.y;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc)) return;
  h[threadIdx.x] = 0;
  __syncthreads();
  const int shift = 32 + 8 * pass;
  uint64_t it[RUN];
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    const int64_t e = (int64_t)c * CHUNK + (int64_t)j * NT + threadIdx.x;
    it[j] = wide_load(a, pass, row, e < a.V ? e : a.V - 1);
  }
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    const int64_t e = (int64_t)c * CHUNK + (int64_t)j * NT + threadIdx.x;
    if (e < a.V) atomicAdd(&h[(uint32_t)(it[j] >> shift) & 0xffu], 1u);
  }
  __syncthreads();
  a.hist[((int64_t)row * 256 + threadIdx.x) * a.C + c] = h[threadIdx.x];
}

// Exclusive scan of a row's (digit, chunk) counts, in place: one workgroup per row.
constexpr int WIDE_SCAN_NT = 1024;
__global__ void __launch_bounds__(WIDE_SCAN_NT) wide_scan(WideArgs a) {
  __shared__ uint32_t buf[WIDE_SCAN_NT];
  const int row = blockIdx.x;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc)) return;
  uint32_t* h = a.hist + (int64_t)row * 256 * a.C;
  const int n = 256 * a.C;
  const int per = (n + WIDE_SCAN_NT - 1) / WIDE_SCAN_NT;
  const int lo = threadIdx.x * per;
  uint32_t run = 0;
  for (int i = lo; i < lo + per && i < n; ++i) run += h[i];
  buf[threadIdx.x] = run;
  __syncthreads();
  for (int off = 1; off < WIDE_SCAN_NT; off <<= 1) {
    const uint32_t v = threadIdx.x >= (unsigned)off ? buf[threadIdx.x - off] : 0u;
    __syncthreads();
    buf[threadIdx.x] += v;
    __syncthreads();
  }
  uint32_t pre = buf[threadIdx.x] - run;
  for (int i = lo; i < lo + per && i < n; ++i) {
    const uint32_t v = h[i];
    h[i] = pre;
    pre += v;
  }
}

// Stable scatter: element e = c * CHUNK + j * NT + t goes in round j, lane order within the
// round, so ranks follow e. A wave finds the lanes sharing its digit with eight ballots.
__global__ void __launch_bounds__(NT) wide_scatter(WideArgs a, int pass) {
  __shared__ uint32_t base[256];
  __shared__ uint32_t wcnt[NT / WAVE][256];
  const int c = blockIdx.x, row = blockIdx.y;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc)) return;
  const int t = threadIdx.x, w = t / WAVE, lane = t % WAVE;
  const int shift = 32 + 8 * pass;
  base[t] = a.hist[((int64_t)row * 256 + t) * a.C + c];
#pragma unroll
  for (int ww = 0; ww < NT / WAVE; ++ww) wcnt[ww][t] = 0u;
  uint64_t it[RUN];
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    const int64_t e = (int64_t)c * CHUNK + (int64_t)j * NT + t;
    it[j] = wide_load(a, pass, row, e < a.V ? e : a.V - 1);
  }
  uint64_t* out = a.items[pass & 1] + (int64_t)row * a.V;
  const uint64_t below = (1ull << lane) - 1ull;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RUN; ++j) {
    const int64_t e = (int64_t)c * CHUNK + (int64_t)j * NT + t;
    const bool live = e < a.V;
    const uint32_t d = (uint32_t)(it[j] >> shift) & 0xffu;
    uint64_t same = __ballot(live);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t ones = __ballot((d >> b) & 1u);
      same &= ((d >> b) & 1u) ? ones : ~ones;
    }
    const uint32_t rank = (uint32_t)__popcll(same & below);
    if (live && rank == 0) wcnt[w][d] = (uint32_t)__popcll(same);
    __syncthreads();
    if (live) {
      uint32_t pos = base[d] + rank;
      for (int ww = 0; ww < w; ++ww) pos += wcnt[ww][d];
      out[pos] = it[j];
    }
    __syncthreads();
    uint32_t tot = 0;
#pragma unroll
    for (int ww = 0; ww < NT / WAVE; ++ww) {
      tot += wcnt[ww][t];
      wcnt[ww][t] = 0u;
    }
    base[t] += tot;
    __syncthreads();
  }
}

// p of sorted position i (the probability itself, read back by its index).
__device__ __forceinline__ float wide_p(const WideArgs& a, int row, uint64_t item) {
  return a.dense[(int64_t)row * a.V + (uint32_t)item];
}

__device__ __forceinline__ float wide_sum_f(const uint64_t* part, int C, uint64_t* red) {
  uint64_t s = 0;
  for (int i = threadIdx.x; i < C; i += NT) s += part[i];
  return canon_unfix(block_sum_u64<NT>(s, red));
}

// Fixed-point sums of the top k per chunk of the sorted row.
__global__ void __launch_bounds__(NT) wide_sums(WideArgs a) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc)) return;
  const uint64_t* it = a.items[1] + (int64_t)row * a.V;
  uint64_t s = 0;
  for (int j = 0; j < RUN; ++j) {
    const int64_t i = (int64_t)c * CHUNK + (int64_t)j * NT + threadIdx.x;
    if (i < k) s += canon_fix(wide_p(a, row, it[i]));
  }
  s = block_sum_u64<NT>(s, red);
  if (threadIdx.x == 0) a.part_s[(int64_t)row * a.C + c] = s;
}

// v = p / S over the top k, and its fixed-point sums per chunk (nucleus rows).
__global__ void __launch_bounds__(NT) wide_vsums(WideArgs a) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc) || !nuc) return;
  const float Sf = wide_sum_f(a.part_s + (int64_t)row * a.C, a.C, red);
  const uint64_t* it = a.items[1] + (int64_t)row * a.V;
  uint64_t s = 0;
  for (int j = 0; j < RUN; ++j) {
    const int64_t i = (int64_t)c * CHUNK + (int64_t)j * NT + threadIdx.x;
    if (i < k) s += canon_fix(Sf > 0.0f ? canon_div(wide_p(a, row, it[i]), Sf) : 0.0f);
  }
  s = block_sum_u64<NT>(s, red);
  if (threadIdx.x == 0) a.part_v[(int64_t)row * a.C + c] = s;
}

// The top-p cut: position `cut` of the first element whose exclusive prefix reaches the limit
// (k when none does) and the kept sum K. One workgroup per nucleus row.
__global__ void __launch_bounds__(NT) wide_cut(WideArgs a) {
  __shared__ uint64_t buf[NT];
  __shared__ uint64_t red[NT / WAVE];
  __shared__ int s_chunk;
  __shared__ uint64_t s_base;
  const int row = blockIdx.x;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc) || !nuc) return;
  const double limit = (double)a.top_p[row] * (double)(1ull << SV_FIX_BITS);
  const uint64_t* pv = a.part_v + (int64_t)row * a.C;
  const float Sf = wide_sum_f(a.part_s + (int64_t)row * a.C, a.C, red);
  if (threadIdx.x == 0) {
    uint64_t pre = 0;
    int c = 0;
    for (; c < a.C; ++c) {
      if ((double)(pre + pv[c]) >= limit) break;
      pre += pv[c];
    }
    s_chunk = c;
    s_base = pre;
  }
  __syncthreads();
  const int c = s_chunk;
  uint64_t cut = (uint64_t)k, kept = s_base;
  if (c < a.C) {
    // exclusive prefixes inside chunk c, thread t owning RUN consecutive positions
    const uint64_t* it = a.items[1] + (int64_t)row * a.V;
    const int64_t lo = (int64_t)c * CHUNK + (int64_t)threadIdx.x * RUN;
    uint64_t f[RUN];
    uint64_t run = 0;
#pragma unroll
    for (int j = 0; j < RUN; ++j) {
      const int64_t i = lo + j;
      f[j] = i < k ? canon_fix(Sf > 0.0f ? canon_div(wide_p(a, row, it[i]), Sf) : 0.0f) : 0ull;
      run += f[j];
    }
    uint64_t pre = s_base + block_exclusive_scan_u64<NT>(run, buf);
    uint64_t n_keep = 0, keep_sum = 0;
#pragma unroll
    for (int j = 0; j < RUN; ++j) {
      if (lo + j < k && (double)pre < limit) {
        ++n_keep;
        keep_sum += f[j];
      }
      pre += f[j];
    }
    n_keep = block_sum_u64<NT>(n_keep, red);
    keep_sum = block_sum_u64<NT>(keep_sum, red);
    cut = (uint64_t)c * CHUNK + n_keep;
    kept = s_base + keep_sum;
  } else {
    uint64_t s = 0;
    for (int i = threadIdx.x; i < a.C; i += NT) s += pv[i];
    kept = block_sum_u64<NT>(s, red);
  }
  if (threadIdx.x == 0) {
    a.cut[(int64_t)row * 2 + 0] = cut;
    a.cut[(int64_t)row * 2 + 1] = kept;
  }
}

// The lists: sorted ids, v = p / S (then v / K inside the top-p prefix, 0 past it); slots
// past k are (0, -1).
__global__ void __launch_bounds__(NT) wide_write(WideArgs a, float* __restrict__ values,
                                                 int64_t* __restrict__ ids) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  int64_t k;
  bool nuc;
  if (!wide_row(a, row, &k, &nuc)) return;
  const float Sf = wide_sum_f(a.part_s + (int64_t)row * a.C, a.C, red);
  const int64_t cut = nuc ? (int64_t)a.cut[(int64_t)row * 2 + 0] : k;
  const float Kf = nuc ? canon_unfix(a.cut[(int64_t)row * 2 + 1]) : 1.0f;
  const uint64_t* it = a.items[1] + (int64_t)row * a.V;
  float* ov = values + (int64_t)row * a.width;
  int64_t* oi = ids + (int64_t)row * a.width;
  for (int j = 0; j < RUN; ++j) {
    const int64_t i = (int64_t)c * CHUNK + (int64_t)j * NT + threadIdx.x;
    if (i >= a.width) break;
    if (i < k) {
      const uint64_t item = it[i];
      float v = Sf > 0.0f ? canon_div(wide_p(a, row, item), Sf) : 0.0f;
      if (nuc) v = (i >= cut || !(Kf > 0.0f)) ? 0.0f : canon_div(v, Kf);
      ov[i] = v;
      oi[i] = (int64_t)(uint32_t)item;
    } else {
      ov[i] = 0.0f;
      oi[i] = -1;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Rejection sampling (DFlash verify).
// ---------------------------------------------------------------------------------------
struct RejectArgs {
  const float* p;
  const int64_t* ids;
  const int64_t* drafts;
  const int64_t* cand;
  const float* q;
  const int32_t* slots;
  const int32_t* valid;
  const float* uniform;
  int64_t* out;
  int64_t* accepted;
  int64_t b, width, p_width, q_width;
};

// Probability assigned to `token` by a candidate row (sum over matching ids; ids are unique
// in lists produced by topk_topp and the selector, so the direct slot is tried first).
__device__ float row_prob_block(const float* probs, const int64_t* ids, int64_t n,
                                int64_t token, float* red_f) {
  __shared__ int s_direct;
  if (threadIdx.x == 0) s_direct = (token >= 0 && token < n && ids[token] == token);
  __syncthreads();
  if (s_direct) {
    float r = probs[token];
    __syncthreads();
    return r;
  }
  // general case: block-parallel search, matches summed in index order
  __shared__ int s_count;
  __shared__ int64_t s_first;
  if (threadIdx.x == 0) { s_count = 0; s_first = -1; }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    if (ids[i] == token) {
      atomicAdd(&s_count, 1);
      s_first = i;  // unique case: the only writer
    }
  }
  __syncthreads();
  float r = 0.0f;
  if (s_count == 1) {
    r = probs[s_first];
  } else if (s_count > 1) {
    if (threadIdx.x == 0) {
      float acc = 0.0f;
      for (int64_t i = 0; i < n; ++i)
        if (ids[i] == token) acc = __fadd_rn(acc, probs[i]);
      red_f[0] = acc;
    }
    __syncthreads();
    r = red_f[0];
  }
  __syncthreads();
  return r;
}

// Per-thread lookup used inside the residual (q rows are short, or the identity layout).
__device__ __forceinline__ float row_prob_thread(const float* probs, const int64_t* ids, int64_t n,
                                                 int64_t token) {
  if (token >= 0 && token < n && ids[token] == token) return probs[token];
  float acc = 0.0f;
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] == token) acc = __fadd_rn(acc, probs[i]);
  return acc;
}

__global__ void __launch_bounds__(NT) reject_scan(RejectArgs a) {
  __shared__ float red_f[4];
  const int r = blockIdx.x;
  const int64_t length = a.width - 1;
  const int slot = a.slots[r];
  const bool valid = a.valid[r] != 0;
  int64_t first = length;
  for (int64_t j = 0; j < length; ++j) {
    const int64_t token = a.drafts[r * length + j];
    const int64_t prow = r * a.width + j;
    float pt = row_prob_block(a.p + prow * a.p_width, a.ids + prow * a.p_width, a.p_width, token,
                              red_f);
    float qt = 1.0f;
    if (valid) {
      const int64_t qrow = ((int64_t)slot * length + j) * a.q_width;
      qt = row_prob_block(a.q + qrow, a.cand + qrow, a.q_width, token, red_f);
    }
    if (__fmul_rn(a.uniform[r * a.width + j], qt) >= pt) {
      first = j;
      break;
    }
  }
  if (threadIdx.x == 0) g_first[r] = (int32_t)first;
  for (int64_t j = threadIdx.x; j < a.width; j += NT)
    a.out[r * a.width + j] = j < first ? a.drafts[r * length + j] : -1;
}

struct ResidualRow {
  const float* p;       // p row at position `first`
  const int64_t* ids;   // ids row at position `first`
  const float* q;       // q row (or null when the proposal is not valid)
  const int64_t* cand;
  int64_t q_width;
  int64_t draft;        // draft token at `first` (used when q is null)
  bool subtract;        // false for the bonus position
  const uint32_t* bits = nullptr;  // staged rows: bit (id mod 2^16) set for every candidate id
  __device__ float operator()(int64_t k) const {
    return from_loaded(k, p[k], subtract ? ids[k] : 0);
  }
  // The same residual from p[k] and ids[k] already loaded (id unused for the bonus position).
  __device__ float from_loaded(int64_t k, float pk, int64_t id) const {
    if (!subtract) return pk;
    float qk;
    if (bits) {
      // q(id) = 0 unless id may be a candidate; candidates are then searched exactly
      const uint32_t h = (uint32_t)id & 0xffffu;
      qk = ((bits[h >> 5] >> (h & 31)) & 1u) ? row_prob_thread(q, cand, q_width, id) : 0.0f;
    } else if (q) {
      // identity layouts (ids[k] == k, cand[k] == k) resolve with loads independent of id
      const bool in_q = k < q_width;
      const float qd = in_q ? q[k] : 0.0f;
      const int64_t cd = in_q ? cand[k] : -1;
      qk = (id == k && cd == k) ? qd : row_prob_thread(q, cand, q_width, id);
    } else {
      qk = (id == draft) ? 1.0f : 0.0f;
    }
    float d = __fsub_rn(pk, qk);
    return d > 0.0f ? d : 0.0f;
  }
};

__device__ ResidualRow residual_row(const RejectArgs& a, int r, int64_t first) {
  const int64_t length = a.width - 1;
  const int64_t prow = r * a.width + first;
  ResidualRow w;
  w.p = a.p + prow * a.p_width;
  w.ids = a.ids + prow * a.p_width;
  w.subtract = first < length;
  const bool valid = a.valid[r] != 0;
  const int slot = a.slots[r];
  if (w.subtract && valid) {
    const int64_t qrow = ((int64_t)slot * length + first) * a.q_width;
    w.q = a.q + qrow;
    w.cand = a.cand + qrow;
  } else {
    w.q = nullptr;
    w.cand = nullptr;
  }
  w.q_width = a.q_width;
  w.draft = w.subtract ? a.drafts[r * length + first] : -1;
  return w;
}

// Short candidate rows (the selector's 16) are staged in LDS, so the per-element lookup of the
// residual reads LDS instead of global memory. All threads call it.
// They also get a 2^16-bit membership filter of their ids (id mod 2^16), so an element whose
// id is not a candidate skips the search: q(id) = 0 and the residual is p.
constexpr int Q_STAGE = 64;
constexpr int Q_BITS_WORDS = 65536 / 32;
__device__ __forceinline__ void stage_q(ResidualRow& w, int64_t* s_cand, float* s_q,
                                        uint32_t* s_bits) {
  const bool stage = w.subtract && w.q && w.q_width <= Q_STAGE;
  if (stage) {
    for (int i = threadIdx.x; i < Q_BITS_WORDS; i += blockDim.x) s_bits[i] = 0u;
    for (int i = threadIdx.x; i < w.q_width; i += blockDim.x) {
      s_cand[i] = w.cand[i];
      s_q[i] = w.q[i];
    }
  }
  __syncthreads();
  if (stage) {
    for (int i = threadIdx.x; i < w.q_width; i += blockDim.x) {
      const uint32_t h = (uint32_t)s_cand[i] & 0xffffu;
      atomicOr(&s_bits[h >> 5], 1u << (h & 31));
    }
  }
  __syncthreads();
  if (stage) {
    w.cand = s_cand;
    w.q = s_q;
    w.bits = s_bits;
  }
}

__global__ void __launch_bounds__(NT) reject_chunks(RejectArgs a, int C) {
  __shared__ uint64_t red[NT / WAVE];
  __shared__ int64_t s_cand[Q_STAGE];
  __shared__ float s_q[Q_STAGE];
  __shared__ uint32_t s_bits[Q_BITS_WORDS];
  const int c = blockIdx.x, r = blockIdx.y;
  const int64_t first = g_first[r];
  ResidualRow w = residual_row(a, r, first);
  stage_q(w, s_cand, s_q, s_bits);
  uint64_t rs = 0, ps = 0;
  // every p and id load of the thread in flight before the first residual
  float pv[RUN];
  int64_t idv[RUN];
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    const int64_t i = (int64_t)c * CHUNK + threadIdx.x + (int64_t)k * NT;
    const int64_t ii = i < a.p_width ? i : a.p_width - 1;  // loads stay unconditional
    pv[k] = w.p[ii];
    idv[k] = w.subtract ? w.ids[ii] : 0;
  }
#pragma unroll
  for (int k = 0; k < RUN; ++k) {
    const int64_t i = (int64_t)c * CHUNK + threadIdx.x + (int64_t)k * NT;
    const int64_t ii = i < a.p_width ? i : a.p_width - 1;
    const uint64_t r1 = canon_fix(w.from_loaded(ii, pv[k], idv[k])), p1 = canon_fix(pv[k]);
    if (i < a.p_width) {
      rs += r1;
      ps += p1;
    }
  }
  rs = block_sum_u64<NT>(rs, red);
  ps = block_sum_u64<NT>(ps, red);
  if (threadIdx.x == 0) {
    g_chunk_sums[(r * CHUNKS_MAX + c) * 2 + 0] = rs;
    g_chunk_sums[(r * CHUNKS_MAX + c) * 2 + 1] = ps;
  }
}

__global__ void __launch_bounds__(NT) reject_pick(RejectArgs a, int C) {
  __shared__ uint64_t buf[NT];
  __shared__ uint64_t red[NT / WAVE];
  __shared__ int s_chunk;
  __shared__ uint64_t s_base, s_target;
  __shared__ int s_use_p;
  __shared__ uint64_t s_sums[CHUNKS_MAX][2];
  __shared__ int64_t s_cand[Q_STAGE];
  __shared__ float s_q[Q_STAGE];
  __shared__ uint32_t s_bits[Q_BITS_WORDS];
  const int r = blockIdx.x;
  const int64_t first = g_first[r];
  for (int i = threadIdx.x; i < 2 * C; i += NT)
    s_sums[i >> 1][i & 1] = g_chunk_sums[(r * CHUNKS_MAX + (i >> 1)) * 2 + (i & 1)];
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t R = 0;
    for (int c = 0; c < C; ++c) R += s_sums[c][0];
    int use_p = 0;
    if (R == 0) {
      use_p = 1;
      for (int c = 0; c < C; ++c) R += s_sums[c][1];
    }
    const uint64_t target = canon_scale_floor(a.uniform[r * a.width + a.width - 1], R);
    uint64_t pre = 0;
    int c = 0;
    for (; c < C; ++c) {
      uint64_t s = s_sums[c][use_p];
      if (pre + s > target) break;
      pre += s;
    }
    s_chunk = c;
    s_base = pre;
    s_target = target;
    s_use_p = use_p;
  }
  __syncthreads();
  int64_t pick;
  if (s_chunk >= C) {
    pick = a.p_width - 1;
  } else {
    ResidualRow w = residual_row(a, r, first);
    if (s_use_p) w.subtract = false;
    stage_q(w, s_cand, s_q, s_bits);
    uint32_t cnt = count_in_chunk(w, a.p_width, s_chunk, s_base, s_target, buf, red);
    pick = (int64_t)s_chunk * CHUNK + cnt;
    if (pick > a.p_width - 1) pick = a.p_width - 1;
  }
  if (threadIdx.x == 0) {
    const int64_t prow = r * a.width + first;
    a.out[r * a.width + first] = a.ids[prow * a.p_width + pick];
    a.accepted[r] = first + 1;
  }
}

// ---------------------------------------------------------------------------------------
// Sampling from candidate lists: pick = #(u >= cumsum(values)), clamped to the last slot.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(NT) sample_chunks(const float* __restrict__ values,
                                                    int64_t width, uint64_t* __restrict__ sums,
                                                    int C) {
  __shared__ uint64_t red[NT / WAVE];
  const int c = blockIdx.x, row = blockIdx.y;
  const float* v = values + (int64_t)row * width;
  uint64_t s = 0;
  for (int k = 0; k < RUN; ++k) {
    int64_t i = (int64_t)c * CHUNK + threadIdx.x + (int64_t)k * NT;
    if (i < width) s += canon_fix(v[i]);
  }
  s = block_sum_u64<NT>(s, red);
  if (threadIdx.x == 0) sums[row * C + c] = s;
}

__global__ void __launch_bounds__(NT) sample_pick(const float* __restrict__ values,
                                                  const int64_t* __restrict__ ids, int64_t width,
                                                  const uint64_t* __restrict__ sums,
                                                  const float* __restrict__ uniform,
                                                  int64_t* __restrict__ out, int C) {
  __shared__ uint64_t buf[NT];
  __shared__ uint64_t red[NT / WAVE];
  __shared__ int s_chunk;
  __shared__ uint64_t s_base, s_target;
  const int row = blockIdx.x;
  if (threadIdx.x == 0) {
    // u >= prefix  <=>  floor(u * 2^44) >= prefix for integer prefixes
    const float u = uniform[row];
    const uint64_t target = u > 0.0f ? (uint64_t)__builtin_floorf(__builtin_ldexpf(u, SV_FIX_BITS)) : 0;
    uint64_t pre = 0;
    int c = 0;
    for (; c < C; ++c) {
      uint64_t s = sums[row * C + c];
      if (pre + s > target) break;
      pre += s;
    }
    s_chunk = c;
    s_base = pre;
    s_target = target;
  }
  __syncthreads();
  int64_t pick;
  if (s_chunk >= C) {
    pick = width - 1;
  } else {
    ValuesRow w{values + (int64_t)row * width};
    uint32_t cnt = count_in_chunk(w, width, s_chunk, s_base, s_target, buf, red);
    pick = (int64_t)s_chunk * CHUNK + cnt;
    if (pick > width - 1) pick = width - 1;
  }
  if (threadIdx.x == 0) {
    // never land on an unused (-1) slot: step back to the last real candidate
    int64_t id = ids[(int64_t)row * width + pick];
    while (id < 0 && pick > 0) id = ids[(int64_t)row * width + (--pick)];
    out[row] = id;
  }
}

// ---------------------------------------------------------------------------------------
// Repetition / frequency / presence penalties on one logit row, for the listed token ids
// (the prompt's and output's ids of a request, each once) with their output counts: the
// repetition penalty divides a positive logit and multiplies a non-positive one, then the
// frequency penalty times the count and the presence penalty (count > 0) are subtracted, one
// binary32 operation each (the published convention of OpenAI-style sampling parameters).
// ---------------------------------------------------------------------------------------
__global__ void penalties_kernel(float* __restrict__ logits, const int64_t* __restrict__ ids,
                                 const int32_t* __restrict__ counts, int n, int vocab,
                                 float presence, float frequency, float repetition) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t t = ids[i];
  if (t < 0 || t >= vocab) return;
  const int c = counts[i];
  float x = logits[t];
  // plain operators: this file's contract(off) keeps the product and the difference apart
  // (the __f*_rn helpers are header code that the compiler may fuse into an fma)
  if (repetition != 1.0f) x = x > 0.0f ? x / repetition : x * repetition;
  x = x - frequency * (float)c;
  x = x - (c > 0 ? presence : 0.0f);
  logits[t] = x;
}

inline hipStream_t S(void* s) { return (hipStream_t)s; }

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

SV_API int64_t snowllm_sampling_max_k(void) { return VOCAB_MAX; }

SV_API int snowllm_sampling_argmax(const float* logits, int64_t* out, int64_t B, int64_t V,
                                   void* stream) {
  if (B < 0 || V <= 0 || V > VOCAB_MAX) return B == 0 ? SV_OK : SV_EINVAL;
  if (B == 0) return SV_OK;
  const int C = chunks_of(V);
  for (int64_t r0 = 0; r0 < B; r0 += ROWS_MAX) {
    const int rows = (int)((B - r0) < ROWS_MAX ? (B - r0) : ROWS_MAX);
    hipLaunchKernelGGL(argmax_chunks, dim3(C, rows), dim3(NT), 0, S(stream), logits + r0 * V, V,
                       C);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(argmax_final, dim3(rows), dim3(WAVE), 0, S(stream), out + r0, C);
    SV_CHECK_LAUNCH();
  }
  return SV_OK;
}

SV_API int snowllm_spec_accept(const int64_t* tokens, const int64_t* drafts, int64_t* acc,
                               int64_t b, int64_t t, int64_t tokens_stride,
                               int64_t drafts_stride, void* stream) {
  if (b < 0 || t < 1) return SV_EINVAL;
  if (b == 0) return SV_OK;
  const int nt = 64;
  hipLaunchKernelGGL(spec_accept_kernel, dim3((unsigned)((b + nt - 1) / nt)), dim3(nt), 0,
                     S(stream), tokens, drafts, acc, b, t, tokens_stride, drafts_stride);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Workspace: dense probabilities [batch, vocab] f32, then the softmax row statistics, then
// the candidate lists used by snowllm_sampling_sample (values f32 and ids i64 [batch, width])
// and their chunk sums.
// Penalties on one logit row (snowllm/_capi.py:589; wrapper snowllm/ops/sampling.py:94-100).
SV_API int snowllm_sampling_penalties(float* logits, const int64_t* ids, const int32_t* counts,
                                      int n, int vocab, float presence, float frequency,
                                      float repetition, void* stream) {
  if (n < 0 || vocab <= 0 || !(repetition > 0.0f)) return SV_EINVAL;
  if (n == 0) return SV_OK;
  if (!logits || !ids || !counts) return SV_EINVAL;
  hipLaunchKernelGGL(penalties_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     S(stream), logits, ids, counts, n, vocab, presence, frequency, repetition);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Lists wider than TOPK_MAX add the wide-list sort: two [batch, vocab] u64 item buffers, the
// per-pass chunk histograms and the per-row sums.
namespace {
size_t lists_bytes(int64_t batch, int64_t vocab, int64_t width) {
  const int64_t C = chunks_of(vocab);
  const int64_t Cw = chunks_of(width > 0 ? width : 1);
  size_t bytes = align256((size_t)batch * vocab * 4);
  bytes += align256((size_t)batch * C * 4);
  bytes += align256((size_t)batch * C * 8);
  bytes += align256((size_t)batch * width * 4);
  bytes += align256((size_t)batch * width * 8);
  bytes += align256((size_t)batch * Cw * 8);
  return bytes;
}

WideArgs wide_view(const float* dense, int64_t rows, int64_t vocab, int64_t width,
                   const int32_t* top_k, const float* top_p) {
  const int64_t C = chunks_of(vocab);
  char* p = (char*)dense + lists_bytes(rows, vocab, width);
  WideArgs a;
  a.dense = dense;
  a.top_k = top_k;
  a.top_p = top_p;
  a.items[0] = (uint64_t*)p;
  p += align256((size_t)rows * vocab * 8);
  a.items[1] = (uint64_t*)p;
  p += align256((size_t)rows * vocab * 8);
  a.hist = (uint32_t*)p;
  p += align256((size_t)rows * 256 * C * 4);
  a.part_s = (uint64_t*)p;
  p += align256((size_t)rows * C * 8);
  a.part_v = (uint64_t*)p;
  p += align256((size_t)rows * C * 8);
  a.cut = (uint64_t*)p;
  a.V = vocab;
  a.width = width;
  a.C = (int)C;
  return a;
}
}  // namespace

SV_API int64_t snowllm_sampling_workspace_bytes(int64_t batch, int64_t vocab, int64_t width) {
  if (batch < 0 || vocab <= 0) return 0;
  size_t bytes = lists_bytes(batch, vocab, width);
  if (width > TOPK_MAX) {
    const int64_t C = chunks_of(vocab);
    bytes += 2 * align256((size_t)batch * vocab * 8) + align256((size_t)batch * 256 * C * 4) +
             2 * align256((size_t)batch * C * 8) + align256((size_t)batch * 16);
  }
  return (int64_t)bytes;
}

namespace {
SoftmaxTail softmax_tail(void* dense, int64_t rows, int64_t vocab) {
  const int64_t C = chunks_of(vocab);
  char* base = (char*)dense + align256((size_t)rows * vocab * 4);
  SoftmaxTail t;
  t.max_keys = (uint32_t*)base;
  t.sums = (uint64_t*)(base + align256((size_t)rows * C * 4));
  return t;
}

int launch_softmax(const float* logits, float* dense, int64_t rows, int64_t vocab,
                   const float* temperature, hipStream_t s) {
  const int C = chunks_of(vocab);
  SoftmaxTail tail = softmax_tail(dense, rows, vocab);
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const int n = (int)((rows - r0) < 65535 ? (rows - r0) : 65535);
    SoftmaxTail t = tail;
    t.max_keys += r0 * C;
    t.sums += r0 * C;
    const float* tr = temperature ? temperature + r0 : nullptr;
    hipLaunchKernelGGL(softmax_max, dim3(C, n), dim3(NT), 0, s, logits + r0 * vocab, vocab, tr,
                       t, C);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(softmax_exp, dim3(C, n), dim3(NT), 0, s, logits + r0 * vocab, vocab, tr,
                       dense + r0 * vocab, t, C);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(softmax_norm, dim3(C, n), dim3(NT), 0, s, dense + r0 * vocab, vocab, t, C);
    SV_CHECK_LAUNCH();
  }
  return SV_OK;
}

int launch_topk_topp(const float* dense, float* values, int64_t* ids, int64_t rows,
                     int64_t vocab, int64_t width, const int32_t* top_k, const float* top_p,
                     hipStream_t s) {
  hipLaunchKernelGGL(topk_topp_rows, dim3((unsigned)rows, (unsigned)chunks_of(width)),
                     dim3(TOPK_NT), 0, s, dense, values, ids, vocab, width, top_k, top_p);
  SV_CHECK_LAUNCH();
  if (width <= TOPK_MAX) return SV_OK;  // no row can need a wide list
  if (rows > 65535) return SV_ENOTSUP;    // rows are the grids' y dimension
  // rows wider than TOPK_MAX: sort, sums, top-p cut, lists (the other rows return at once)
  const WideArgs a = wide_view(dense, rows, vocab, width, top_k, top_p);
  const dim3 grid((unsigned)a.C, (unsigned)rows);
  for (int pass = 0; pass < 4; ++pass) {
    hipLaunchKernelGGL(wide_hist, grid, dim3(NT), 0, s, a, pass);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(wide_scan, dim3((unsigned)rows), dim3(WIDE_SCAN_NT), 0, s, a);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(wide_scatter, grid, dim3(NT), 0, s, a, pass);
    SV_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(wide_sums, grid, dim3(NT), 0, s, a);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(wide_vsums, grid, dim3(NT), 0, s, a);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(wide_cut, dim3((unsigned)rows), dim3(NT), 0, s, a);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(wide_write, dim3((unsigned)chunks_of(width), (unsigned)rows), dim3(NT), 0,
                     s, a, values, ids);
  SV_CHECK_LAUNCH();
  return SV_OK;
}
}  // namespace

SV_API int snowllm_sampling_softmax(const float* logits, float* dense, int64_t rows,
                                    int64_t vocab, const float* temperature, void* stream) {
  if (rows < 0 || vocab <= 0 || vocab > VOCAB_MAX) return SV_EINVAL;
  if (rows == 0) return SV_OK;
  return launch_softmax(logits, dense, rows, vocab, temperature, S(stream));
}

// Every top-k up to the vocabulary, with or without top-p. `dense` must be the start of a
// workspace of snowllm_sampling_workspace_bytes(rows, vocab, width) bytes (the wide lists
// sort behind the dense block). A row whose top-k exceeds `width` cannot be written and
// comes out as (NaN, -2); callers size the width as the largest top-k of the batch.
SV_API int snowllm_sampling_topk_topp(const float* dense, float* values, int64_t* ids,
                                      int64_t rows, int64_t vocab, int64_t width,
                                      const int32_t* top_k, const float* top_p, void* stream) {
  if (rows < 0 || vocab <= 0 || vocab > VOCAB_MAX || width <= 0) return SV_EINVAL;
  if (rows == 0) return SV_OK;
  return launch_topk_topp(dense, values, ids, rows, vocab, width, top_k, top_p, S(stream));
}

SV_API int snowllm_sampling_sample(const float* logits, const int32_t* top_k, const float* top_p,
                                   const float* temperature, const float* uniform, int64_t* out,
                                   void* ws, int64_t ws_bytes, int64_t B, int64_t V,
                                   int64_t width, void* stream) {
  if (B < 0 || V <= 0 || V > VOCAB_MAX || width <= 0) return SV_EINVAL;
  if (B == 0) return SV_OK;
  if (ws_bytes < snowllm_sampling_workspace_bytes(B, V, width)) return SV_EINVAL;
  const int64_t C = chunks_of(V);
  const int Cw = chunks_of(width);
  float* dense = (float*)ws;
  char* p = (char*)ws + align256((size_t)B * V * 4) + align256((size_t)B * C * 4) +
            align256((size_t)B * C * 8);
  float* values = (float*)p;
  p += align256((size_t)B * width * 4);
  int64_t* ids = (int64_t*)p;
  p += align256((size_t)B * width * 8);
  uint64_t* sums = (uint64_t*)p;
  hipStream_t s = S(stream);
  int rc = launch_softmax(logits, dense, B, V, temperature, s);
  if (rc) return rc;
  rc = launch_topk_topp(dense, values, ids, B, V, width, top_k, top_p, s);
  if (rc) return rc;
  for (int64_t r0 = 0; r0 < B; r0 += 65535) {
    const int n = (int)((B - r0) < 65535 ? (B - r0) : 65535);
    hipLaunchKernelGGL(sample_chunks, dim3(Cw, n), dim3(NT), 0, s, values + r0 * width, width,
                       sums + r0 * Cw, Cw);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(sample_pick, dim3(n), dim3(NT), 0, s, values + r0 * width,
                       ids + r0 * width, width, sums + r0 * Cw, uniform + r0, out + r0, Cw);
    SV_CHECK_LAUNCH();
  }
  return SV_OK;
}

SV_API int snowllm_draft_reject(const float* p, const int64_t* ids, const int64_t* drafts,
                                const int64_t* cand, const float* q, const int32_t* slots,
                                const int32_t* valid, const float* uniform, int64_t* out,
                                int64_t* accepted, int64_t b, int64_t width, int64_t p_width,
                                int64_t q_width, void* stream) {
  if (b < 0 || width < 1 || p_width <= 0 || p_width > VOCAB_MAX || q_width < 0)
    return SV_EINVAL;
  if (b == 0) return SV_OK;
  const int C = chunks_of(p_width);
  hipStream_t s = S(stream);
  for (int64_t r0 = 0; r0 < b; r0 += ROWS_MAX) {
    const int n = (int)((b - r0) < ROWS_MAX ? (b - r0) : ROWS_MAX);
    RejectArgs a;
    a.p = p + r0 * width * p_width;
    a.ids = ids + r0 * width * p_width;
    a.drafts = drafts + r0 * (width - 1);
    a.cand = cand;
    a.q = q;
    a.slots = slots + r0;
    a.valid = valid + r0;
    a.uniform = uniform + r0 * width;
    a.out = out + r0 * width;
    a.accepted = accepted + r0;
    a.b = n;
    a.width = width;
    a.p_width = p_width;
    a.q_width = q_width;
    hipLaunchKernelGGL(reject_scan, dim3(n), dim3(NT), 0, s, a);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(reject_chunks, dim3(C, n), dim3(NT), 0, s, a, C);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(reject_pick, dim3(n), dim3(NT), 0, s, a, C);
    SV_CHECK_LAUNCH();
  }
  return SV_OK;
}

// =======================================================================================
// Acceptance straight from the target logits, for requests whose candidate lists are the
// whole vocabulary in vocabulary order (top-k at least the vocabulary, top-p 1): the
// arithmetic of snowllm_sampling_softmax + snowllm_sampling_topk_topp + snowllm_draft_reject
// on those rows -- the same bits -- without the dense [rows, V] probabilities, in three
// launches; and the greedy form (argmax of every row + prefix acceptance) in one.
//
// Workgroup (row, w) takes slice w (FA_SLICE logits, FA_E per thread, coalesced) of a row.
//   1. slice maxima of x / T;
//   2. numerators e = exp(x / T - M) with the row maximum M, the slice's fixed-point sum and
//      the draft token's numerator, and in one more workgroup per draft row the proposal's
//      q(d_j); the request's last workgroup to finish (a counter) forms every row's Z and
//      the accepted prefix, one thread per draft row;
//   3. one workgroup per 4 * FA_NT-logit sub-chunk of the row where the prefix stops forms
//      the residual max(p - q, 0) (p at the bonus row) and its fixed-point sums; the
//      request's last one finds the sub-chunk holding floor(u R) (a wave's prefix scan over
//      the sub-chunk sums), counts its prefix there and writes the outputs.
// Nothing waits for another workgroup. A counter advances by exactly FA_QUANTUM per launch
// (each participant adds 1, one adds the quantum's rest), so the last arriver is the one
// whose add completes the quantum; nothing is ever reset. Statistics are written with
// device-scope stores, each thread waits for its stores (vmcnt(0)) before its workgroup's
// add, and the last arriver reads them with device-scope loads after its add returned.
// =======================================================================================
namespace {

constexpr int FA_NT = 512;                      // threads per workgroup
constexpr int FA_E = 16;                        // logits per thread
constexpr int FA_SLICE = FA_NT * FA_E;          // logits per workgroup
constexpr int FA_P_MAX = (int)(VOCAB_MAX / FA_SLICE);  // slices per row
constexpr int FA_SUB = 4 * FA_NT;               // logits per sub-chunk of a slice
constexpr int FA_SUBCHUNKS = FA_E / 4;          // sub-chunks per slice
constexpr int FA_ROWS = 256;                    // rows (b * width) per launch
constexpr uint64_t FA_QUANTUM = 1ull << 20;
static_assert(FA_SLICE * FA_P_MAX == VOCAB_MAX, "slices cover the vocabulary limit");

__device__ uint32_t g_fa_maxkey[FA_ROWS][FA_P_MAX];
__device__ uint64_t g_fa_sum[FA_ROWS][FA_P_MAX];
__device__ uint32_t g_fa_edraft[FA_ROWS];       // a draft token's numerator (f32 bits)
__device__ uint32_t g_fa_qt[FA_ROWS];           // q(d_j) of a draft row (f32 bits)
__device__ int32_t g_fa_first[FA_ROWS];         // per request: where the prefix stops
__device__ uint64_t g_fa_rsub[FA_ROWS][FA_P_MAX][FA_SUBCHUNKS];
__device__ uint64_t g_fa_psub[FA_ROWS][FA_P_MAX][FA_SUBCHUNKS];
__device__ uint64_t g_fa_amax[FA_ROWS][FA_P_MAX];
__device__ uint64_t g_fa_cnt[3][FA_ROWS];       // per request: stage 2, stage 3, greedy
// the first level of two-level arrivals: per row (stage 2, greedy) or per slice (stage 3), a
// counter per 128-byte line, so that the many workgroups of a launch finishing together do not
// all queue on one address
constexpr int FA_LINE = 16;  // uint64 per 128-byte line
__device__ __attribute__((aligned(128))) uint64_t g_fa_cnt1[3][FA_ROWS * FA_P_MAX][FA_LINE];

template <class T>
__device__ __forceinline__ void dev_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T dev_load(T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This workgroup's arrival at a request's counter of n participants (lead: the one that
// adds the rest of the quantum). True in every thread of the workgroup that arrived last.
// Device-scope atomics on one address complete one after another, so a launch's many
// workgroups count in two levels (fa_last_arrival2).
__device__ bool fa_last_arrival(uint64_t* cnt, int n, bool lead) {
  __shared__ uint32_t s_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint64_t inc = lead ? FA_QUANTUM - (uint64_t)n + 1 : 1;
    const uint64_t old =
        __hip_atomic_fetch_add(cnt, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = ((old + inc) & (FA_QUANTUM - 1)) == 0;
  }
  __syncthreads();
  return s_last != 0;
}

// Two levels: the last of n1 workgroups at cnt1 goes on to cnt2 as one of its n2
// participants; true in the workgroup that arrives last there. lead1 / lead2 add the quanta's
// rests. Every participant's stores completed before its first-level add, and each level's
// last arrival saw the count of everything before it, so the final workgroup's device-scope
// loads, issued after its second add returned, see every participant's stores.
__device__ bool fa_last_arrival2(uint64_t* cnt1, int n1, bool lead1, uint64_t* cnt2, int n2,
                                 bool lead2) {
  if (!fa_last_arrival(cnt1, n1, lead1)) return false;
  return fa_last_arrival(cnt2, n2, lead2);
}

struct FaArgs {
  const float* logits;       // [b * width, V]
  const float* temperature;  // [b * width] or null
  const int64_t* drafts;     // [b, width - 1]
  const int64_t* cand;       // [S, width - 1, q_width]
  const float* q;
  const int32_t* slots;
  const int32_t* valid;
  const float* uniform;      // [b, width]
  int64_t* out;              // [b, width]
  int64_t* accepted;         // [b]
  int V, width, P;
  int64_t q_width;
};

// x[i] / T of this thread's FA_E logits of slice w (loads at clamped indices, all in flight)
__device__ __forceinline__ void fa_load_slice(const float* x, int lo, int V, float T,
                                              float (&v)[FA_E]) {
#pragma unroll
  for (int k = 0; k < FA_E; ++k) {
    const int i = lo + k * FA_NT + (int)threadIdx.x;
    v[k] = x[i < V ? i : V - 1];
  }
#pragma unroll
  for (int k = 0; k < FA_E; ++k) v[k] = __fdiv_rn(v[k], T);
}

// Statistics are read one per lane (a device-scope load is a round trip to memory; one
// thread reading them in turn would pay it per value), then reduced in wave 0.
__device__ __forceinline__ float fa_row_max(int row, int P) {
  __shared__ uint32_t s_m;
  if (threadIdx.x < WAVE) {
    uint32_t m = 0;
    for (int i = threadIdx.x; i < P; i += WAVE) {
      const uint32_t k = dev_load(&g_fa_maxkey[row][i]);
      m = k > m ? k : m;
    }
    m = wave_max(m);
    if (threadIdx.x == 0) s_m = m;
  }
  __syncthreads();
  return ord_key_to_float(s_m);
}

// Z of a row (wave 0; the result in lane 0 is broadcast through s_z by the caller).
__device__ __forceinline__ uint64_t fa_row_zsum(int row, int P) {
  uint64_t z = 0;
  for (int i = threadIdx.x; i < P; i += WAVE) z += dev_load(&g_fa_sum[row][i]);
  return wave_sum_u64(z);
}

__global__ void __launch_bounds__(FA_NT) fa_max_kernel(const float* __restrict__ h_logits, const float* __restrict__ h_temperature, int h_V, int h_width, int h_P, FaArgs a) {
  a.logits = h_logits, a.temperature = h_temperature, a.V = h_V, a.width = h_width, a.P = h_P;
  __shared__ uint64_t red[FA_NT / WAVE];
  const int w = blockIdx.x, row = blockIdx.y;  // grid (P, rows)
  const int lo = w * FA_SLICE;
  float v[FA_E];
  fa_load_slice(a.logits + (int64_t)row * a.V, lo, a.V, row_temperature(a.temperature, row), v);
  uint32_t mk = 0;
#pragma unroll
  for (int k = 0; k < FA_E; ++k) {
    const uint32_t key = ord_key(v[k]);
    if (lo + k * FA_NT + (int)threadIdx.x < a.V) mk = key > mk ? key : mk;
  }
  mk = (uint32_t)block_max_u64<FA_NT>(mk, red);
  if (threadIdx.x == 0) dev_store(&g_fa_maxkey[row][w], mk);
}

__global__ void __launch_bounds__(FA_NT) fa_sum_kernel(const float* __restrict__ h_logits, const float* __restrict__ h_temperature, int h_V, int h_width, int h_P, FaArgs a) {
  a.logits = h_logits, a.temperature = h_temperature, a.V = h_V, a.width = h_width, a.P = h_P;
  __shared__ uint64_t red[FA_NT / WAVE];
  __shared__ float red_f[4];
  const int P = a.P, width = a.width, length = width - 1, V = a.V;
  const int w = blockIdx.x, row = blockIdx.y;  // grid (P + 1, rows)
  const int r = row / width, j = row % width;
  const int t = threadIdx.x, lo = w * FA_SLICE;
  const int64_t dtok = j < length ? a.drafts[(int64_t)r * length + j] : -1;
  if (w < P) {
    float v[FA_E];
    fa_load_slice(a.logits + (int64_t)row * V, lo, V, row_temperature(a.temperature, row), v);
    const float M = fa_row_max(row, P);
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < FA_E; ++k) {
      const int i = lo + k * FA_NT + t;
      const float e = canon_exp(__fsub_rn(v[k], M));
      if (i < V) {
        sum += canon_fix(e);
        if (i == dtok) dev_store(&g_fa_edraft[row], __float_as_uint(e));
      }
    }
    sum = block_sum_u64<FA_NT>(sum, red);
    if (t == 0) dev_store(&g_fa_sum[row][w], sum);
  } else if (j < length) {
    // workgroup P of a draft row: q(d_j) (1 when the proposal is not valid), while the
    // slices stream: the direct slot of an identity list, else a search of the list (by one
    // thread when it is short, by the block otherwise). Every value here is uniform.
    float qt = 1.0f;
    if (a.valid[r] != 0) {
      const int64_t qrow = ((int64_t)a.slots[r] * length + j) * a.q_width;
      const float* qr = a.q + qrow;
      const int64_t* cr = a.cand + qrow;
      if (dtok >= 0 && dtok < a.q_width && cr[dtok] == dtok)
        qt = qr[dtok];
      else if (a.q_width <= Q_STAGE)
        qt = row_prob_thread(qr, cr, a.q_width, dtok);
      else
        qt = row_prob_block(qr, cr, a.q_width, dtok, red_f);
    }
    if (t == 0) dev_store(&g_fa_qt[row], __float_as_uint(qt));
  }
  if (!fa_last_arrival2(g_fa_cnt1[0][row], P + 1, w == 0, &g_fa_cnt[0][r], width, j == 0))
    return;
  // the request's last workgroup: u_j q(d_j) >= p(d_j) stops the accepted prefix. Every
  // draft row's sums, numerator and q(d_j) are read at once, one per thread.
  __shared__ uint64_t s_rs[64][FA_P_MAX];
  __shared__ float s_ed[64], s_qt[64];
  for (int i = t; i < length * P; i += FA_NT)
    s_rs[i / P][i % P] = dev_load(&g_fa_sum[r * width + i / P][i % P]);
  for (int jj = t; jj < length; jj += FA_NT) {
    s_ed[jj] = __uint_as_float(dev_load(&g_fa_edraft[r * width + jj]));
    s_qt[jj] = __uint_as_float(dev_load(&g_fa_qt[r * width + jj]));
  }
  __syncthreads();
  if (t < WAVE) {
    // lane jj decides draft row jj (the same sums in the same order as a walk over the rows);
    // the prefix stops at the first row that rejects
    bool stop = false;
    if (t < length) {
      const int64_t token = a.drafts[(int64_t)r * length + t];
      uint64_t z = 0;
      for (int i = 0; i < P; ++i) z += s_rs[t][i];
      const float Zf = canon_unfix(z);
      float pt = 0.0f;
      if (token >= 0 && token < V) pt = Zf > 0.0f ? canon_div(s_ed[t], Zf) : 0.0f;
      stop = __fmul_rn(a.uniform[(int64_t)r * width + t], s_qt[t]) >= pt;
    }
    const uint64_t b = __ballot(stop);
    if (t == 0) g_fa_first[r] = b ? (int)__builtin_ctzll(b) : length;
  }
}

// The residual of row `first` for stage 3: q row staged (short candidate lists) or read
// directly (the identity layout), or the one-hot draft when the proposal is not valid.
__device__ ResidualRow fa_residual(const FaArgs& a, int r, int first, int64_t* s_cand,
                                   float* s_q, uint32_t* s_bits) {
  const int length = a.width - 1;
  ResidualRow rr;
  rr.p = nullptr;
  rr.ids = nullptr;
  rr.subtract = first < length;
  if (rr.subtract && a.valid[r] != 0) {
    const int64_t qrow = ((int64_t)a.slots[r] * length + first) * a.q_width;
    rr.q = a.q + qrow;
    rr.cand = a.cand + qrow;
  } else {
    rr.q = nullptr;
    rr.cand = nullptr;
  }
  rr.q_width = a.q_width;
  rr.draft = rr.subtract ? a.drafts[(int64_t)r * length + first] : -1;
  stage_q(rr, s_cand, s_q, s_bits);
  return rr;
}

__global__ void __launch_bounds__(FA_NT) fa_pick_kernel(const float* __restrict__ h_logits, const float* __restrict__ h_temperature, int h_V, int h_width, int h_P, FaArgs a) {
  a.logits = h_logits, a.temperature = h_temperature, a.V = h_V, a.width = h_width, a.P = h_P;
  __shared__ uint64_t red[FA_NT / WAVE];
  __shared__ uint64_t s_sub[2][FA_NT / WAVE];
  __shared__ uint64_t buf[FA_NT];
  __shared__ int64_t s_cand[Q_STAGE];
  __shared__ float s_q[Q_STAGE];
  __shared__ uint32_t s_bits[Q_BITS_WORDS];
  __shared__ float s_zf;
  __shared__ int s_slice, s_sub_i, s_use_p;
  __shared__ uint64_t s_base, s_target;
  // one workgroup per sub-chunk c of slice w (the thread's logits k in [4c, 4c + 4) of the
  // slice): four times the workgroups of one per slice, a quarter of the arithmetic each
  const int P = a.P, width = a.width, length = width - 1, V = a.V;
  const int c = blockIdx.x, w = blockIdx.y, r = blockIdx.z;  // grid (sub-chunks, P, b)
  const int t = threadIdx.x, lo = w * FA_SLICE;
  const int first = g_fa_first[r];
  const int row = r * width + first;
  const float* x = a.logits + (int64_t)row * V;
  const float T = row_temperature(a.temperature, row);
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = lo + (4 * c + k) * FA_NT + t;
    v[k] = x[i < V ? i : V - 1];
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = __fdiv_rn(v[k], T);
  const float M = fa_row_max(row, P);
  if (t < WAVE) {
    const uint64_t z = fa_row_zsum(row, P);
    if (t == 0) s_zf = canon_unfix(z);
  }
  ResidualRow rr = fa_residual(a, r, first, s_cand, s_q, s_bits);  // (synchronises the block)
  const float Zf = s_zf;
  // residual and p of the sub-chunk's logits, summed. An identity q row is read here, all of
  // the thread's values at once.
  float qv[4];
  int64_t cv[4];
  const bool direct_q = rr.q && !rr.bits && rr.subtract;
  if (direct_q) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = lo + (4 * c + k) * FA_NT + t;
      const bool in_q = i < rr.q_width;
      qv[k] = in_q ? rr.q[i] : 0.0f;
      cv[k] = in_q ? rr.cand[i] : -1;
    }
  }
  auto residual = [&](int k, int ii, float p) -> float {
    if (!direct_q) return rr.from_loaded(ii, p, ii);
    // as ResidualRow::from_loaded on an identity layout (ids[k] == k)
    const float qk = cv[k] == ii ? qv[k] : row_prob_thread(rr.q, rr.cand, rr.q_width, ii);
    const float d = __fsub_rn(p, qk);
    return d > 0.0f ? d : 0.0f;
  };
  const int wv = t / WAVE, l = t % WAVE;
  {
    uint64_t rs = 0, ps = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = lo + (4 * c + k) * FA_NT + t;
      const int ii = i < V ? i : V - 1;
      const float e = canon_exp(__fsub_rn(v[k], M));
      const float p = Zf > 0.0f ? canon_div(e, Zf) : 0.0f;
      if (i < V) {  // (padding never reaches the list search)
        rs += canon_fix(residual(k, ii, p));
        ps += canon_fix(p);
      }
    }
    rs = wave_sum_u64(rs);
    ps = wave_sum_u64(ps);
    if (l == 0) {
      s_sub[0][wv] = rs;
      s_sub[1][wv] = ps;
    }
  }
  __syncthreads();
  if (t < 2) {
    uint64_t s = 0;
    for (int q = 0; q < FA_NT / WAVE; ++q) s += s_sub[t][q];
    dev_store(t ? &g_fa_psub[r][w][c] : &g_fa_rsub[r][w][c], s);
  }
  if (!fa_last_arrival2(g_fa_cnt1[1][r * FA_P_MAX + w], FA_SUBCHUNKS, c == 0, &g_fa_cnt[1][r], P,
                        w == 0))
    return;
  // the request's last workgroup: #{k : prefix(k) <= floor(u R)} over the row; every
  // sub-chunk sum read at once, one per thread
  __shared__ uint64_t s_all[2][FA_P_MAX * FA_SUBCHUNKS];
  for (int i = t; i < 2 * P * FA_SUBCHUNKS; i += FA_NT) {
    const int kind = i / (P * FA_SUBCHUNKS), e = i % (P * FA_SUBCHUNKS);
    s_all[kind][e] = kind ? dev_load(&g_fa_psub[r][e / FA_SUBCHUNKS][e % FA_SUBCHUNKS])
                          : dev_load(&g_fa_rsub[r][e / FA_SUBCHUNKS][e % FA_SUBCHUNKS]);
  }
  __syncthreads();
  if (t < WAVE) {
    // wave 0: R, the target floor(u R) and the first sub-chunk whose running sum exceeds it
    // (lane l holds sub-chunks 2l and 2l + 1; integer sums, so the same R and prefix as a
    // sequential walk)
    const int n = P * FA_SUBCHUNKS;
    const int e0 = 2 * t, e1 = 2 * t + 1;
    uint64_t a0 = e0 < n ? s_all[0][e0] : 0, a1 = e1 < n ? s_all[0][e1] : 0;
    uint64_t R = wave_sum_u64(a0 + a1);
    int use_p = 0;
    if (R == 0) {  // (uniform)
      use_p = 1;
      a0 = e0 < n ? s_all[1][e0] : 0;
      a1 = e1 < n ? s_all[1][e1] : 0;
      R = wave_sum_u64(a0 + a1);
    }
    const uint64_t target = canon_scale_floor(a.uniform[(int64_t)r * width + width - 1], R);
    const uint64_t pair = a0 + a1;
    uint64_t incl = pair;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
      const uint32_t lo32 = (uint32_t)__shfl_up((int)(uint32_t)incl, d, WAVE);
      const uint32_t hi32 = (uint32_t)__shfl_up((int)(uint32_t)(incl >> 32), d, WAVE);
      if (t >= d) incl += ((uint64_t)hi32 << 32) | lo32;
    }
    const uint64_t excl = incl - pair;
    const uint64_t b0 = __ballot(e0 < n && excl + a0 > target);
    const uint64_t b1 = __ballot(e1 < n && excl + pair > target);
    const uint64_t any = b0 | b1;
    if (t == 0) {
      s_target = target;
      s_use_p = use_p;
    }
    if (any == 0) {
      if (t == 0) {
        s_slice = P;
        s_sub_i = FA_SUBCHUNKS;
        s_base = R;
      }
    } else {
      const int L = (int)__builtin_ctzll(any);
      const bool at0 = (b0 >> L) & 1ull;
      if (t == L) {
        const int e = at0 ? e0 : e1;
        s_slice = e / FA_SUBCHUNKS;
        s_sub_i = e % FA_SUBCHUNKS;
        s_base = at0 ? excl : excl + a0;
      }
    }
  }
  __syncthreads();
  int64_t pick = V - 1;  // past every prefix: the last index (clamp)
  if (s_slice < P) {
    // the sub-chunk again in vocabulary order: thread t holds logits 4t .. 4t + 3
    const bool use_p = s_use_p != 0;
    const uint64_t target = s_target;
    const int c0 = s_slice * FA_SLICE + s_sub_i * FA_SUB + 4 * t;
    uint64_t f[4];
    uint64_t run = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = c0 + e;
      const int ii = i < V ? i : V - 1;
      const float ex = canon_exp(__fsub_rn(__fdiv_rn(x[ii], T), M));
      const float p = Zf > 0.0f ? canon_div(ex, Zf) : 0.0f;
      const float wgt = use_p ? p : rr.from_loaded(ii, p, ii);
      f[e] = i < V ? canon_fix(wgt) : 0;
      run += f[e];
    }
    uint64_t pre = s_base + block_exclusive_scan_u64<FA_NT>(run, buf);
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (c0 + e < V) {
        pre += f[e];
        cnt += pre <= target;
      }
    }
    cnt = (uint32_t)block_sum_u64<FA_NT>(cnt, red);
    pick = (int64_t)s_slice * FA_SLICE + (int64_t)s_sub_i * FA_SUB + cnt;
    if (pick > V - 1) pick = V - 1;
  }
  if (t < width) {
    a.out[(int64_t)r * width + t] =
        t < first ? a.drafts[(int64_t)r * length + t] : (t == first ? pick : -1);
  }
  if (t == 0) a.accepted[r] = first + 1;
}

__global__ void __launch_bounds__(FA_NT) fa_greedy_kernel(const float* __restrict__ h_logits, const float* __restrict__ h_temperature, int h_V, int h_width, int h_P, FaArgs a) {
  a.logits = h_logits, a.temperature = h_temperature, a.V = h_V, a.width = h_width, a.P = h_P;
  __shared__ uint64_t red[FA_NT / WAVE];
  __shared__ int64_t s_tok[64];
  const int P = a.P, width = a.width, length = width - 1, V = a.V;
  const int w = blockIdx.x, row = blockIdx.y;  // grid (P, rows)
  const int r = row / width, j = row % width;
  const int t = threadIdx.x, lo = w * FA_SLICE;
  const float* x = a.logits + (int64_t)row * V;
  float v[FA_E];
#pragma unroll
  for (int k = 0; k < FA_E; ++k) {
    const int i = lo + k * FA_NT + t;
    v[k] = x[i < V ? i : V - 1];
  }
  uint64_t best = 0;
#pragma unroll
  for (int k = 0; k < FA_E; ++k) {
    const int i = lo + k * FA_NT + t;
    const uint64_t key = argmax_key(v[k], (uint32_t)i);
    if (i < V) best = key > best ? key : best;
  }
  best = block_max_u64<FA_NT>(best, red);
  if (t == 0) dev_store(&g_fa_amax[row][w], best);
  if (!fa_last_arrival2(g_fa_cnt1[2][row], P, w == 0, &g_fa_cnt[2][r], width, j == 0)) return;
  __shared__ uint64_t s_keys[64][FA_P_MAX];
  for (int i = t; i < width * P; i += FA_NT)
    s_keys[i / P][i % P] = dev_load(&g_fa_amax[r * width + i / P][i % P]);
  __syncthreads();
  if (t < width) {
    uint64_t b = 0;
    for (int i = 0; i < P; ++i) b = s_keys[t][i] > b ? s_keys[t][i] : b;
    const int64_t tok = (int64_t)argmax_key_index(b);
    s_tok[t] = tok;
    a.out[(int64_t)r * width + t] = tok;
  }
  __syncthreads();
  if (t == 0) {
    int64_t acc = 1;
    while (acc < width && s_tok[acc - 1] == a.drafts[(int64_t)r * length + acc - 1]) ++acc;
    a.accepted[r] = acc;
  }
}

int fa_slices(int64_t V) { return (int)((V + FA_SLICE - 1) / FA_SLICE); }

}  // namespace

// Extension: rejection-sampling acceptance straight from the logits for requests whose
// candidate lists are the whole vocabulary (see above). logits [b * width, vocab]; the
// remaining arguments as snowllm_draft_reject with p = softmax(logits / T) over the
// vocabulary. b * width <= 256, width <= 64. Calls on one device must be stream-ordered
// (library-owned statistics and counters).
SV_API int snowverify_accept_reject(const float* logits, const float* temperature,
                                    const int64_t* drafts, const int64_t* cand, const float* q,
                                    const int32_t* slots, const int32_t* valid,
                                    const float* uniform, int64_t* out, int64_t* accepted,
                                    int64_t b, int64_t width, int64_t vocab, int64_t q_width,
                                    void* stream) {
  if (b <= 0 || width < 1 || vocab <= 0 || q_width < 0 || !logits || !slots || !valid ||
      !uniform || !out || !accepted || (width > 1 && !drafts))
    return SV_EINVAL;
  // beyond the fused kernels' shapes: the caller takes probabilities + draft_reject
  if (width > 64 || b * width > FA_ROWS || vocab > VOCAB_MAX) return SV_ENOTSUP;
  const int P = fa_slices(vocab);
  FaArgs a{logits, temperature, drafts, cand, q, slots, valid, uniform, out, accepted,
           (int)vocab, (int)width, P, q_width};
  // grids without division (slice in x); the fields the first loads need come again as
  // leading arguments, which arrive preloaded in SGPRs (the struct does not)
  const dim3 rows((unsigned)P, (unsigned)(b * width)), reqs(FA_SUBCHUNKS, (unsigned)P, (unsigned)b);
  hipLaunchKernelGGL(fa_max_kernel, rows, dim3(FA_NT), 0, S(stream), logits, temperature,
                     (int)vocab, (int)width, P, a);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(fa_sum_kernel, dim3((unsigned)(P + 1), (unsigned)(b * width)), dim3(FA_NT), 0,
                     S(stream), logits, temperature,
                     (int)vocab, (int)width, P, a);
  SV_CHECK_LAUNCH();
  hipLaunchKernelGGL(fa_pick_kernel, reqs, dim3(FA_NT), 0, S(stream), logits, temperature,
                     (int)vocab, (int)width, P, a);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension: greedy acceptance straight from the logits: tokens [b, width] = argmax of each
// row (NaN as -inf, first index) and accepted [b] = 1 + leading matches with drafts [b,
// width - 1] -- snowllm_sampling_argmax + snowllm_spec_accept in one launch. Limits as
// snowverify_accept_reject.
SV_API int snowverify_accept_greedy(const float* logits, const int64_t* drafts, int64_t* tokens,
                                    int64_t* accepted, int64_t b, int64_t width, int64_t vocab,
                                    void* stream) {
  if (b <= 0 || width < 1 || vocab <= 0 || !logits || !tokens || !accepted ||
      (width > 1 && !drafts))
    return SV_EINVAL;
  // beyond the fused kernel's shapes: the caller takes argmax + spec_accept
  if (width > 64 || b * width > FA_ROWS || vocab > VOCAB_MAX) return SV_ENOTSUP;
  const int P = fa_slices(vocab);
  FaArgs a{logits, nullptr, drafts, nullptr, nullptr, nullptr, nullptr, nullptr, tokens,
           accepted, (int)vocab, (int)width, P, 0};
  hipLaunchKernelGGL(fa_greedy_kernel, dim3((unsigned)P, (unsigned)(b * width)), dim3(FA_NT), 0,
                     S(stream), logits, (const float*)nullptr, (int)vocab, (int)width, P, a);
  SV_CHECK_LAUNCH();
  return SV_OK;
}
