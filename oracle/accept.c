/*
 * CPU oracle for the acceptance side of the verify step. TEST INFRASTRUCTURE ONLY: it is
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker,
 * never by the product path.
 *
 * It restates the reference's sampling semantics with one canonical arithmetic:
 *   - softmax numerators e = exp(x - max) by Cody & Waite reduction + degree-7 Taylor
 *     polynomial (every step one IEEE binary32 operation, fmaf for the fused ones);
 *   - every sum that feeds a decision in 44-bit fixed point, floor(w * 2^44), so the result
 *     does not depend on summation order;
 *   - probabilities below FLT_MIN flushed to zero.
 * Built with gcc -O2 -ffp-contract=off (no reassociation, no contraction).
 *
 * Reference semantics followed (paths relative to the SnowLLM tree):
 *   argmax          tests/test_sampling_argmax.py:29-30 (NaN -> -inf, first index)
 *   spec_accept     snowllm/engine/spec_decode.py:196-207 (1 + leading matches)
 *   probabilities   tests/test_dflash_sampling.py:199-209, snowllm/engine/request.py:29-35
 *   reject          tests/test_dflash_sampling.py:94-119
 *   sample          tests/test_dflash_sampling.py:212-217
 *   penalties       snowllm/ops/sampling.py:94-100 (closed kernel: the published convention,
 *                   pinned by tests/test_runtime_buffers.py:136-143 and exact-arithmetic cases)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define FIX_BITS 44

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oc_exp(float x) {
  if (!(x >= -86.0f)) return 0.0f;
  const float kLog2e = 1.44269502162933349609375f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.428606765330187045037746429443359375e-06f;
  float t = x * kLog2e;
  float n = rintf(t);
  float r = fmaf(-n, kLn2Hi, x);
  r = fmaf(-n, kLn2Lo, r);
  float p = 1.98412698412698412698e-4f;
  p = fmaf(p, r, 1.38888888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

float oc_div(float a, float b) {
  float q = a / b;
  return fabsf(q) < 1.17549435082228750797e-38f ? 0.0f : q;
}

uint64_t oc_fix(float w) {
  if (!(w > 0.0f)) return 0;
  return (uint64_t)floorf(ldexpf(w, FIX_BITS));
}

float oc_u64_to_f32(uint64_t v) {
  if (v == 0) return 0.0f;
  int msb = 63 - __builtin_clzll(v);
  if (msb <= 23) return (float)(uint32_t)v;
  int shift = msb - 23;
  uint64_t mant = v >> shift;
  uint64_t rem = v & ((1ull << shift) - 1);
  uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (mant & 1))) {
    mant += 1;
    if (mant == (1ull << 24)) { mant >>= 1; shift += 1; }
  }
  return ldexpf((float)(uint32_t)mant, shift);
}

float oc_unfix(uint64_t v) { return ldexpf(oc_u64_to_f32(v), -FIX_BITS); }

uint64_t oc_scale_floor(float u, uint64_t R) {
  if (!(u > 0.0f)) return 0;
  uint32_t bits = f2u(u);
  int e = (int)((bits >> 23) & 0xff);
  uint64_t m = (e == 0) ? (bits & 0x7fffffu) : ((bits & 0x7fffffu) | 0x800000u);
  int exp2 = (e == 0 ? 1 : e) - 127 - 23;
  unsigned __int128 prod = (unsigned __int128)m * (unsigned __int128)R;
  int sh = -exp2;
  if (sh >= 128) return 0;
  return (uint64_t)(prod >> sh);
}

uint32_t oc_ord_key(float f) {
  if (f != f) f = -INFINITY;
  if (f == 0.0f) f = 0.0f;
  uint32_t u = f2u(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static float ord_key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return u2f(u);
}

/* ---- argmax: tests/test_sampling_argmax.py:29-30 ---------------------------------- */
void oc_argmax(const float* logits, int64_t* out, int64_t B, int64_t V) {
  for (int64_t r = 0; r < B; ++r) {
    const float* x = logits + r * V;
    uint32_t best = 0;
    int64_t idx = 0;
    for (int64_t i = 0; i < V; ++i) {
      uint32_t k = oc_ord_key(x[i]);
      if (k > best) { best = k; idx = i; }
    }
    /* all keys equal to the minimum (e.g. every entry -inf or NaN): first index */
    out[r] = idx;
  }
}

/* ---- spec_accept: snowllm/engine/spec_decode.py:196-207 ----------------------------- */
void oc_spec_accept(const int64_t* tokens, const int64_t* drafts, int64_t* acc, int64_t b,
                    int64_t t, int64_t ts, int64_t ds) {
  for (int64_t r = 0; r < b; ++r) {
    int64_t a = 1;
    for (int64_t j = 0; j + 1 < t; ++j) {
      if (tokens[r * ts + j] != drafts[r * ds + j]) break;
      ++a;
    }
    acc[r] = a;
  }
}

/* ---- temperature softmax (dense) ------------------------------------------------------
 * p_i = e_i / Z, e_i = exp(x_i / T - max_j x_j / T), Z = sum of fixed-point e_i.
 * (softmax(scores / T): tests/test_dflash_sampling.py:206; kernel_temperature 1.0 for T<=0:
 * snowllm/engine/request.py:34-35) */
void oc_softmax(const float* logits, float* dense, int64_t rows, int64_t vocab,
                const float* temperature) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = logits + r * vocab;
    float* e = dense + r * vocab;
    float T = temperature ? temperature[r] : 1.0f;
    if (!(T > 0.0f)) T = 1.0f;
    uint32_t mk = 0;
    for (int64_t i = 0; i < vocab; ++i) {
      uint32_t k = oc_ord_key(x[i] / T);
      if (k > mk) mk = k;
    }
    const float M = ord_key_to_float(mk);
    uint64_t Z = 0;
    for (int64_t i = 0; i < vocab; ++i) {
      float v = oc_exp((x[i] / T) - M);
      e[i] = v;
      Z += oc_fix(v);
    }
    const float Zf = oc_unfix(Z);
    for (int64_t i = 0; i < vocab; ++i) e[i] = Zf > 0.0f ? oc_div(e[i], Zf) : 0.0f;
  }
}

/* ---- top-k / top-p candidate lists ---------------------------------------------------
 * tests/test_dflash_sampling.py:199-209: top-k of the row, softmax over the survivors,
 * keep while (exclusive cumulative mass) < top_p, renormalise. Ties go to the lower id. */
typedef struct { uint32_t key; uint32_t idx; } KeyIdx;

static int cmp_desc(const void* a, const void* b) {
  const KeyIdx* x = (const KeyIdx*)a;
  const KeyIdx* y = (const KeyIdx*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

int oc_topk_topp(const float* dense, float* values, int64_t* ids, int64_t rows, int64_t vocab,
                 int64_t width, const int32_t* top_k, const float* top_p) {
  int unsupported = 0;
  KeyIdx* buf = (KeyIdx*)malloc(sizeof(KeyIdx) * (size_t)vocab);
  for (int64_t r = 0; r < rows; ++r) {
    const float* p = dense + r * vocab;
    float* ov = values + r * width;
    int64_t* oi = ids + r * width;
    int64_t k = top_k ? (int64_t)top_k[r] : vocab;
    if (k <= 0 || k > vocab) k = vocab;
    const float tp = top_p ? top_p[r] : 1.0f;
    const int nucleus = tp < 1.0f;
    if (k >= vocab && !nucleus) {
      for (int64_t i = 0; i < width; ++i) {
        ov[i] = i < vocab ? p[i] : 0.0f;
        oi[i] = i < vocab ? i : -1;
      }
      continue;
    }
    if (k > width) {  /* the list cannot hold the top k */
      for (int64_t i = 0; i < width; ++i) { ov[i] = NAN; oi[i] = -2; }
      unsupported = 1;
      continue;
    }
    for (int64_t i = 0; i < vocab; ++i) { buf[i].key = oc_ord_key(p[i]); buf[i].idx = (uint32_t)i; }
    qsort(buf, (size_t)vocab, sizeof(KeyIdx), cmp_desc);
    uint64_t S = 0;
    for (int64_t i = 0; i < k; ++i) S += oc_fix(p[buf[i].idx]);
    const float Sf = oc_unfix(S);
    uint64_t* fix = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)k);
    int* dropped = (int*)malloc(sizeof(int) * (size_t)k);
    for (int64_t i = 0; i < k; ++i) {
      float v = Sf > 0.0f ? oc_div(p[buf[i].idx], Sf) : 0.0f;
      ov[i] = v;
      oi[i] = buf[i].idx;
      fix[i] = oc_fix(v);
    }
    for (int64_t i = k; i < width; ++i) { ov[i] = 0.0f; oi[i] = -1; }
    if (!nucleus) { free(fix); free(dropped); continue; }
    const double limit = (double)tp * (double)(1ull << FIX_BITS);
    uint64_t pre = 0, kept = 0;
    for (int64_t i = 0; i < k; ++i) {
      int keep = (double)pre < limit;
      pre += fix[i];
      dropped[i] = !keep;
      if (keep) kept += fix[i];
    }
    const float Kf = oc_unfix(kept);
    for (int64_t i = 0; i < k; ++i)
      ov[i] = (dropped[i] || !(Kf > 0.0f)) ? 0.0f : oc_div(ov[i], Kf);
    free(fix);
    free(dropped);
  }
  free(buf);
  return unsupported;
}

/* ---- penalties: snowllm/ops/sampling.py:94-100, staged by snowllm/engine/sampler.py:187-220 --
 * The reference kernel is closed; this restates the published convention of OpenAI-style
 * sampling parameters (also the reference's own test expectation at
 * tests/test_runtime_buffers.py:136-143: repetition 2 turns a logit of 8 into 4): a listed id's
 * logit is divided by the repetition penalty when positive and multiplied by it otherwise,
 * then frequency * count and presence (count > 0) are subtracted, one binary32 operation each. */
void oc_penalties(float* logits, const int64_t* ids, const int32_t* counts, int64_t n,
                  int64_t vocab, float presence, float frequency, float repetition) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t t = ids[i];
    if (t < 0 || t >= vocab) continue;
    const int c = counts[i];
    float x = logits[t];
    if (repetition != 1.0f) x = x > 0.0f ? x / repetition : x * repetition;
    x = x - frequency * (float)c;
    x = x - (c > 0 ? presence : 0.0f);
    logits[t] = x;
  }
}

/* ---- sample: pick = #(u >= cumsum(values)) clamped: tests/test_dflash_sampling.py:212-217 */
void oc_pick_rows(const float* values, const int64_t* ids, int64_t rows, int64_t width,
                  const float* uniform, int64_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = values + r * width;
    const int64_t* id = ids + r * width;
    const float u = uniform[r];
    const uint64_t target = u > 0.0f ? (uint64_t)floorf(ldexpf(u, FIX_BITS)) : 0;
    uint64_t pre = 0;
    int64_t pick = 0;
    for (int64_t i = 0; i < width; ++i) {
      pre += oc_fix(v[i]);
      if (pre <= target) ++pick; else break;
    }
    if (pick > width - 1) pick = width - 1;
    int64_t t = id[pick];
    while (t < 0 && pick > 0) t = id[--pick];
    out[r] = t;
  }
}

/* ---- rejection sampling: tests/test_dflash_sampling.py:94-119 ----------------------- */
/* Sum of the probabilities of every slot whose id equals token. A row that is exactly the
 * identity list 0..n-1 has one match, at index token. */
static int is_identity(const int64_t* idsr, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (idsr[i] != i) return 0;
  return 1;
}

static float row_prob(const float* probs, const int64_t* idsr, int64_t n, int64_t token) {
  float acc = 0.0f;
  for (int64_t i = 0; i < n; ++i)
    if (idsr[i] == token) acc = acc + probs[i];
  return acc;
}

void oc_reject(const float* p, const int64_t* ids, const int64_t* drafts, const int64_t* cand,
               const float* q, const int32_t* slots, const int32_t* valid, const float* uniform,
               int64_t* out, int64_t* accepted, int64_t b, int64_t width, int64_t p_width,
               int64_t q_width) {
  const int64_t length = width - 1;
  for (int64_t r = 0; r < b; ++r) {
    const int64_t slot = slots[r];
    int64_t first = length;
    for (int64_t j = 0; j < length; ++j) {
      const int64_t token = drafts[r * length + j];
      const int64_t prow = r * width + j;
      const float pt = is_identity(ids + prow * p_width, p_width)
                           ? ((token >= 0 && token < p_width) ? 0.0f + p[prow * p_width + token] : 0.0f)
                           : row_prob(p + prow * p_width, ids + prow * p_width, p_width, token);
      float qt = 1.0f;
      if (valid[r]) {
        const int64_t qrow = (slot * length + j) * q_width;
        qt = is_identity(cand + qrow, q_width)
                 ? ((token >= 0 && token < q_width) ? 0.0f + q[qrow + token] : 0.0f)
                 : row_prob(q + qrow, cand + qrow, q_width, token);
      }
      if (uniform[r * width + j] * qt >= pt) { first = j; break; }
    }
    for (int64_t j = 0; j < width; ++j) out[r * width + j] = j < first ? drafts[r * length + j] : -1;
    const int64_t prow = r * width + first;
    const float* pr = p + prow * p_width;
    const int64_t* ir = ids + prow * p_width;
    float* res = (float*)malloc(sizeof(float) * (size_t)p_width);
    const int64_t qrow_f = (slot * length + (first < length ? first : 0)) * q_width;
    const int q_ident = (first < length && valid[r]) ? is_identity(cand + qrow_f, q_width) : 0;
    for (int64_t k = 0; k < p_width; ++k) {
      float v = pr[k];
      if (first < length) {
        float qk;
        if (valid[r]) {
          const int64_t qrow = qrow_f;
          if (q_ident)
            qk = (ir[k] >= 0 && ir[k] < q_width) ? 0.0f + q[qrow + ir[k]] : 0.0f;
          else
            qk = row_prob(q + qrow, cand + qrow, q_width, ir[k]);
        } else {
          qk = ir[k] == drafts[r * length + first] ? 1.0f : 0.0f;
        }
        float d = v - qk;
        v = d > 0.0f ? d : 0.0f;
      }
      res[k] = v;
    }
    uint64_t R = 0;
    for (int64_t k = 0; k < p_width; ++k) R += oc_fix(res[k]);
    if (R == 0) {
      for (int64_t k = 0; k < p_width; ++k) { res[k] = pr[k]; R += oc_fix(pr[k]); }
    }
    const uint64_t target = oc_scale_floor(uniform[r * width + width - 1], R);
    uint64_t pre = 0;
    int64_t pick = 0;
    for (int64_t k = 0; k < p_width; ++k) {
      pre += oc_fix(res[k]);
      if (pre <= target) ++pick; else break;
    }
    if (pick > p_width - 1) pick = p_width - 1;
    out[r * width + first] = ir[pick];
    accepted[r] = first + 1;
    free(res);
  }
}

/* ---- DFlash 2 selector: snowllm/ops/dflash.py:164-198; tests/test_dflash_sampling.py:44-75,
 * tests/test_dflash_selector_topk.py:42-61 -----------------------------------------------------
 * Per batch row b and position j (row = b * ell + j, prev = the previous pick, anchor[b] at
 * j = 0): the 16 largest logits in stable descending order (NaN as -inf, -0 == +0), scores =
 * value + correction, then the first argmax (greedy: no temperature or T <= 0) or a pick from
 * softmax(scores / T). The correction is the device's canonical sum: the products
 * pred * hp * succ are exact in binary32 (sampling rows round pred * hp to bf16 first, as
 * torch's bf16 product does); lane l of 64 sums r = l E .. l E + E - 1 (E = R / 64) in order,
 * and the 64 lane sums meet in a balanced binary tree in lane order; sampling rows round the
 * sum to bf16. The softmax and the pick use the canonical exp / fixed-point arithmetic. */
#define SEL_K 16

static float bf16f(uint16_t h) { return u2f((uint32_t)h << 16); }

static float round_bf16(float f) {
  if (f != f) return f;
  uint32_t u = f2u(f);
  u += 0x7fffu + ((u >> 16) & 1u);  /* round to nearest even on the dropped 16 bits */
  return u2f(u & 0xffff0000u);
}

float oc_round_bf16(float f) { return round_bf16(f); }

float oc_select_dot(const uint16_t* pred_row, const uint16_t* hp_row, const uint16_t* succ_row,
                    int64_t R, int sampling) {
  const int64_t E = R / 64;
  float lanes[64];
  for (int l = 0; l < 64; ++l) {
    float part = 0.0f;
    for (int64_t i = 0; i < E; ++i) {
      const int64_t r = l * E + i;
      float prod = bf16f(pred_row[r]) * bf16f(hp_row[r]);
      if (sampling) prod = round_bf16(prod);
      part = part + prod * bf16f(succ_row[r]);
    }
    lanes[l] = part;
  }
  for (int step = 1; step < 64; step *= 2)
    for (int l = 0; l < 64; l += 2 * step) lanes[l] = lanes[l] + lanes[l + step];
  return sampling ? round_bf16(lanes[0]) : lanes[0];
}

void oc_select(const uint16_t* hp, const float* logits, const uint16_t* pred,
               const uint16_t* succ, const int64_t* anchor, const float* temperature,
               const float* uniform, const int32_t* slots, int64_t* path, int64_t* cand,
               float* q, int64_t b, int64_t ell, int64_t V, int64_t R) {
  KeyIdx* buf = (KeyIdx*)malloc(sizeof(KeyIdx) * (size_t)V);
  for (int64_t bi = 0; bi < b; ++bi) {
    int64_t prev = anchor[bi];
    const float T = temperature ? temperature[bi] : 0.0f;
    const int sampling = T > 0.0f;
    for (int64_t j = 0; j < ell; ++j) {
      const int64_t row = bi * ell + j;
      const float* x = logits + row * V;
      for (int64_t i = 0; i < V; ++i) { buf[i].key = oc_ord_key(x[i]); buf[i].idx = (uint32_t)i; }
      qsort(buf, (size_t)V, sizeof(KeyIdx), cmp_desc);
      int64_t id[SEL_K];
      float score[SEL_K], qv[SEL_K];
      for (int c = 0; c < SEL_K; ++c) {
        id[c] = buf[c].idx;
        const float corr = oc_select_dot(pred + prev * R, hp + row * R, succ + id[c] * R, R,
                                         sampling);
        score[c] = ord_key_to_float(buf[c].key) + corr;
      }
      int pick = 0;
      if (!sampling) {
        uint32_t best = oc_ord_key(score[0]);
        for (int c = 1; c < SEL_K; ++c) {
          const uint32_t k = oc_ord_key(score[c]);
          if (k > best) { best = k; pick = c; }
        }
        for (int c = 0; c < SEL_K; ++c) qv[c] = c == pick ? 1.0f : 0.0f;
      } else {
        float xs[SEL_K], e[SEL_K];
        uint32_t mk = 0;
        for (int c = 0; c < SEL_K; ++c) {
          xs[c] = score[c] / T;
          const uint32_t k = oc_ord_key(xs[c]);
          if (k > mk) mk = k;
        }
        const float M = ord_key_to_float(mk);
        uint64_t Z = 0;
        for (int c = 0; c < SEL_K; ++c) { e[c] = oc_exp(xs[c] - M); Z += oc_fix(e[c]); }
        const float Zf = oc_unfix(Z);
        for (int c = 0; c < SEL_K; ++c) qv[c] = Zf > 0.0f ? oc_div(e[c], Zf) : 0.0f;
        const float u = uniform[row];
        const uint64_t target = u > 0.0f ? (uint64_t)floorf(ldexpf(u, FIX_BITS)) : 0;
        uint64_t pre = 0;
        int n = 0;
        for (int c = 0; c < SEL_K; ++c) { pre += oc_fix(qv[c]); n += pre <= target; }
        pick = n < SEL_K - 1 ? n : SEL_K - 1;
      }
      path[row] = id[pick];
      if (cand) {
        const int64_t base = ((int64_t)slots[bi] * ell + j) * SEL_K;
        for (int c = 0; c < SEL_K; ++c) { cand[base + c] = id[c]; q[base + c] = qv[c]; }
      }
      prev = id[pick];
    }
  }
  free(buf);
}
