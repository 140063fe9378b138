// Paged GQA attention of a verify block (T query rows per request) against a paged bf16 KV
// cache, split over the context (flash-decoding) and merged by a second kernel.
//
// KV pool layouts are the reference's (tests/test_lfm2_dspark_reference.py:30-36):
//   K: [blocks, Hkv, d/16, page, 16]   V: [blocks, Hkv, page/4, d, 4]   (bf16, page = 16)
// so one (page, kv head) is a contiguous 2*d*16-byte run of each.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16), per wave = one 16-row tile of query rows of one kv
// head, over 32-key chunks (two pages):
//   S^T[key, row] = K[key, :] . Q[row, :]      A = K (16 keys x 32 d, 16-byte lane loads)
//                                              B = Q^T (held in registers)
//   O^T[d, row]  += V^T[d, key] . P^T[key, row] A = V^T (two 8-byte lane loads per page)
//                                              B = P^T, straight from the S^T registers
// Putting keys on the M side makes the C layout of S^T (row = lane & 15, key = 4*(lane>>4)+i)
// exactly the B layout P^T needs, so the softmax never leaves registers.
//
// Query rows of a kv head are ordered r = t * G + g (token t of the block, q head g of the
// group); rows >= T*G are padding. Row t of request b sees context keys [0, L - T) and block
// key j (position L - T + j) iff bit j of its ancestor mask is set (causal: j <= t).
#include "common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int PAGE = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int SPLITS_MAX = 512;

struct AttnArgs {
  const uint16_t* q;        // [batch*T, Hq, D]
  const uint16_t* k_pool;   // [blocks, Hkv, D/16, 16, 16]
  const uint16_t* v_pool;   // [blocks, Hkv, 4, D, 4]
  const int32_t* table;     // [batch, table_stride]
  const int32_t* lens;      // [batch] total keys incl. the block
  const uint64_t* tree;     // [batch*T] ancestor masks or null (causal)
  float* part_o;            // [batch, Hkv, NRT, S, 16, D]
  float* part_ml;           // [batch, Hkv, NRT, S, 16, 2]
  int T, Hq, Hkv, G, NRT, S, pages_per_split, table_stride;
  float qk_scale;           // softmax scale * log2(e)
};

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  u32x4 v = *(const u32x4*)p;
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}

template <int D>
__global__ void __launch_bounds__(64) attn_split_kernel(AttnArgs a) {
  constexpr int DS = D / 32;  // MFMA k-steps over the head dimension
  constexpr int DT = D / 16;  // 16-wide d tiles of the output
  const int lane = threadIdx.x;
  const int kq = lane >> 4, col = lane & 15;

  // XCD-aware block mapping: consecutive block ids land on different XCDs (id % 8), so the
  // NRT row tiles of one (request, kv head, split) are given ids that share id % 8.
  const int nblk = gridDim.x;
  const int id = blockIdx.x;
  int lin;
  {
    const int per_x = nblk / 8, rem = nblk % 8;
    const int xcd = id % 8, local = id / 8;
    lin = (xcd < rem) ? xcd * (per_x + 1) + local : rem * (per_x + 1) + (xcd - rem) * per_x + local;
    if (nblk < 8) lin = id;
  }
  const int tile = lin % a.NRT;
  int rest = lin / a.NRT;
  const int split = rest % a.S;
  rest /= a.S;
  const int h = rest % a.Hkv;
  const int b = rest / a.Hkv;

  int L = a.lens[b];
  if (L > a.table_stride * PAGE) L = a.table_stride * PAGE;  // never read past the table row
  const int ctx = L - a.T;
  const int n_pages = (L + PAGE - 1) / PAGE;
  const int p0 = split * a.pages_per_split;
  int p1 = p0 + a.pages_per_split;
  if (p1 > n_pages) p1 = n_pages;

  // this lane's query row (column of S^T / O^T)
  const int r = tile * 16 + col;
  const bool row_live = r < a.T * a.G;
  const int t = row_live ? r / a.G : 0;
  const int g = row_live ? r % a.G : 0;
  const int hq = h * a.G + g;
  uint64_t anc;
  if (a.tree) anc = row_live ? a.tree[(int64_t)b * a.T + t] : 1ull;
  else anc = (t >= 63) ? ~0ull : ((2ull << t) - 1ull);
  // Q^T operand: 8 consecutive d per k-step
  bf16x8 qb[DS];
  {
    const uint16_t* qrow = a.q + (((int64_t)b * a.T + t) * a.Hq + hq) * D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      if (row_live) qb[ds] = load_bf16x8(qrow + ds * 32 + kq * 8);
      else qb[ds] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    }
  }

  floatx4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_huge_valf();  // running max (log2 domain)
  float l = 0.f;

  const int64_t page_elems = (int64_t)PAGE * D;          // one (page, head) of K or V
  const int64_t block_elems = page_elems * a.Hkv;
  const int32_t* trow = a.table + (int64_t)b * a.table_stride;

  for (int pg = p0; pg < p1; pg += 2) {
    const bool has2 = pg + 1 < p1;
    const int blk0 = trow[pg];
    const int blk1 = has2 ? trow[pg + 1] : blk0;
    const uint16_t* k0 = a.k_pool + blk0 * block_elems + h * page_elems;
    const uint16_t* k1 = a.k_pool + blk1 * block_elems + h * page_elems;
    const uint16_t* v0 = a.v_pool + blk0 * block_elems + h * page_elems;
    const uint16_t* v1 = a.v_pool + blk1 * block_elems + h * page_elems;
    // S^T for the two pages
    floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      // K layout [D/16][16 keys][16 d]: d = ds*32 + kq*8 .. +7 -> chunk 2*ds + kq/2, offset 8*(kq&1)
      const int chunk = 2 * ds + (kq >> 1);
      const int off = (chunk * PAGE + col) * 16 + 8 * (kq & 1);
      bf16x8 ka = load_bf16x8(k0 + off);
      bf16x8 kb = load_bf16x8(k1 + off);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[ds], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qb[ds], s1, 0, 0, 0);
    }
    // mask + online softmax (row = col; keys 4*kq+i of each page)
    float sv[8];
    float cmax = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int page = pg + (i >> 2);
      const int key = 4 * kq + (i & 3);
      const int pos = page * PAGE + key;
      bool vis = pos < L && (i < 4 || has2);
      if (vis && pos >= ctx) vis = (anc >> (pos - ctx)) & 1ull;
      const float s = (i < 4 ? s0[i & 3] : s1[i & 3]) * a.qk_scale;
      sv[i] = vis ? s : -__builtin_huge_valf();
      cmax = sv[i] > cmax ? sv[i] : cmax;
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(m, cmax);
    const float msafe = (m_new == -__builtin_huge_valf()) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - msafe);  // exp2(-inf) = 0
    float psum = 0.f;
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = __builtin_amdgcn_exp2f(sv[i] - msafe);
      psum += p[i];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int i = 0; i < DT; ++i) o[i] *= alpha;
    // P^T operand: slots 0..3 page 0 keys 4kq+i, slots 4..7 page 1 keys 4kq+i. P is carried
    // as a bf16 pair (hi + lo residual), which keeps ~16 significant bits through the MFMA.
    float plo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) plo[i] = p[i] - bf16_to_f32(f32_to_bf16(p[i]));
    u32x4 pw = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                pack_bf16x2(p[6], p[7])};
    u32x4 pwl = {pack_bf16x2(plo[0], plo[1]), pack_bf16x2(plo[2], plo[3]),
                 pack_bf16x2(plo[4], plo[5]), pack_bf16x2(plo[6], plo[7])};
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
    const bf16x8 pbl = __builtin_bit_cast(bf16x8, pwl);
    // O^T += V^T P^T ; V layout [4 key groups][D][4 keys]: keys 4kq..4kq+3 of d -> 8 bytes
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = dt * 16 + col;
      const int off = (kq * D + d) * 4;
      u32x2 va = *(const u32x2*)(v0 + off);
      u32x2 vb = *(const u32x2*)(v1 + off);
      if (!has2) vb = u32x2{0u, 0u};
      u32x4 vv = {va.x, va.y, vb.x, vb.y};
      const bf16x8 vt = __builtin_bit_cast(bf16x8, vv);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pb, o[dt], 0, 0, 0);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pbl, o[dt], 0, 0, 0);
    }
  }
  // partial results: O^T lane holds row col, d = dt*16 + 4*kq + i
  const int64_t pidx = ((((int64_t)b * a.Hkv + h) * a.NRT + tile) * a.S + split);
  float* po = a.part_o + pidx * 16 * D + (int64_t)col * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) *(floatx4*)(po + dt * 16 + 4 * kq) = o[dt];
  if (kq == 0) {
    float* pml = a.part_ml + (pidx * 16 + col) * 2;
    pml[0] = m;
    pml[1] = l;
  }
}

// Merge the splits of one (request, kv head, row tile): out = sum_s 2^(m_s-M) O_s / sum_s 2^(m_s-M) l_s
template <int D>
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnArgs a, uint16_t* __restrict__ out) {
  __shared__ float w[16][SPLITS_MAX];  // per-row split weights
  __shared__ float inv_l[16];
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t pbase = (((int64_t)b * a.Hkv + h) * a.NRT + tile) * a.S;
  if (threadIdx.x < 16) {
    const int row = threadIdx.x;
    float M = -__builtin_huge_valf();
    for (int s = 0; s < a.S; ++s) M = fmaxf(M, a.part_ml[((pbase + s) * 16 + row) * 2]);
    const float Ms = (M == -__builtin_huge_valf()) ? 0.f : M;
    float lsum = 0.f;
    for (int s = 0; s < a.S; ++s) {
      const float ms = a.part_ml[((pbase + s) * 16 + row) * 2];
      const float ls = a.part_ml[((pbase + s) * 16 + row) * 2 + 1];
      const float ws = __builtin_amdgcn_exp2f(ms - Ms);
      w[row][s] = ws;
      lsum += ws * ls;
    }
    inv_l[row] = lsum > 0.f ? 1.0f / lsum : 0.f;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * D; idx += 256) {
    const int row = idx / D, d = idx % D;
    const int r = tile * 16 + row;
    if (r >= a.T * a.G) continue;
    float acc = 0.f;
    for (int s = 0; s < a.S; ++s) acc += w[row][s] * a.part_o[((pbase + s) * 16 + row) * D + d];
    const int t = r / a.G, g = r % a.G;
    out[(((int64_t)b * a.T + t) * a.Hq + h * a.G + g) * D + d] = f32_to_bf16(acc * inv_l[row]);
  }
}

inline int n_row_tiles(int T, int G) { return (T * G + 15) / 16; }

int choose_splits(int64_t batch, int Hkv, int NRT, int64_t pages) {
  // aim for ~2 waves of row-tile programs per CU, at least two pages per split
  const int64_t programs = batch * Hkv * NRT;
  int64_t s = (2 * 256 * 4 + programs - 1) / programs;
  const int64_t max_by_pages = (pages + 1) / 2;
  if (s > max_by_pages) s = max_by_pages;
  if (s < 1) s = 1;
  if (s > SPLITS_MAX) s = SPLITS_MAX;
  return (int)s;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

// Scratch for the split partials of snowverify_paged_attention.
SV_API int64_t snowverify_paged_attention_scratch_bytes(int64_t batch, int64_t tokens,
                                                        int64_t num_heads, int64_t num_kv_heads,
                                                        int64_t head_size) {
  if (batch <= 0 || tokens <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const int G = (int)(num_heads / num_kv_heads);
  const int NRT = n_row_tiles((int)tokens, G);
  const size_t parts = (size_t)batch * num_kv_heads * NRT * SPLITS_MAX * 16;
  return (int64_t)(align256(parts * head_size * 4) + align256(parts * 2 * 4));
}

// Extension entry with explicit shapes (the reference's geometry is compiled in; this build
// takes shapes at run time). q [batch*tokens, Hq, D] bf16; out same; table [batch, stride]
// i32; lens [batch] i32 = context + tokens; tree [batch*tokens] u64 ancestor masks or null for
// causal. The block's K/V must already be in the pools.
SV_API int snowverify_paged_attention(const void* q, const void* k_pool, const void* v_pool,
                                      void* out, const int32_t* table, const int32_t* lens,
                                      const uint64_t* tree, int64_t batch, int64_t tokens,
                                      int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
                                      int64_t page_size, int64_t table_stride, float scale,
                                      void* scratch, int64_t scratch_bytes, void* stream) {
  if (batch <= 0 || tokens <= 0 || tokens > 64 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads || page_size != PAGE || table_stride <= 0)
    return SV_EINVAL;
  if (head_size != 128 && head_size != 256) return SV_ENOTSUP;
  if (scratch_bytes < snowverify_paged_attention_scratch_bytes(batch, tokens, num_heads,
                                                              num_kv_heads, head_size))
    return SV_EINVAL;
  AttnArgs a;
  a.q = (const uint16_t*)q;
  a.k_pool = (const uint16_t*)k_pool;
  a.v_pool = (const uint16_t*)v_pool;
  a.table = table;
  a.lens = lens;
  a.tree = tree;
  a.T = (int)tokens;
  a.Hq = (int)num_heads;
  a.Hkv = (int)num_kv_heads;
  a.G = (int)(num_heads / num_kv_heads);
  a.NRT = n_row_tiles(a.T, a.G);
  a.table_stride = (int)table_stride;
  a.S = choose_splits(batch, a.Hkv, a.NRT, table_stride);
  a.pages_per_split = (int)((table_stride + a.S - 1) / a.S);
  if (a.pages_per_split & 1) a.pages_per_split += 1;
  a.S = (int)((table_stride + a.pages_per_split - 1) / a.pages_per_split);
  a.qk_scale = scale * kLog2e;
  const size_t parts = (size_t)batch * a.Hkv * a.NRT * SPLITS_MAX * 16;
  a.part_o = (float*)scratch;
  a.part_ml = (float*)((char*)scratch + align256(parts * head_size * 4));
  hipStream_t s = (hipStream_t)stream;
  const int64_t nprog = batch * a.Hkv * a.NRT * a.S;
  if (head_size == 128) {
    hipLaunchKernelGGL(attn_split_kernel<128>, dim3((unsigned)nprog), dim3(64), 0, s, a);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(a.NRT, a.Hkv, (unsigned)batch), dim3(256), 0,
                       s, a, (uint16_t*)out);
  } else {
    hipLaunchKernelGGL(attn_split_kernel<256>, dim3((unsigned)nprog), dim3(64), 0, s, a);
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(attn_merge_kernel<256>, dim3(a.NRT, a.Hkv, (unsigned)batch), dim3(256), 0,
                       s, a, (uint16_t*)out);
  }
  SV_CHECK_LAUNCH();
  return SV_OK;
}
