// Paged GQA attention of a verify block (T query rows per request) against a paged bf16 KV
// cache, split over the context (flash-decoding) and merged by a second kernel.
//
// KV pool layouts are the reference's (tests/test_lfm2_dspark_reference.py:30-36):
//   K: [blocks, Hkv, d/16, page, 16]   V: [blocks, Hkv, page/4, d, 4]   (bf16, page = 16)
// so one (page, kv head) is a contiguous 32*d-byte run of each.
//
// One workgroup per (request, kv head, context split), one wave per 16-row tile of the
// head's query rows. The pages of the split stream through an LDS ring with direct
// global->LDS loads (global_load_lds_dwordx4, 1 KiB per wave instruction), RING - 1 pages
// ahead of the MFMAs, so K and V leave HBM once per workgroup whatever the number of tiles.
// Each wave waits for its own loads of a page (vmcnt) and a barrier publishes the page.
//
// MFMA mapping, per wave and 32-key chunk (two pages):
//   S^T[key, row] = K[key, :] . Q[row, :]      v_mfma_f32_16x16x32_bf16 over d, per page:
//                                              A = K (16 keys x 32 d, ds_read_b128)
//                                              B = Q^T (held in registers)
//   O^T[d, row]  += V^T[d, key] . P^T[key, row] v_mfma_f32_16x16x32_bf16 over the 32 keys:
//                                              A = V^T (two ds_read_b64 per d tile)
//                                              B = P^T, straight from the S^T registers
// Putting keys on the M side makes the C layout of S^T (row = lane & 15, key = 4*(lane>>4)+i)
// exactly the B layout P^T needs, so the softmax never leaves registers.
//
// Query rows of a kv head are ordered r = t * G + g (token t of the block, q head g of the
// group); rows >= T*G are padding. Row t of request b sees context keys [0, L - T) and block
// key j (position L - T + j) iff bit j of its ancestor mask is set (causal: j <= t).
#include "common.h"
#include "geometry.h"
#include "kquant_core.h"
#include "qknorm.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short short4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(4))) const int32_t cint32;

constexpr int PAGE = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int SPLITS_MAX = 512;
constexpr int MAX_TILES = 8;     // row tiles per workgroup: T * G <= 128
constexpr int MAX_TILES_DH = 4;  // up to 4 tiles, each tile's output columns split over 2 waves
// Waves of a split workgroup: eight for one wave per tile (with or without row groups) and for
// the mixed form; two per tile, rounded up to a power of two, for two waves per tile. A page's
// sixteen 1 KiB loads then split evenly over the waves, with no repeated chunk, and waves past
// the workgroup's row tiles only load pages (more waves issuing the loads: config 4 attention
// 21.2 -> 20.0 us per launch with four waves per row group, 19.5 with eight).
__host__ __device__ inline int split_waves(int dh, int nrt) {
  if (dh != 2) return MAX_TILES;
  return nrt <= 1 ? 2 : nrt <= 2 ? 4 : 8;
}
// The fused QK-norm form rotates at most 128 dims of a head (half <= 64): wider rotations of a
// 256-wide head would not fit the kernel's registers, and the entry point refuses them.
constexpr int FUSED_MAX_HS = 2;

struct AttnArgs {
  const uint16_t* q;        // [batch*T, Hq, D], rows q_stride elements apart
  int64_t q_stride;
  const uint16_t* k_pool;   // [blocks, Hkv, D/16, 16, 16]
  const uint16_t* v_pool;   // [blocks, Hkv, 4, D, 4]
  const int32_t* table;     // [batch, table_stride]
  const int32_t* lens;      // [batch] total keys incl. the block
  const uint64_t* tree;     // [batch*T] ancestor masks or null (causal)
  float* part_o;            // [batch, Hkv, NRT, S, 16, D]
  float* part_ml;           // [batch, Hkv, NRT, S, 16, 2]
  int T, Hq, Hkv, G, NRT, S, pages_per_split, table_stride;
  int RG;                   // row groups: workgroups that share one (request, head, split)
  float qk_scale;           // softmax scale * log2(e)
  // QK-norm + RoPE + the block's K/V write done here (proj != null): q head hq of block row m
  // at proj + m * proj_stride + hq * q_head_stride, k / v head h at k_off / v_off + h * D;
  // cos/sin rows cs_stride apart; slots [batch*T] the rows' cache slots; q_out optional.
  const uint16_t* proj;
  int64_t proj_stride, q_head_stride, k_off, v_off, cs_stride;
  const uint16_t* q_gamma;
  const uint16_t* k_gamma;
  const float* cosv;
  const float* sinv;
  const int32_t* slots;
  uint16_t* q_out;
  uint16_t* k_pool_w;
  uint16_t* v_pool_w;
  int rot_half;
  float eps;
};

// LDS image of one (page, kv head): K as in HBM, then V with its four key groups padded apart
// (VPAD bytes) so the four lane groups of a V^T read fall on different banks.
template <int D>
struct SlotGeo {
  static constexpr int KBYTES = PAGE * D * 2;           // K (and V) bytes of one page
  static constexpr int CHUNKS = 2 * KBYTES / 1024;      // 1 KiB load chunks per page, K then V
  static constexpr int VGROUP = D * 8;                  // bytes of one V key group (4 keys x D)
  static constexpr int VPAD = 128;
  static constexpr int BYTES = KBYTES + 4 * (VGROUP + VPAD);
};

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  u32x4 v = *(const u32x4*)p;
  return __builtin_bit_cast(bf16x8, v);
}

// s_waitcnt on the LDS/scalar counter only: this wave's LDS writes have completed.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
}

// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 7 and lgkmcnt 15 = no wait on those).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that the compiler may not move memory accesses across, without the
// release fence of __syncthreads (which would wait for every load in flight).
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Issue wave w's CPW chunk loads of one (page, head) into an LDS slot. Chunk ids past the
// page wrap around (an identical second copy), so every wave issues exactly CPW loads and the
// vmcnt bookkeeping is the same for all waves.
template <int D, int CPW>
__device__ __forceinline__ void dma_page(const uint8_t* __restrict__ kp,
                                         const uint8_t* __restrict__ vp, uint8_t* slot, int w,
                                         int NW, int lane) {
  using G = SlotGeo<D>;
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    int c = w + i * NW;
    if (c >= G::CHUNKS) c -= G::CHUNKS;
    const uint8_t* src;
    uint8_t* dst;
    if (c < G::CHUNKS / 2) {
      src = kp + c * 1024;
      dst = slot + c * 1024;
    } else {
      const int off = (c - G::CHUNKS / 2) * 1024;
      src = vp + off;
      dst = slot + G::KBYTES + (off / G::VGROUP) * (G::VGROUP + G::VPAD) + off % G::VGROUP;
    }
    __builtin_amdgcn_global_load_lds((const void*)(src + lane * 16), (lds_void*)dst, 16, 0, 0);
  }
}

// Online-softmax state of one wave (16 query rows = lanes' columns, D / DH output columns):
// O^T, the row's reference maximum m (log2 domain) and this lane's part of the row sum l.
template <int D, int DH>
struct AttnState {
  floatx4 o[D / 16 / DH];
  float m, l;
};
constexpr float RESCALE = 8.0f;  // p = 2^(s - m) stays <= 2^8 between rescales

// Two pages (32 keys) from their LDS slots: the two S^T products are independent MFMA
// chains; P^T of both pages forms one 16x16x32 B operand (slots 0..3 = page A keys 4kq + i,
// slots 4..7 = page B keys 4kq + i) and V^T reads the same keys of both pages, so O^T += V^T P^T
// takes half the MFMA cycles of two 16x16x16 steps. Keys of page B are masked when !has_b.
// SPLIT_S (two waves per row tile): each wave of the pair takes the S^T of one page and the
// pair swaps them through LDS (xch: the tile's two 1 KiB halves), so a K page is read and
// multiplied once per tile. XBAR: a wave of a mixed workgroup that computes its own S^T takes
// part in the same barrier. Every wave of a workgroup makes the same number of barrier calls.
template <int D, int DH, bool SPLIT_S = false, bool XBAR = false>
__device__ __forceinline__ void attend_chunk(AttnState<D, DH>& st, const uint8_t* sa, bool has_b,
                                             const bf16x8 (&qb)[D / 32], int pg, int L, int ctx,
                                             uint64_t anc, float qk_scale, int kq, int col,
                                             int dhalf, floatx4 (*xch)[64] = nullptr) {
  using G = SlotGeo<D>;
  constexpr int DS = D / 32, DT = D / 16 / DH;
  constexpr int NK = SPLIT_S ? 1 : 2;  // pages whose S^T this wave computes
  static_assert(!SPLIT_S || DH == 2, "S^T is split between the two waves of a tile");
  const uint8_t* sb = sa + G::BYTES;  // the chunk's second page: the next ring slot
  // V^T operands first: one ds_read2st64_b64 per d tile reads the same 8 bytes (keys 4kq..4kq+3
  // at one d) of both slots, G::BYTES apart, into the x,y (page A) and z,w (page B) halves of
  // the MFMA's A operand. The compiler does not count these reads, so they are issued before
  // its own K reads (LDS reads complete in order: its waits for K then also cover them) and an
  // explicit wait precedes their use.
  static_assert(G::BYTES % 512 == 0 && G::BYTES / 512 + (DT * 2 * 16 * 8) / 512 <= 255,
                "ds_read2st64 offsets");
  u32x4 vr[DT];
  {
    const uint32_t v0 = (uint32_t)(uintptr_t)(const lds_void*)(sa + G::KBYTES) +
                        kq * (G::VGROUP + G::VPAD) + (dhalf * DT * 16 + col) * 8;
    uint32_t va[4];
#pragma unroll
    for (int i = 0; i < 4 && i < DT; ++i) va[i] = v0 + i * 128;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      asm volatile("ds_read2st64_b64 %0, %1 offset0:%2 offset1:%3"
                   : "=v"(vr[dt])
                   : "v"(va[dt & 3]), "i"(dt >> 2), "i"((dt >> 2) + G::BYTES / 512));
  }
  u32x4 kr[NK][DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const int off = ((2 * ds + (kq >> 1)) * PAGE + col) * 32 + (kq & 1) * 16;
    if constexpr (NK == 1) {
      kr[0][ds] = *(const u32x4*)((dhalf ? sb : sa) + off);
    } else {
      kr[0][ds] = *(const u32x4*)(sa + off);
      kr[NK - 1][ds] = *(const u32x4*)(sb + off);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  floatx4 sk[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) sk[k] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
#pragma unroll
    for (int k = 0; k < NK; ++k)
      sk[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[k][ds]),
                                                     qb[ds], sk[k], 0, 0, 0);
  floatx4 s0, s1;
  if constexpr (SPLIT_S) {
    const int lane = kq * 16 + col;
    xch[dhalf][lane] = sk[0];
    wait_lgkmcnt0();
    block_barrier();
    const floatx4 other = xch[dhalf ^ 1][lane];
    s0 = dhalf ? other : sk[0];
    s1 = dhalf ? sk[0] : other;
  } else {
    if constexpr (XBAR) block_barrier();
    s0 = sk[0];
    s1 = sk[NK - 1];
  }
  // raw scores (masked keys -inf); the softmax scale goes into the exponent's fma, and the
  // maximum of the raw scores times the (positive) scale is the maximum of the scaled ones
  float sv[8];
  if (has_b && (pg + 2) * PAGE <= ctx) {
    // both pages lie wholly in the context before the block: every key is visible (the same
    // scores as the masked form below, without its per-key tests)
#pragma unroll
    for (int i = 0; i < 8; ++i) sv[i] = i < 4 ? s0[i & 3] : s1[i & 3];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int pos = (pg + (i >> 2)) * PAGE + 4 * kq + (i & 3);
      bool vis = pos < L && (i < 4 || has_b);
      if (vis && pos >= ctx) vis = (anc >> (pos - ctx)) & 1ull;
      sv[i] = vis ? (i < 4 ? s0[i & 3] : s1[i & 3]) : -__builtin_huge_valf();
    }
  }
  float cmax = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                     fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
  cmax *= qk_scale;
  // Lazy rescaling: the row maximum (shared by the four lanes of a row, which hold different
  // keys of one P^T column) moves only when some score exceeds it by more than 2^RESCALE in
  // the exp2 domain; otherwise p <= 2^RESCALE and nothing is rescaled. The decision is
  // wave-uniform, so every lane of a row keeps the same reference. Row sums stay per lane
  // until the end of the split.
  if (__builtin_amdgcn_ballot_w64(cmax > st.m + RESCALE) != 0) {
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(st.m, cmax);
    // 0 when the row had no visible key yet; 1 for a row that still has none
    const float alpha =
        m_new == -__builtin_huge_valf() ? 1.0f : __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.o[dt] *= alpha;
    st.l *= alpha;
    st.m = m_new;
  }
  const float nm = (st.m == -__builtin_huge_valf()) ? 0.f : -st.m;
  float p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], qk_scale, nm));
    st.l += p[i];
  }
  // P^T as a bf16 pair through the MFMA, ~16 significant bits: hi = p truncated to its upper
  // 16 bits (the packed pair is a byte permute of two values), lo = p - hi (exact in fp32),
  // rounded to bf16
  uint32_t ph[4], pl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = __float_as_uint(p[2 * j]), b = __float_as_uint(p[2 * j + 1]);
    ph[j] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    pl[j] = pack_bf16x2(p[2 * j] - __uint_as_float(a & 0xffff0000u),
                        p[2 * j + 1] - __uint_as_float(b & 0xffff0000u));
  }
  const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{ph[0], ph[1], ph[2], ph[3]});
  const bf16x8 pbl = __builtin_bit_cast(bf16x8, u32x4{pl[0], pl[1], pl[2], pl[3]});
  // the V^T reads have completed (and the registers are not used before this point)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) asm volatile("" : "+v"(vr[dt]));
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const bf16x8 vt = __builtin_bit_cast(bf16x8, vr[dt]);
    floatx4 o = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pb, st.o[dt], 0, 0, 0);
    st.o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pbl, o, 0, 0, 0);
  }
}

// DH: waves per row tile, 1 or 2 for every tile; 3 = mixed: the first 2 NRT - NW tiles have one
// wave each, the remaining NW - NRT tiles two (the pairs split S^T, see attend_chunk), so that
// up to eight waves spread the tiles' matrix work evenly over the four SIMDs.
// The fields the prologue needs first come again as leading scalar arguments: those arrive
// preloaded in SGPRs, while the struct is read from kernel-argument memory.
template <int D, int CPW, int RING, int DH>
__global__ void __launch_bounds__(DH == 2 ? MAX_TILES_DH * 2 * 64 : MAX_TILES * 64)
attn_split_kernel(const int32_t* __restrict__ h_table, const int32_t* __restrict__ h_lens,
                  int h_S, int h_Hkv, int h_pps, int h_tstride, int h_T, int h_G, int h_NRT,
                  int h_RG, AttnArgs a) {
  a.table = h_table, a.lens = h_lens, a.S = h_S, a.Hkv = h_Hkv, a.pages_per_split = h_pps;
  a.table_stride = h_tstride, a.T = h_T, a.G = h_G, a.NRT = h_NRT;
  using G = SlotGeo<D>;
  constexpr int DS = D / 32;
  constexpr bool MIXED = DH == 3;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING * G::BYTES];
  __shared__ floatx4 xch[MIXED ? MAX_TILES : 1][2][64];  // S^T swap of the pairs (mixed)
  // Q operands of the row tiles that two waves share: the first wave of the pair fetches (and,
  // fused, normalises and rotates) the rows and passes the operands on through LDS
  constexpr int QSH_PAIRS = MIXED ? MAX_TILES - 5 : (DH == 2 ? MAX_TILES_DH : 0);
  constexpr size_t QSH_BYTES = (size_t)QSH_PAIRS * DS * 64 * 16;
  constexpr bool QSHARE =
      QSH_PAIRS > 0 && RING * G::BYTES + QSH_BYTES + sizeof(xch) <= 150 * 1024;
  __shared__ u32x4 qsh[QSHARE ? QSH_PAIRS : 1][DS][64];
  // waves (the launch's; blockDim would be a kernel-argument load)
  const int NW = split_waves(DH, h_NRT);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int w, dhalf;  // row tile, output-column part
  bool pair;     // two waves share the tile
  if constexpr (DH == 1) {
    w = wv, dhalf = 0, pair = false;
  } else if constexpr (DH == 2) {
    w = wv >> 1, dhalf = wv & 1, pair = true;
  } else {
    const int nx = 2 * a.NRT - NW;  // single-wave tiles
    pair = wv >= nx;
    w = pair ? nx + ((wv - nx) >> 1) : wv;
    dhalf = pair ? (wv - nx) & 1 : 0;
  }
  const int kq = lane >> 4, col = lane & 15;
  // grid (S, Hkv, batch): the workgroups of a head's splits stay consecutive, and no division.
  // Two row groups (one wave per tile): x = 16 * (split / 8) + 8 * group + split % 8, so the
  // two workgroups of a split are 8 apart in dispatch order and land on the same XCD (the
  // XCDs take workgroups in turn), where the second one's page loads are served by that
  // XCD's L2; x past the last split returns at once.
  int split = blockIdx.x;
  bool idle = false;  // wave-uniform
  if constexpr (DH == 1) {
    if (h_RG == 2) {
      const int x = blockIdx.x;
      const int half = (h_NRT + 1) >> 1;  // tiles of the first group
      split = ((x >> 4) << 3) | (x & 7);
      idle = w >= half;
      w += (x & 8) ? half : 0;
      if (split >= h_S) return;
    }
  }
  const int h = blockIdx.y, b = blockIdx.z;
  // a wave past its group's row tiles loads its share of the pages and takes part in every
  // barrier, but multiplies and writes nothing
  idle = idle || w >= h_NRT;

  // this lane's query row (column of S^T / O^T)
  const int r = w * 16 + col;
  const bool row_live = !idle && r < a.T * a.G;
  const int t = row_live ? r / a.G : 0;
  const int g = row_live ? r % a.G : 0;
  const int hq = h * a.G + g;
  const int64_t m_row = (int64_t)b * a.T + t;
  // The block ids of the split's first pages need no sequence length: they load with it, so
  // that the page loads wait for one round trip instead of two (block table through the
  // constant address space: scalar loads, which count on lgkmcnt and so never wait for the
  // page loads in flight on vmcnt).
  const int p0 = split * a.pages_per_split;
  const cint32* trow = (const cint32*)(a.table + (int64_t)b * a.table_stride);
  int pre[RING - 2];
#pragma unroll
  for (int i = 0; i < RING - 2; ++i)
    pre[i] = trow[p0 + i < a.table_stride ? p0 + i : a.table_stride - 1];
  int L = a.lens[b];
  if (L > a.table_stride * PAGE) L = a.table_stride * PAGE;  // never read past the table row
  const int ctx = L - a.T;
  const int n_pages = (L + PAGE - 1) / PAGE;
  int p1 = p0 + a.pages_per_split;
  if (p1 > n_pages) p1 = n_pages;
  uint64_t anc;
  if (a.tree) anc = row_live ? a.tree[(int64_t)b * a.T + t] : 1ull;
  else anc = (t >= 63) ? ~0ull : ((2ull << t) - 1ull);

  // the state, set just before the first chunk (the accumulators are not live across the
  // prologue), and the partial results of a wave holding DHW-th of its tile's columns
  auto init_state = [&](auto& st) {
    constexpr int DT = (int)(sizeof(st.o) / sizeof(st.o[0]));
#pragma unroll
    for (int i = 0; i < DT; ++i) st.o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    st.m = -__builtin_huge_valf();
    st.l = 0.f;
  };
  auto write_partials = [&](auto& st) {
    constexpr int DT = (int)(sizeof(st.o) / sizeof(st.o[0]));
    // O^T lane holds row col, d = dt*16 + 4*kq + i
    const int64_t pidx = ((((int64_t)b * a.Hkv + h) * a.NRT + w) * a.S + split);
    // (a padding row's partials are left unwritten: the merges never combine them into an
    // output)
    float* po = a.part_o + pidx * 16 * D + (int64_t)col * D;
    if (row_live)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *(floatx4*)(po + (dhalf * DT + dt) * 16 + 4 * kq) = st.o[dt];
    // row sums: add the four lanes of each row in a fixed order
    float l = st.l + __shfl_xor(st.l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (kq == 0 && dhalf == 0 && row_live) {
      float* pml = a.part_ml + (pidx * 16 + col) * 2;
      pml[0] = st.m;
      pml[1] = l;
    }
  };
  // runs f with this wave's state type (D / 16 / DHW accumulator tiles)
  auto with_state = [&](auto f) {
    if constexpr (DH == 1 || DH == 2) {
      AttnState<D, DH> st;
      f(st);
    } else if (pair) {
      AttnState<D, 2> st;
      f(st);
    } else {
      AttnState<D, 1> st;
      f(st);
    }
  };

  if (p0 < p1) {  // uniform over the workgroup
    // Q^T operand (8 consecutive d per k-step), loaded before the page loads are queued; the
    // fused form fetches the raw projection row and its norm operands here and normalises the
    // row once the first pages are on their way. The second wave of a shared tile takes the
    // operands from LDS after the loop's first barrier instead.
    const int qpi = MIXED ? w - (2 * a.NRT - NW) : w;  // the tile's index among the pairs
    const bool q_from_lds = QSHARE && pair && dhalf == 1;  // wave-uniform
    const bool q_to_lds = QSHARE && pair && dhalf == 0;
    bf16x8 qb[DS];
    QkRaw<D> qraw;
    QkAux<D> qaux;
    if (a.proj) {
      // the block rows whose cache position falls in this split: K normalised and rotated,
      // K and V into the pools (wave 0, 16 rows per pass)
      const int t_lo = p0 * PAGE - ctx > 0 ? p0 * PAGE - ctx : 0;
      const int t_hi = p1 * PAGE - ctx < a.T ? p1 * PAGE - ctx : a.T;
      if (t_lo < t_hi) {  // uniform: this split holds block rows
        if (wv == 0)
          for (int t0 = t_lo; t0 < t_hi; t0 += 16) {
            const int tr = t0 + col;
            const bool live = tr < t_hi;
            const int64_t m = (int64_t)b * a.T + (live ? tr : t_lo);
            uint4 kr[DS];
            qk_load_norm_rope<D, FUSED_MAX_HS>(a.proj + m * a.proj_stride + a.k_off + (int64_t)h * D, live,
                                 a.k_gamma, a.cosv + m * a.cs_stride, a.sinv + m * a.cs_stride,
                                 a.rot_half, a.eps, kq, kr);
            if (live)
              qk_store_kv<D>(kr, a.proj + m * a.proj_stride + a.v_off + (int64_t)h * D,
                             a.k_pool_w, a.v_pool_w, a.slots[m], h, a.Hkv, PAGE, kq);
          }
        wait_vmcnt<0>();  // the block's K/V stores are done ...
        block_barrier();  // ... before any wave queues a page load
      }
      if (!q_from_lds) {
        qk_fetch<D>(qraw, a.proj + m_row * a.proj_stride + (int64_t)hq * a.q_head_stride, kq,
                    row_live);
        qk_fetch_aux<D>(qaux, a.q_gamma, a.cosv + m_row * a.cs_stride,
                        a.sinv + m_row * a.cs_stride, a.rot_half, kq);
      }
    } else if (!q_from_lds) {
      const uint16_t* qrow = a.q + m_row * a.q_stride + (int64_t)hq * D;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        if (row_live) qb[ds] = load_bf16x8(qrow + ds * 32 + kq * 8);
        else qb[ds] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
      }
      wait_vmcnt<0>();  // Q has landed: the loop below then waits on page loads only
    }
    const int64_t page_bytes = (int64_t)G::KBYTES;
    const int64_t block_bytes = page_bytes * a.Hkv;
    const uint8_t* kbase = (const uint8_t*)a.k_pool + h * page_bytes;
    const uint8_t* vbase = (const uint8_t*)a.v_pool + h * page_bytes;
    // pages past the split reload page p0 into a free slot (finite data under the masked
    // second page of an odd last chunk; before the loop the wait for the query row below
    // counts on every wave's RING - 2 page loads behind it). In the loop a chunk that lies
    // wholly past the split is not loaded, and a step waits for every load in flight when
    // fewer than RING - 4 pages are queued behind its own (so the last steps queue nothing
    // that the workgroup's end would have to wait for).
    auto issue = [&](int pg, int slot_idx) {
      const int pgc = pg < p1 ? pg : p0;
      int64_t blk = pgc - p0 < RING - 2 ? pre[0] : trow[pgc];
#pragma unroll
      for (int i = 1; i < RING - 2; ++i)
        if (pgc - p0 == i) blk = pre[i];
      dma_page<D, CPW>(kbase + blk * block_bytes, vbase + blk * block_bytes,
                       ring + slot_idx * G::BYTES, wv, NW, lane);
    };
    // pages go two per step (one 32-key chunk); RING - 2 pages are queued ahead of a step
#pragma unroll
    for (int i = 0; i < RING - 2; ++i) issue(p0 + i, i);
    if (a.proj && !q_from_lds) {
      // this lane's query row, normalised and rotated while the first pages load (angles of
      // sub-blocks past the first, when half > 32, load here behind the pages)
      uint4 qo[DS];
      wait_vmcnt<(RING - 2) * CPW>();  // the row and its operands, not the pages behind them
      qk_norm_rope<D, FUSED_MAX_HS>(qraw, qaux, a.cosv + m_row * a.cs_stride, a.sinv + m_row * a.cs_stride,
                      a.rot_half, a.eps, kq, qo);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const uint4 o = qo[ds];
        qb[ds] = row_live ? __builtin_bit_cast(bf16x8, u32x4{o.x, o.y, o.z, o.w})
                          : __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        if (a.q_out && split == 0 && dhalf == 0 && row_live)
          *(uint4*)(a.q_out + (m_row * a.Hq + hq) * D + ds * 32 + kq * 8) = o;
      }
    }
    if (q_to_lds) {
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) qsh[qpi][ds][lane] = __builtin_bit_cast(u32x4, qb[ds]);
      wait_lgkmcnt0();  // visible to the pair's other wave at the loop's first barrier
    }
    with_state([&](auto& st) {
      constexpr int DT = (int)(sizeof(st.o) / sizeof(st.o[0]));
      constexpr int DHW = D / 16 / DT;
      init_state(st);
      int slot = 0;  // first ring slot of the current chunk (even)
      for (int pg = p0; pg < p1; pg += 2) {
        // this wave's loads of pages pg, pg + 1 have landed (RING - 4 pages queued behind them
        // while both chunks behind this one are loaded) ...
        if (RING == 4 || pg + RING - 4 < p1) wait_vmcnt<(RING - 4) * CPW>();
        else wait_vmcnt<0>();
        block_barrier();                 // ... and every wave's; the previous chunk is free
        if (q_from_lds && pg == p0)
#pragma unroll
          for (int ds = 0; ds < DS; ++ds) qb[ds] = __builtin_bit_cast(bf16x8, qsh[qpi][ds][lane]);
        const int prev = slot == 0 ? RING - 2 : slot - 2;
        if (pg + RING - 2 < p1) {  // (uniform) the chunk is one a later step multiplies
          issue(pg + RING - 2, prev);
          issue(pg + RING - 1, prev + 1);
        }
        if (!idle)
          attend_chunk<D, DHW, MIXED && DHW == 2, MIXED && DHW == 1>(
              st, ring + slot * G::BYTES, pg + 1 < p1, qb, pg, L, ctx,
              anc, a.qk_scale, kq, col, dhalf, xch[MIXED ? w : 0]);
        slot = slot == RING - 2 ? 0 : slot + 2;
      }
      wait_vmcnt<0>();  // no load may still target LDS when the workgroup retires
      if (!idle) write_partials(st);
    });
  } else if (!idle) {
    with_state([&](auto& st) {
      init_state(st);
      write_partials(st);
    });
  }
}

// Merge the splits: out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s. A block covers
// MERGE_ROWS rows x MERGE_D columns of one (request, kv head, row tile). Wave sg sums the
// splits s = sg mod MERGE_SG in increasing s, the MERGE_SG partial sums are added in wave
// order, and wave j < MERGE_ROWS also computes the split weights of row j. Every wave issues
// the loads of its first MERGE_PF splits before the weights are known, so that the partials
// and the (m, l) pairs come back in one round trip.
constexpr int MERGE_ROWS = 4, MERGE_D = 64, MERGE_SG = 8, MERGE_PF = 16;
constexpr int MERGE_THREADS = MERGE_ROWS * (MERGE_D / 4) * MERGE_SG;  // 512

// The split weights of one row (one wave): w[s] = 2^(m_s - M), 1 / sum_s w[s] l_s.
__device__ __forceinline__ void merge_weights(const AttnArgs& a, int64_t pbase, int row,
                                              float* w, float* inv_l, int lane) {
  float M = -__builtin_huge_valf();
  for (int s = lane; s < a.S; s += 64) M = fmaxf(M, a.part_ml[((pbase + s) * 16 + row) * 2]);
  M = wave_max(M);
  const float Ms = (M == -__builtin_huge_valf()) ? 0.f : M;
  float lsum = 0.f;
  for (int s = lane; s < a.S; s += 64) {
    const float* ml = a.part_ml + ((pbase + s) * 16 + row) * 2;
    const float ws = __builtin_amdgcn_exp2f(ml[0] - Ms);
    w[s] = ws;
    lsum += ws * ml[1];
  }
  lsum = wave_sum(lsum);
  if (lane == 0) *inv_l = lsum > 0.f ? 1.0f / lsum : 0.f;
}

// acc (NV floatx4 of this thread's columns) += sum over this group's splits of w[s] * O_s, in
// increasing s; po points at split sg's first column word, sstride = one group step.
template <int NV>
__device__ __forceinline__ void merge_group(const AttnArgs& a, const float* po, int64_t sstride,
                                            const float* w, int sg, floatx4 (&pf)[MERGE_PF][NV],
                                            floatx4 (&acc)[NV]) {
  for (int s0 = sg;; s0 += MERGE_PF * MERGE_SG) {
#pragma unroll
    for (int k = 0; k < MERGE_PF; ++k) {
      const int s = s0 + k * MERGE_SG;
      if (s < a.S)
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] += w[s] * pf[k][v];
    }
    const int next = s0 + MERGE_PF * MERGE_SG;
    if (next >= a.S) break;
    // splits past this batch: the next MERGE_PF, all loads in flight
    po += MERGE_PF * sstride;
#pragma unroll
    for (int k = 0; k < MERGE_PF; ++k)
      if (next + k * MERGE_SG < a.S)
#pragma unroll
        for (int v = 0; v < NV; ++v) pf[k][v] = *(const floatx4*)(po + k * sstride + 4 * v);
  }
}

template <int NV>
__device__ __forceinline__ void merge_prefetch(const AttnArgs& a, const float* po,
                                               int64_t sstride, int sg,
                                               floatx4 (&pf)[MERGE_PF][NV]) {
#pragma unroll
  for (int k = 0; k < MERGE_PF; ++k)
    if (sg + k * MERGE_SG < a.S)
#pragma unroll
      for (int v = 0; v < NV; ++v) pf[k][v] = *(const floatx4*)(po + k * sstride + 4 * v);
}

template <int D>
__global__ void __launch_bounds__(MERGE_THREADS) attn_merge_kernel(AttnArgs a,
                                                                  uint16_t* __restrict__ out) {
  __shared__ float w[MERGE_ROWS][SPLITS_MAX];
  __shared__ float inv_l[MERGE_ROWS];
  __shared__ floatx4 red[MERGE_SG][MERGE_ROWS][MERGE_D / 4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // grid (tile, h * row groups + row group, b * column groups + column group)
  constexpr int RG = 16 / MERGE_ROWS, DG = D / MERGE_D;
  const int tile = blockIdx.x, h = blockIdx.y / RG, b = blockIdx.z / DG;
  const int row0 = (blockIdx.y % RG) * MERGE_ROWS;
  const int d0 = (blockIdx.z % DG) * MERGE_D;
  const int64_t pbase = (((int64_t)b * a.Hkv + h) * a.NRT + tile) * a.S;
  const int sg = wv, rr = lane >> 4, d4 = lane & 15;
  const int row = row0 + rr;
  const int64_t sstride = (int64_t)16 * D * MERGE_SG;
  const float* po = a.part_o + ((pbase + sg) * 16 + row) * D + d0 + 4 * d4;
  floatx4 pf[MERGE_PF][1];
  merge_prefetch<1>(a, po, sstride, sg, pf);
  if (wv < MERGE_ROWS) merge_weights(a, pbase, row0 + wv, w[wv], &inv_l[wv], lane);
  __syncthreads();
  floatx4 acc[1] = {{0.f, 0.f, 0.f, 0.f}};
  merge_group<1>(a, po, sstride, w[rr], sg, pf, acc);
  red[sg][rr][d4] = acc[0];
  __syncthreads();
  if (sg != 0) return;
  floatx4 v = red[0][rr][d4];
#pragma unroll
  for (int j = 1; j < MERGE_SG; ++j) v += red[j][rr][d4];
  const int rg = tile * 16 + row;
  if (rg >= a.T * a.G) return;
  const float il = inv_l[rr];
  const int t = rg / a.G, g = rg % a.G;
  uint16_t* dst = out + (((int64_t)b * a.T + t) * a.Hq + h * a.G + g) * D + d0 + 4 * d4;
  *(u32x2*)dst = u32x2{pack_bf16x2(v[0] * il, v[1] * il), pack_bf16x2(v[2] * il, v[3] * il)};
}

// The merge that also writes the output projection's operand workspace (D = 256: one head's
// output is one 256-wide superblock of the projection's input row, so the projection can take
// prepared operands instead of converting the bf16 output itself). A block covers one row x
// all D columns of one (request, kv head, row tile) -- one block per row puts twice the blocks
// of two rows per block on the CUs; half wave sg sums the splits s = sg mod MERGE_SG for 8
// columns per thread, and the MERGE_SG partial sums are added in group order: the same sums in
// the same order as attn_merge_kernel, so the same output bits.
// Workspace rows are the output rows b * T + t; rows past them are left as they are (the
// GEMV reads none of their operands).
constexpr int MWS_THREADS = (256 / 8) * MERGE_SG;  // 256: one row, a split group per half wave

template <int D>
// (The fields the first loads need come again as leading scalar arguments: those arrive
// preloaded in SGPRs, while the struct is read from kernel-argument memory.)
__global__ void __launch_bounds__(MWS_THREADS) attn_merge_ws_kernel(
    float* __restrict__ h_part_o, float* __restrict__ h_part_ml, int h_S, int h_NRT, int h_Hkv,
    int h_T, int h_G, int h_Hq, AttnArgs a, uint16_t* __restrict__ out, void* __restrict__ ws,
    size_t tile_bytes) {
  a.part_o = h_part_o, a.part_ml = h_part_ml, a.S = h_S, a.NRT = h_NRT, a.Hkv = h_Hkv;
  a.T = h_T, a.G = h_G, a.Hq = h_Hq;
  static_assert(D == 256, "one head per superblock");
  __shared__ float w[SPLITS_MAX];
  __shared__ float inv_l;
  __shared__ floatx4 red[MERGE_SG][D / 8][2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // grid (tile, 16 h + row, b)
  const int tile = blockIdx.x, row = blockIdx.y & 15, h = blockIdx.y >> 4, b = blockIdx.z;
  const int rg = tile * 16 + row;
  if (rg >= a.T * a.G) return;  // a padding row: no output, no operands (uniform)
  const int64_t pbase = (((int64_t)b * a.Hkv + h) * a.NRT + tile) * a.S;
  // half wave sg sums split group sg; a row's 32 words sit in one half wave (the operand
  // conversion reduces over it)
  const int sg = tid >> 5, lw = tid & 31;
  const int64_t sstride = (int64_t)16 * D * MERGE_SG;
  const float* po = a.part_o + ((pbase + sg) * 16 + row) * D + lw * 8;
  floatx4 pf[MERGE_PF][2];
  merge_prefetch<2>(a, po, sstride, sg, pf);
  if (wv == 0) merge_weights(a, pbase, row, w, &inv_l, lane);
  __syncthreads();
  floatx4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  merge_group<2>(a, po, sstride, w, sg, pf, acc);
  red[sg][lw][0] = acc[0];
  red[sg][lw][1] = acc[1];
  __syncthreads();
  if (wv != 0) return;  // wave 0 (a whole wave; its upper half repeats the lower) finishes
  floatx4 v0 = red[0][lw][0], v1 = red[0][lw][1];
#pragma unroll
  for (int j = 1; j < MERGE_SG; ++j) {
    v0 += red[j][lw][0];
    v1 += red[j][lw][1];
  }
  const float il = inv_l;
  const int t = rg / a.G, g = rg % a.G;
  const int hq = h * a.G + g;
  const uint32_t yo[4] = {pack_bf16x2(v0[0] * il, v0[1] * il), pack_bf16x2(v0[2] * il, v0[3] * il),
                          pack_bf16x2(v1[0] * il, v1[1] * il), pack_bf16x2(v1[2] * il, v1[3] * il)};
  if (lane < 32)
    *(u32x4*)(out + (((int64_t)b * a.T + t) * a.Hq + hq) * D + lw * 8) =
        u32x4{yo[0], yo[1], yo[2], yo[3]};
  float y[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[2 * i] = __uint_as_float(yo[i] << 16);
    y[2 * i + 1] = __uint_as_float(yo[i] & 0xffff0000u);
  }
  kq::word_operand(y, hq * 32 + lw, (int64_t)b * a.T + t, ws, tile_bytes,
                   (int64_t)a.Hq * D / kq::QK, lane < 32);
}

inline int n_row_tiles(int T, int G) { return (T * G + 15) / 16; }

int g_pages_per_split = 0;  // 0: automatic

// Compute units of the current device (queried once per device).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                   ? n : 256;
  }
  return cus[dev];
}

// A workgroup's time grows with its pages (measured on MI355X: about 1.2 us per page at
// head_size 256), and one workgroup per CU runs best, so the splits are sized for one round of
// workgroups over the CUs: the fewest pages per split that keep batch * Hkv * splits <= CUs,
// rounded up to an even count, since the pages go two per step and an odd split's last step
// costs as much as a full one (measured: 26.1 -> 25.0 us per layer at 8K with 2 KV heads,
// 5 -> 6 pages; 20.9 -> 20.5 us with 8 KV heads, 17 -> 18). Very short contexts keep at least
// 6 pages per split (more splits only add merge work), 8 at head size 256, where a split's
// fixed start and its partials weigh more against its pages than the CUs it leaves idle
// (2 KV heads over 8K: 65 splits instead of 86, 3.392 -> 3.369 ms per config-4 step; 10 pages:
// 3.404 ms).
int choose_pages_per_split(int64_t batch, int Hkv, int64_t pages, int64_t head_size) {
  int64_t pps = g_pages_per_split;
  if (pps <= 0) {
    const int64_t heads = batch * Hkv;
    const int64_t cus = device_cus();
    const int64_t splits = heads < cus ? cus / heads : 1;
    pps = (pages + splits - 1) / splits;
    pps += pps & 1;
    const int64_t least = head_size >= 256 ? 8 : 6;
    if (pps < least) pps = least;
  }
  while ((pages + pps - 1) / pps > SPLITS_MAX) ++pps;
  return (int)pps;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Waves per row tile: two (each computing S for the full head and O for half of its columns)
// when the tiles fit, so that a workgroup keeps more waves per SIMD; loads per wave per page:
// the page's chunks over the waves, rounded up to a power of two.
int g_ring = 0;  // LDS ring pages: 0 automatic, 4 or 8

template <int D, int DH, int RING>
int launch_split_ring(const AttnArgs& a, int64_t nblocks, hipStream_t s) {
  constexpr int CH = SlotGeo<D>::CHUNKS;
  const int rg = DH == 1 ? a.RG : 1;
  const int nw = split_waves(DH, a.NRT);
  int cpw = 1;
  while (cpw * nw < CH) cpw *= 2;
  if (RING == 8 && cpw == 16) return launch_split_ring<D, DH, 4>(a, nblocks, s);  // vmcnt range
  const unsigned gx = rg == 2 ? (unsigned)(16 * ((a.S + 7) / 8)) : (unsigned)a.S;
  const dim3 grid(gx, (unsigned)a.Hkv, (unsigned)(nblocks / ((int64_t)a.S * a.Hkv))),
      block((unsigned)(64 * nw));
#define SV_SPLIT(CPW_, RING_)                                                                   \
  hipLaunchKernelGGL((attn_split_kernel<D, CPW_, RING_, DH>), grid, block, 0, s, a.table, a.lens, \
                     a.S, a.Hkv, a.pages_per_split, a.table_stride, a.T, a.G, a.NRT, rg, a)
  switch (cpw) {
    case 1: SV_SPLIT(1, RING); break;
    case 2: SV_SPLIT(2, RING); break;
    case 4: SV_SPLIT(4, RING); break;
    case 8: SV_SPLIT(8, RING); break;
    case 16: SV_SPLIT(16, 4); break;
    default: return SV_ENOTSUP;
  }
#undef SV_SPLIT
  return SV_OK;
}

template <int D, int DH>
int launch_split_dh(const AttnArgs& a, int64_t nblocks, hipStream_t s) {
  // long splits keep more pages in flight: eight-page ring from 32 pages per split (220K
  // context, 108 pages per split: 7.33 -> 7.22 ms per config-5 step); shorter ones run as
  // fast on four with half the LDS (config 4: 3.369 against 3.423 ms with eight)
  if (g_ring == 8 || (g_ring == 0 && a.pages_per_split >= 32))
    return launch_split_ring<D, DH, 8>(a, nblocks, s);
  return launch_split_ring<D, DH, 4>(a, nblocks, s);
}

int g_d_split = 0;  // 0: automatic, 1, 2 or 3 (mixed) forced

// automatic: two waves per tile up to MAX_TILES_DH tiles, one wave per tile above (no swap
// barrier). Config 4's five tiles: 3.362 -> 3.351 ms per forward pass against the mixed form;
// config 5's six: 7.21 -> 6.99 ms per step once the one-wave form ran on eight waves (on six,
// with repeated page chunks, the mixed form had been ahead, 7.18 against 7.30 ms).
int choose_dh(int NRT) {
  return g_d_split ? g_d_split : (NRT <= MAX_TILES_DH ? 2 : 1);
}

int g_row_groups = 0;  // 0: automatic, 1 or 2 forced

// Row groups of the one-wave-per-tile form: two workgroups per split, each with half of the
// row tiles, when that keeps the splits nearly as long -- a short context, whose pages per
// split sit at the lower bound, so that one group per split leaves CUs idle while each CU
// runs two tiles on one of its SIMDs. Returns 1 or 2.
int choose_row_groups(int dh, int NRT, int64_t batch, int Hkv, int64_t pages, int64_t head_size) {
  if (dh != 1 || NRT < 3) return 1;
  if (g_row_groups) return g_row_groups;
  const int64_t one = choose_pages_per_split(batch, Hkv, pages, head_size);
  const int64_t two = choose_pages_per_split(2 * batch, Hkv, pages, head_size);
  return two <= one + 2 ? 2 : 1;
}

template <int D>
int launch_split(const AttnArgs& a, int64_t nblocks, hipStream_t s) {
  const int dh = choose_dh(a.NRT);
  if (dh == 2 && a.NRT <= MAX_TILES_DH) return launch_split_dh<D, 2>(a, nblocks, s);
  if (dh == 3 && a.NRT > MAX_TILES / 2 && a.NRT < MAX_TILES)
    return launch_split_dh<D, 3>(a, nblocks, s);
  return launch_split_dh<D, 1>(a, nblocks, s);
}

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
namespace {

int paged_attention_impl(AttnArgs a, const void* q, const void* k_pool, const void* v_pool,
                         void* out, const int32_t* table, const int32_t* lens,
                         const uint64_t* tree, int64_t batch, int64_t tokens, int64_t num_heads,
                         int64_t num_kv_heads, int64_t head_size, int64_t page_size,
                         int64_t table_stride, float scale, void* scratch, int64_t scratch_bytes,
                         void* stream, void* out_ws = nullptr) {
  if (batch <= 0 || tokens <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
      page_size != PAGE || table_stride <= 0)
    return SV_EINVAL;
  if (head_size != 128 && head_size != 256) return SV_ENOTSUP;
  if (out_ws && head_size != 256) return SV_ENOTSUP;
  // grid y/z extents: 16 * kv heads and batch * (head_size / 64) stay within 65535
  if (num_kv_heads > 4095 || batch * (head_size / MERGE_D) > 65535) return SV_ENOTSUP;
  if (n_row_tiles((int)tokens, (int)(num_heads / num_kv_heads)) > MAX_TILES) return SV_ENOTSUP;
  if (scratch_bytes < snowverify_paged_attention_scratch_bytes(batch, tokens, num_heads,
                                                              num_kv_heads, head_size))
    return SV_EINVAL;
  a.q = (const uint16_t*)q;
  if (a.q_stride == 0) a.q_stride = num_heads * head_size;
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
  {
    const int dh = choose_dh(a.NRT);
    // the launch's own test of the form (launch_split): one wave per tile unless two or mixed
    const int dh_run = (dh == 2 && a.NRT <= MAX_TILES_DH) ? 2
                       : (dh == 3 && a.NRT > MAX_TILES / 2 && a.NRT < MAX_TILES) ? 3 : 1;
    a.RG = choose_row_groups(dh_run, a.NRT, batch, a.Hkv, table_stride, head_size);
  }
  // a row group counts as a head for the split sizing: RG * batch * Hkv * S <= CUs
  a.pages_per_split = choose_pages_per_split(batch * a.RG, a.Hkv, table_stride, head_size);
  a.S = (int)((table_stride + a.pages_per_split - 1) / a.pages_per_split);
  a.qk_scale = scale * kLog2e;
  const size_t parts = (size_t)batch * a.Hkv * a.NRT * SPLITS_MAX * 16;
  a.part_o = (float*)scratch;
  a.part_ml = (float*)((char*)scratch + align256(parts * head_size * 4));
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblocks = batch * a.Hkv * a.S;
  const dim3 mgrid((unsigned)a.NRT, (unsigned)(a.Hkv * (16 / MERGE_ROWS)),
                   (unsigned)(batch * (head_size / MERGE_D)));
  int rc;
  if (head_size == 128) {
    rc = launch_split<128>(a, nblocks, s);
    if (rc != SV_OK) return rc;
    SV_CHECK_LAUNCH();
    hipLaunchKernelGGL(attn_merge_kernel<128>, mgrid, dim3(MERGE_THREADS), 0, s, a, (uint16_t*)out);
  } else {
    rc = launch_split<256>(a, nblocks, s);
    if (rc != SV_OK) return rc;
    SV_CHECK_LAUNCH();
    if (out_ws) {
      const size_t tb = kq::xprep_tile_bytes(num_heads * head_size / kq::QK);
      hipLaunchKernelGGL(attn_merge_ws_kernel<256>,
                         dim3((unsigned)a.NRT, (unsigned)(16 * a.Hkv), (unsigned)batch),
                         dim3(MWS_THREADS), 0, s,
                         a.part_o, a.part_ml, a.S, a.NRT, a.Hkv, a.T, a.G, a.Hq, a,
                         (uint16_t*)out, out_ws, tb);
    } else {
      hipLaunchKernelGGL(attn_merge_kernel<256>, mgrid, dim3(MERGE_THREADS), 0, s, a,
                         (uint16_t*)out);
    }
  }
  SV_CHECK_LAUNCH();
  return SV_OK;
}

}  // namespace

SV_API int snowverify_paged_attention(const void* q, const void* k_pool, const void* v_pool,
                                      void* out, const int32_t* table, const int32_t* lens,
                                      const uint64_t* tree, int64_t batch, int64_t tokens,
                                      int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
                                      int64_t page_size, int64_t table_stride, float scale,
                                      void* scratch, int64_t scratch_bytes, void* stream) {
  AttnArgs a = {};
  return paged_attention_impl(a, q, k_pool, v_pool, out, table, lens, tree, batch, tokens,
                              num_heads, num_kv_heads, head_size, page_size, table_stride, scale,
                              scratch, scratch_bytes, stream);
}

// Extension (no counterpart in the reference, which runs snowllm_qk_norm_rope_cache and then
// snowllm_paged_attention): the two in one pair of launches. The attention's workgroups
// normalise and rotate their own query rows from the raw projection rows, and the workgroup
// whose split holds a block row's cache position writes that row's K (normalised, rotated) and
// V into the pools before loading its pages -- the same bits as the separate writer
// (qknorm.h). proj [batch*tokens, proj_stride] bf16 with q head hq at hq * q_head_stride, k / v
// head h at k_off / v_off + h * head_size; cos/sin [batch*tokens, cs_stride] f32 (first `half`
// used; half a multiple of 32, at most 64: wider rotations return hipErrorNotSupported);
// slots [batch*tokens] the cache slot of each block row (position lens[b] - tokens + t, as
// snowllm_resolve_slots gives it); q_out [batch*tokens, Hq, D] or NULL. Other arguments as
// snowverify_paged_attention.
SV_API int snowverify_paged_attention_qk(
    const void* proj, int64_t proj_stride, int64_t q_head_stride, int64_t k_off, int64_t v_off,
    const void* q_gamma, const void* k_gamma, const float* cos_in, const float* sin_in,
    int64_t cs_stride, int64_t half, float eps, const int32_t* slots, void* q_out, void* k_pool,
    void* v_pool, void* out, const int32_t* table, const int32_t* lens, const uint64_t* tree,
    int64_t batch, int64_t tokens, int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
    int64_t page_size, int64_t table_stride, float scale, void* scratch, int64_t scratch_bytes,
    void* stream) {
  if (!proj || !q_gamma || !k_gamma || !cos_in || !sin_in || !slots || half < 0 || half % 32 ||
      2 * half > head_size || proj_stride % 8 || q_head_stride % 8 || k_off % 8 || v_off % 8)
    return SV_EINVAL;
  if (half > 32 * FUSED_MAX_HS) return SV_ENOTSUP;
  AttnArgs a = {};
  a.proj = (const uint16_t*)proj;
  a.proj_stride = proj_stride;
  a.q_head_stride = q_head_stride;
  a.k_off = k_off;
  a.v_off = v_off;
  a.cs_stride = cs_stride;
  a.q_gamma = (const uint16_t*)q_gamma;
  a.k_gamma = (const uint16_t*)k_gamma;
  a.cosv = cos_in;
  a.sinv = sin_in;
  a.slots = slots;
  a.q_out = (uint16_t*)q_out;
  a.k_pool_w = (uint16_t*)k_pool;
  a.v_pool_w = (uint16_t*)v_pool;
  a.rot_half = (int)half;
  a.eps = eps;
  return paged_attention_impl(a, nullptr, k_pool, v_pool, out, table, lens, tree, batch, tokens,
                              num_heads, num_kv_heads, head_size, page_size, table_stride, scale,
                              scratch, scratch_bytes, stream);
}

// Extension, no counterpart in the reference: snowverify_paged_attention_qk that also writes
// the output projection's operand workspace (snowverify_gemm_kquant_a_prepared's ws for the
// [batch*tokens, num_heads*head_size] output, snowllm_gemm_kquant_a_ws_bytes of that shape), so
// the projection skips its own conversion of the bf16 output: the same operands, the same
// bits. head_size 256 only (hipErrorNotSupported otherwise).
SV_API int snowverify_paged_attention_qk_ws(
    const void* proj, int64_t proj_stride, int64_t q_head_stride, int64_t k_off, int64_t v_off,
    const void* q_gamma, const void* k_gamma, const float* cos_in, const float* sin_in,
    int64_t cs_stride, int64_t half, float eps, const int32_t* slots, void* q_out, void* k_pool,
    void* v_pool, void* out, const int32_t* table, const int32_t* lens, const uint64_t* tree,
    int64_t batch, int64_t tokens, int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
    int64_t page_size, int64_t table_stride, float scale, void* scratch, int64_t scratch_bytes,
    void* out_ws, void* stream) {
  if (!out_ws) return SV_EINVAL;
  if (!proj || !q_gamma || !k_gamma || !cos_in || !sin_in || !slots || half < 0 || half % 32 ||
      2 * half > head_size || proj_stride % 8 || q_head_stride % 8 || k_off % 8 || v_off % 8)
    return SV_EINVAL;
  if (half > 32 * FUSED_MAX_HS) return SV_ENOTSUP;
  AttnArgs a = {};
  a.proj = (const uint16_t*)proj;
  a.proj_stride = proj_stride;
  a.q_head_stride = q_head_stride;
  a.k_off = k_off;
  a.v_off = v_off;
  a.cs_stride = cs_stride;
  a.q_gamma = (const uint16_t*)q_gamma;
  a.k_gamma = (const uint16_t*)k_gamma;
  a.cosv = cos_in;
  a.sinv = sin_in;
  a.slots = slots;
  a.q_out = (uint16_t*)q_out;
  a.k_pool_w = (uint16_t*)k_pool;
  a.v_pool_w = (uint16_t*)v_pool;
  a.rot_half = (int)half;
  a.eps = eps;
  return paged_attention_impl(a, nullptr, k_pool, v_pool, out, table, lens, tree, batch, tokens,
                              num_heads, num_kv_heads, head_size, page_size, table_stride, scale,
                              scratch, scratch_bytes, stream, out_ws);
}

// Tuning knob (extension, no reference counterpart): pages per split of the attention's
// context split (0 restores the automatic choice). Returns the previous value.
SV_API int snowverify_attention_pages_per_split(int pages) {
  const int prev = g_pages_per_split;
  g_pages_per_split = pages < 0 ? 0 : pages;
  return prev;
}

// Tuning knob (extension, no reference counterpart): waves per row tile of the attention's
// split kernel (1 or 2; 3 = one or two per tile over eight waves; 0 restores the automatic
// choice). Returns the previous value.
SV_API int snowverify_attention_d_split(int dh) {
  const int prev = g_d_split;
  g_d_split = (dh == 1 || dh == 2 || dh == 3) ? dh : 0;
  return prev;
}

// Tuning knob (extension, no reference counterpart): row groups of the attention's split
// kernel in its one-wave-per-tile form (1, or 2: two workgroups per split, each with half of the
// row tiles; 0 restores the automatic choice). Returns the previous value.
SV_API int snowverify_attention_row_groups(int groups) {
  const int prev = g_row_groups;
  g_row_groups = (groups == 1 || groups == 2) ? groups : 0;
  return prev;
}

// Tuning knob (extension, no reference counterpart): pages in the attention's LDS ring, 4 or 8
// (0 restores the automatic choice). Returns the previous value.
SV_API int snowverify_attention_ring(int pages) {
  const int prev = g_ring;
  g_ring = (pages == 4 || pages == 8) ? pages : 0;
  return prev;
}

// ---------------------------------------------------------------------------------------
// The reference's split-KV decode entry points (snowllm/_capi.py:243, 358, 364-365, 371-373,
// 506-509, 808-812; ops/attention_full.py:516-518, 539-547, 565-575, 1147-1161, 1232-1238;
// ops/_common.py:35-43), over the active geometry. This build sizes its context splits at
// launch from the block-table width (one round of workgroups over the CUs) and every kernel
// reads the sequence lengths itself, so the decode plan the reference computes from the
// lengths carries nothing here: one int32 element, never written, and the plan call validates
// its arguments and launches nothing. A "slot" is the partials region of one sequence.
// ---------------------------------------------------------------------------------------
namespace {
int geo_group() {
  const BuildGeometry& g = active_geometry();
  return g.num_kv_heads > 0 && g.num_heads % g.num_kv_heads == 0
             ? (int)(g.num_heads / g.num_kv_heads) : 0;
}
}  // namespace

// Page sizes the KV pools support (snowllm/_capi.py:243; ops/_common.py:35-39): writes up to
// n of them to out (when out is not null) and returns how many there are.
SV_API int64_t snowllm_kv_block_sizes(int64_t* out, int64_t n) {
  if (out && n > 0) out[0] = PAGE;
  return 1;
}

// Largest query rows per request of the decode form (snowllm/_capi.py:371; read at import by
// ops/attention_full.py:565): T * G <= 128 rows in one workgroup, T <= 64 (u64 masks).
SV_API int64_t snowllm_paged_decode_max_q_tokens(void) {
  const int G = geo_group();
  if (G <= 0) return 0;
  const int t = MAX_TILES * 16 / G;
  return t < 64 ? t : 64;
}

// Partials regions for num_seqs sequences (snowllm/_capi.py:372).
SV_API int64_t snowllm_paged_decode_num_slots(int64_t num_seqs) {
  return num_seqs > 0 ? num_seqs : 0;
}

// Workspace bytes of snowllm_paged_attn_decode for num_slots sequences of q_tokens rows
// (snowllm/_capi.py:358).
SV_API int64_t snowllm_paged_decode_workspace_size(int64_t num_slots, int64_t q_tokens) {
  const BuildGeometry& g = active_geometry();
  if (num_slots <= 0 || q_tokens <= 0) return 0;
  return snowverify_paged_attention_scratch_bytes(num_slots, q_tokens, g.num_heads,
                                                  g.num_kv_heads, g.head_size);
}

// int32 elements of the decode plan (snowllm/_capi.py:373).
SV_API int64_t snowllm_paged_decode_plan_elems(int64_t num_seqs, int64_t num_slots) {
  (void)num_seqs;
  (void)num_slots;
  return 1;
}

// The decode plan (snowllm/_capi.py:509; ops/attention_full.py:1232-1238): nothing to compute
// (see above); the arguments are checked.
SV_API int snowllm_paged_attn_decode_plan(const int32_t* seq_lens, int32_t* plan,
                                          int64_t num_seqs, int64_t num_slots,
                                          int64_t block_size, int uniform, void* stream) {
  (void)plan;
  (void)uniform;
  (void)stream;
  if (!seq_lens || num_seqs <= 0 || num_slots < num_seqs) return SV_EINVAL;
  if (block_size != PAGE) return SV_ENOTSUP;
  return SV_OK;
}

// Split-KV decode attention (snowllm/_capi.py:506-508; ops/attention_full.py:1147-1161):
// q_tokens query rows per sequence, causal within them, against bf16 pools. q rows are q_pitch
// elements apart (0: num_heads * head_size) starting at row q_row0; out [num_seqs * q_tokens,
// num_heads, head_size] bf16; ws as sized by snowllm_paged_decode_workspace_size(num_slots,
// q_tokens) with num_slots >= num_seqs; block_tables [num_seqs, max_blocks].
SV_API int snowllm_paged_attn_decode(const void* q, const int32_t* seq_lens, const void* k_cache,
                                     const void* v_cache, void* out, const int32_t* block_tables,
                                     const int32_t* plan, int64_t num_seqs, int64_t max_blocks,
                                     int64_t num_slots, void* ws, float scale, int64_t q_tokens,
                                     int64_t block_size, int64_t q_pitch, int64_t q_row0,
                                     void* stream) {
  (void)plan;
  const BuildGeometry& g = active_geometry();
  if (!q || !seq_lens || !k_cache || !v_cache || !out || !block_tables || !ws ||
      num_seqs <= 0 || num_slots < num_seqs || q_tokens <= 0 || q_pitch < 0 || q_row0 < 0)
    return SV_EINVAL;
  if (q_pitch && q_pitch < g.num_heads * g.head_size) return SV_EINVAL;
  if (block_size != PAGE) return SV_ENOTSUP;
  AttnArgs a = {};
  a.q_stride = q_pitch ? q_pitch : g.num_heads * g.head_size;
  const uint16_t* q0 = (const uint16_t*)q + q_row0 * a.q_stride;
  return paged_attention_impl(a, q0, k_cache, v_cache, out, block_tables, seq_lens, nullptr,
                              num_seqs, q_tokens, g.num_heads, g.num_kv_heads, g.head_size,
                              block_size, max_blocks, scale, ws,
                              snowllm_paged_decode_workspace_size(num_slots, q_tokens), stream);
}

// Prepared attention metadata (snowllm/_capi.py:808-812; ops/attention_full.py:136-150): this
// build needs none, so its size is 0 and the reference's wrapper hands no prepared buffer on;
// the runner then skips the decode plan (engine/qwen_runner.py:202-208).
SV_API int64_t snowllm_paged_attention_prepared_bytes(int64_t batch, int64_t tokens,
                                                      int64_t slots, int varlen) {
  (void)batch;
  (void)tokens;
  (void)slots;
  (void)varlen;
  return 0;
}

SV_API int snowllm_paged_attention_prepare(const int32_t* lens, void* result, int64_t batch,
                                           int64_t tokens, int64_t slots, int64_t block_size,
                                           void* stream) {
  (void)result;
  (void)slots;
  (void)stream;
  if (!lens || batch <= 0 || tokens <= 0) return SV_EINVAL;
  if (block_size != PAGE) return SV_ENOTSUP;
  return SV_OK;
}

// Query-block map of a varlen batch (snowllm/_capi.py:364-365; ops/attention_full.py:539-547),
// host arithmetic over host arrays: blocks of 16 query rows; the map lists (sequence, first
// row of the block within the sequence) pairs in order.
SV_API int64_t snowllm_prefill_q_blocks(const int32_t* lens, int64_t B) {
  if (!lens || B < 0) return -1;
  int64_t total = 0;
  for (int64_t b = 0; b < B; ++b) total += lens[b] > 0 ? (lens[b] + 15) / 16 : 0;
  return total;
}

SV_API void snowllm_prefill_q_block_map(const int32_t* lens, int64_t B, int32_t* map) {
  if (!lens || !map || B < 0) return;
  int64_t i = 0;
  for (int64_t b = 0; b < B; ++b)
    for (int32_t r = 0; r < lens[b]; r += 16) {
      map[2 * i] = (int32_t)b;
      map[2 * i + 1] = r;
      ++i;
    }
}
