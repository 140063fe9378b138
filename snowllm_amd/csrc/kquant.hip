// GGUF Q4_K / Q8_0 dequant-GEMV for short verify blocks (M <= 16 rows per pass) on gfx950:
// repack, activation prep and the plain GEMV (shared device code in kquant_core.h).
//
// Weights stay packed in HBM. A one-time repack (snowllm_gemm_kquant_shuffle_b) moves the
// GGUF bytes into MFMA lane order: a 16-column tile of one 256-weight superblock is a single
// contiguous 2 KiB run of nibbles (Q4_K) or 4 KiB of int8 (Q8_0), read with 16-byte loads
// that are fully coalesced across the wave, plus 16 bytes of block header per column.
//
// Arithmetic (per 32-weight sub-block j, column n, row r):
//   y[r,n] = sum_j  a_j * sum_i q_i x_ri  - mn_j * sum_i x_ri
// Quants are turned into exact fp16 values with the 1024-offset trick (0x6400 | q == 1024+q;
// a high nibble left in bits 4..7 reads as 1024+16q), multiplied against fp16 activations on
// v_mfma_f32_16x16x32_f16 (K = 32 = one sub-block), and the sub-block result is scaled by
// a_j in fp32. The offset and min terms are one rank-8 product per superblock, done on
// v_mfma_f32_16x16x4_f32 with the sub-block sums of the activations. Activations are
// converted to fp16 once per call with a power-of-two scale per (row, superblock), exact for
// bf16 input.
#include "kquant_core.h"

#include <mutex>

namespace {
using namespace kq;

// ---------------------------------------------------------------------------------------
// Activation prep kernel: one wave per (row tile, superblock), writing the workspace.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) xprep_kernel(const uint16_t* __restrict__ a, int64_t M,
                                                   int64_t K, void* ws, size_t tile_bytes) {
  const int s = blockIdx.x, tile = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t S = K / QK;
  XPrepView v = xprep_view((char*)ws + tile * tile_bytes, S);
  const int64_t r0 = (int64_t)tile * TILE_M;
  XOperands o;
  convert_superblock(a + r0 * K, K, (int)(M - r0 < TILE_M ? M - r0 : TILE_M), s, lane, o);
  store_operands(v, s, lane, o);
}

// NW waves split the superblocks of NTILE column tiles; the waves' partial sums meet in LDS
// and are added in a fixed order. Reads past the end of a buffer return zero (buffer range
// checking), so the last partial tile group needs no clamping.
// RAW: ws is the bf16 activation matrix [M, S*256] itself, converted in-kernel (one launch
// for the whole operator instead of a prep pass + GEMV).
template <int FMT, int NTILE, int NW, bool RAW = false>
__global__ void __launch_bounds__(NW * 64) kquant_gemv(const u32x4* __restrict__ quant,
                                                       const u32x4* __restrict__ meta,
                                                       const void* __restrict__ ws,
                                                       void* __restrict__ c, int M, int N, int S,
                                                       int c_bf16) {
  __shared__ floatx4 part[NW][NTILE][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int kq = lane >> 4;
  const int tiles = N / TILE_N;
  const int tile0 = blockIdx.x * NTILE;
  const GemvStreams st = make_streams<FMT>(quant, meta, ws, tiles, S, lane, M);
  const uint32_t Mv = decode_magic<FMT>();
  floatx4 acc[NTILE];
#pragma unroll
  for (int t = 0; t < NTILE; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (RAW) {
    const RawX rx = make_raw_x(ws, M, S * QK, lane);
    gemv_loop_raw<FMT, NTILE, NW>(st, rx, w, S, tile0, 1, lane, Mv, acc);
  } else {
    gemv_loop<FMT, NTILE, NW>(st, w, S, tile0, 1, kq, Mv, acc);
  }
  combine_waves<NTILE, NW>(part, acc, w, lane);
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
      if (c_bf16) ((uint16_t*)c)[(int64_t)row * N + n] = f32_to_bf16(v[i]);
      else ((float*)c)[(int64_t)row * N + n] = v[i];
    }
  }
}

// ---------------------------------------------------------------------------------------
// Repack GGUF blocks into (quant, meta).
// ---------------------------------------------------------------------------------------
__global__ void shuffle_q4k(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const uint8_t* blk = gguf + (n * S + s) * 144;
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  uint8_t* mo = meta + (ts * 16 + col) * 16;
  for (int i = 0; i < 16; ++i) mo[i] = blk[i];
  const uint8_t* qs = blk + 16;
  for (int h = 0; h < 2; ++h)
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = col + 16 * kq;
      uint8_t* qo = quant + ((ts * 2 + h) * 64 + lane) * 16;
      for (int i = 0; i < 8; ++i) {
        qo[i] = qs[64 * h + 8 * kq + i];
        qo[8 + i] = qs[64 * h + 32 + 8 * kq + i];
      }
    }
}

__global__ void shuffle_q80(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ quant,
                            uint8_t* __restrict__ meta, int64_t N, int64_t S) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= N * S) return;
  const int64_t n = id / S, s = id % S;
  const int64_t tile = n / TILE_N;
  const int col = (int)(n % TILE_N);
  const int64_t ts = tile * S + s;
  for (int j = 0; j < 8; ++j) {
    const uint8_t* blk = gguf + ((n * S + s) * 8 + j) * 34;
    uint8_t* mo = meta + (ts * 16 + col) * 16 + 2 * j;
    mo[0] = blk[0];
    mo[1] = blk[1];
    const int jp = j >> 1, half = j & 1;
    for (int kq = 0; kq < 4; ++kq) {
      const int lane = col + 16 * kq;
      uint8_t* qo = quant + ((ts * 4 + jp) * 64 + lane) * 16 + 8 * half;
      for (int i = 0; i < 8; ++i) qo[i] = blk[2 + 8 * kq + i];
    }
  }
}

bool fmt_ok(int fmt) { return fmt == FMT_Q4_K || fmt == FMT_Q8_0; }

template <int FMT, int NTILE, int NW, bool RAW = false>
int launch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N, int S,
                int c_bf16, hipStream_t s) {
  const int tiles = N / TILE_N;
  const int grid = (tiles + NTILE - 1) / NTILE;
  hipLaunchKernelGGL((kquant_gemv<FMT, NTILE, NW, RAW>), dim3(grid), dim3(NW * 64), 0, s,
                     (const u32x4*)quant, (const u32x4*)meta, ws, c, M, N, S, c_bf16);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

int g_gemv_variant = 0;  // 0 = automatic; see snowverify_gemv_variant

template <int FMT, bool RAW = false>
int dispatch_gemv(const void* quant, const void* meta, const void* ws, void* c, int M, int N,
                  int S, int c_bf16, hipStream_t s) {
  switch (g_gemv_variant) {
    case 1: return launch_gemv<FMT, 1, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 2: return launch_gemv<FMT, 2, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 3: return launch_gemv<FMT, 4, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 4: return launch_gemv<FMT, 1, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 5: return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    case 6: return launch_gemv<FMT, 4, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    default: break;
  }
  const int tiles = N / TILE_N;
  // measured on MI355X (M = 9): wide outputs want 4 tiles x 8 waves, K >= 4096 narrow outputs
  // 1 x 8, K = 2048 2 x 8 when there are >= 2 tiles per CU, K = 4096 (prepared operands)
  // 2 x 8 from 3 tiles per CU (6144 x 4096: 9.7 -> 7.6 us)
  if (S >= 8) {
    // (Q8_0 keeps two tiles: four tiles of int8 quants exceed the register file)
    if (tiles >= 4 * 192 && FMT == FMT_Q4_K)
      return launch_gemv<FMT, 4, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    if (tiles >= 2 * 128 && S <= 8) return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    if (!RAW && FMT == FMT_Q4_K && tiles >= 3 * 128 && S <= 16)
      return launch_gemv<FMT, 2, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
    return launch_gemv<FMT, 1, 8, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
  }
  if (tiles >= 2 * 256) return launch_gemv<FMT, 2, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
  return launch_gemv<FMT, 1, 4, RAW>(quant, meta, ws, c, M, N, S, c_bf16, s);
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

SV_API int64_t snowllm_kquant_gguf_bytes(int fmt, int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  if (fmt == FMT_Q4_K) return K % 256 ? -1 : N * (K / 256) * 144;
  if (fmt == FMT_Q8_0) return K % 32 ? -1 : N * (K / 32) * 34;
  return -1;
}

SV_API int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  return (fmt == FMT_Q4_K ? N * K / 2 : N * K) + 4;
}

SV_API int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K) {
  if (!fmt_ok(fmt) || N < 0 || K % 256 || N % TILE_N) return -1;
  return N * (K / 256) * 16;
}

SV_API int snowllm_kquant_supported(int fmt) { return fmt_ok(fmt) ? 1 : 0; }

// Extension (tuning knob, no counterpart in the reference): force a GEMV tile shape
// (0 = automatic, 1..6 = fixed (tiles per workgroup, waves) pairs). Process-global.
SV_API void snowverify_gemv_variant(int v) { g_gemv_variant = v; }

SV_API int snowllm_gemm_kquant_shuffle_b(int fmt, const uint8_t* gguf, uint8_t* quant,
                                         uint8_t* meta, int64_t N, int64_t K, void* stream) {
  if (!fmt_ok(fmt) || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  const int64_t S = K / 256;
  const int64_t total = N * S;
  const int nt = 256;
  hipStream_t s = (hipStream_t)stream;
  if (fmt == FMT_Q4_K)
    hipLaunchKernelGGL(shuffle_q4k, dim3((unsigned)((total + nt - 1) / nt)), dim3(nt), 0, s, gguf,
                       quant, meta, N, S);
  else
    hipLaunchKernelGGL(shuffle_q80, dim3((unsigned)((total + nt - 1) / nt)), dim3(nt), 0, s, gguf,
                       quant, meta, N, S);
  SV_CHECK_LAUNCH();
  return SV_OK;
}

SV_API int64_t snowllm_gemm_kquant_a_ws_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 256) return 0;
  const int64_t tiles = (M + TILE_M - 1) / TILE_M;
  return (int64_t)(tiles * xprep_tile_bytes(K / 256));
}

// Extension (no counterpart in the reference): convert activations once into the operand
// workspace so several weights that share an input (gate/up, Q/K/V) reuse it.
SV_API int snowverify_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws,
                                         void* stream) {
  if (M < 0 || K <= 0 || K % 256) return SV_EINVAL;
  if (M == 0) return SV_OK;
  const int64_t S = K / 256;
  const int64_t mt = (M + TILE_M - 1) / TILE_M;
  hipLaunchKernelGGL(xprep_kernel, dim3((unsigned)S, (unsigned)mt), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)a, M, K, ws, xprep_tile_bytes(S));
  SV_CHECK_LAUNCH();
  return SV_OK;
}

// Extension (no counterpart in the reference): the GEMV on a prepared operand workspace.
SV_API int snowverify_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta,
                                          void* c, int64_t M, int64_t N, int64_t K,
                                          int c_is_bf16, const void* ws, void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (M == 0) return SV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t S = K / 256;
  const size_t tb = xprep_tile_bytes(S);
  const int64_t mt = (M + TILE_M - 1) / TILE_M;
  const size_t esz = c_is_bf16 ? 2 : 4;
  for (int64_t t = 0; t < mt; ++t) {
    const int rows = (int)((M - t * TILE_M) < TILE_M ? (M - t * TILE_M) : TILE_M);
    void* ct = (char*)c + (size_t)t * TILE_M * N * esz;
    const void* wst = (const char*)ws + t * tb;
    int rc = fmt == FMT_Q4_K
                 ? dispatch_gemv<FMT_Q4_K>(quant, meta, wst, ct, rows, (int)N, (int)S, c_is_bf16, s)
                 : dispatch_gemv<FMT_Q8_0>(quant, meta, wst, ct, rows, (int)N, (int)S, c_is_bf16, s);
    if (rc) return rc;
  }
  return SV_OK;
}

SV_API int snowllm_gemm_kquant_a(int fmt, const void* a, const uint8_t* quant, const uint8_t* meta,
                                 void* c, int64_t M, int64_t N, int64_t K, int c_is_bf16, void* ws,
                                 void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (M == 0) return SV_OK;
  if (M <= TILE_M && M * K * 2 <= INT32_MAX) {
    // one launch: the GEMV converts the bf16 activations itself (same operands as the
    // prepared path, so the same results); ws is not touched
    hipStream_t s = (hipStream_t)stream;
    return fmt == FMT_Q4_K
               ? dispatch_gemv<FMT_Q4_K, true>(quant, meta, a, c, (int)M, (int)N, (int)(K / 256), c_is_bf16, s)
               : dispatch_gemv<FMT_Q8_0, true>(quant, meta, a, c, (int)M, (int)N, (int)(K / 256), c_is_bf16, s);
  }
  int rc = snowverify_gemm_kquant_prepare_a(a, M, K, ws, stream);
  if (rc) return rc;
  return snowverify_gemm_kquant_a_prepared(fmt, quant, meta, c, M, N, K, c_is_bf16, ws, stream);
}

// ---------------------------------------------------------------------------------------
// The no-allocation form of snowllm_gemm_kquant_a, for callers that cannot allocate (code
// under HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc). Up to 16
// rows the GEMV converts the activations itself and needs no workspace; above that the
// operand workspace lives in `scratch`, a file-scope device array of a fixed size -- each GPU
// the library runs on holds its own copy until the process ends. Host code never passes the
// array's name to a kernel: its device address is read once per device with
// hipGetSymbolAddress, with that device current, and kept.
// ---------------------------------------------------------------------------------------
namespace {
constexpr int64_t NOALLOC_MAX_M = 64, NOALLOC_MAX_K = 16384;
constexpr size_t NOALLOC_WS_BYTES = 2244608;  // snowllm_gemm_kquant_a_ws_bytes(64, 16384)
static __device__ __align__(256) uint8_t scratch[NOALLOC_WS_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];

// The current device's address of `scratch`.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return SV_ENOTSUP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return SV_EINVAL;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SV_OK;
}
}  // namespace

SV_API int snowverify_gemm_kquant_a_noalloc(int fmt, const void* a, const uint8_t* quant,
                                            const uint8_t* meta, void* c, int64_t M, int64_t N,
                                            int64_t K, int c_is_bf16, void* stream) {
  if (!fmt_ok(fmt) || M < 0 || N <= 0 || K <= 0 || K % 256 || N % TILE_N) return SV_EINVAL;
  if (M > NOALLOC_MAX_M || K > NOALLOC_MAX_K) return SV_EINVAL;  // beyond the array
  if (M == 0) return SV_OK;
  if (M <= TILE_M)  // the one-launch form: no workspace
    return snowllm_gemm_kquant_a(fmt, a, quant, meta, c, M, N, K, c_is_bf16, nullptr, stream);
  if ((size_t)snowllm_gemm_kquant_a_ws_bytes(M, K) > NOALLOC_WS_BYTES) return SV_EINVAL;
  void* ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc) return rc;
  // the prep pass writes every byte of the workspace the GEMV reads (padding rows included),
  // so nothing needs clearing between calls
  rc = snowverify_gemm_kquant_prepare_a(a, M, K, ws, stream);
  if (rc) return rc;
  return snowverify_gemm_kquant_a_prepared(fmt, quant, meta, c, M, N, K, c_is_bf16, ws, stream);
}
