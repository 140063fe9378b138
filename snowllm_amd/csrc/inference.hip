// The reference's geometry-driven operator entry points for the verify path, composed from this
// library's kernels: fused-norm QKV projection, attention output projection, paged attention
// through its step descriptor, the MoE block (with and without the fused post-attention norm),
// the dense MLP and the LM head (snowllm/_capi.py:218-225, 251, 315, 355, 599, 687-692, 805-807;
// wrappers snowllm/ops/inference.py:10-104, snowllm/ops/attention_full.py:54-177).
//
// Shapes come from the active geometry, as in the reference. Weights arrive in the reference's
// _Weight descriptor (snowllm/ops/inference.py:10-22), holding this library's repacked layouts:
// k-quant matrices as (quant, meta) from snowllm_gemm_kquant_shuffle_b (kind 2, or kind 3 for an
// expert stack: the experts' packed matrices back to back), 16-bit dense matrices (router, LM
// head) as repacked by snowverify_dense_shuffle (kind 0). Features of the reference that the
// verify path of this build does not carry -- int8 KV, gated attention output, split Q/KV
// weights, fp8 dense scales, the DSA indexer, hashed routing, varlen prefill -- return
// hipErrorNotSupported instead of computing something else.
//
// Workspaces are carved from the caller's scratch with 256-byte alignment; the *_bytes queries
// return the totals. No entry point allocates or synchronises.
#include "common.h"
#include "geometry.h"

#include <string.h>

namespace {

struct Weight {  // snowllm/ops/inference.py:10-12
  void* data[3];
  void* scale;
  int kind;  // -1 absent, 0 dense, 1 dense + scale, 2 k-quant, 3 k-quant expert stack
  int fmt;
};

struct PagedAttentionStep {  // snowllm/ops/attention_full.py:120-123
  void* inputs[10];  // q, k_pool, v_pool, k_scale, v_scale, cu_seqlens, table, lens, qmap, gate
  void* outputs[3];  // out, plan, workspace
  int64_t batch, pages, q_blocks, slots, tokens, page_size, gate_stride, gate_row0;
  float scale;
  int varlen;  // bit 0: varlen, bit 1: host lengths, bit 2: prepared metadata
};

constexpr int WT_F16 = 1, WT_BF16 = 2;  // snowverify_dense_gemv weight types
constexpr int MAX_ROWS = 16;            // rows per dense-MLP call (one 16-row tile)
constexpr int MOE_ROWS = 64;            // rows per MoE call (the plan's limit)

inline size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

bool kquant(const Weight* w) { return w && (w->kind == 2 || w->kind == 3) && w->data[0] && w->data[1]; }
bool absent(const Weight* w) { return !w || w->kind < 0; }

// Carves consecutive 256-byte aligned regions out of a scratch buffer.
struct Carve {
  char* p;
  size_t used = 0;
  explicit Carve(void* base) : p((char*)base) {}
  void* take(size_t n) {
    void* r = p ? p + used : nullptr;
    used += a256(n);
    return r;
  }
};

}  // namespace

extern "C" {
int64_t snowllm_gemm_kquant_a_ws_bytes(int64_t M, int64_t K);
int snowllm_gemm_kquant_a(int fmt, const void* a, const uint8_t* quant, const uint8_t* meta,
                          void* c, int64_t M, int64_t N, int64_t K, int c_is_bf16, void* ws,
                          void* stream);
int snowverify_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws, void* stream);
int snowverify_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta, void* c,
                                   int64_t M, int64_t N, int64_t K, int c_is_bf16,
                                   const void* ws, void* stream);
int snowverify_gemm_kquant_a_prepared_ld(int fmt, const uint8_t* quant, const uint8_t* meta,
                                         void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                         int c_is_bf16, const void* ws, void* stream);
int snowverify_norm_prep(const void* x, const void* res_in, void* res_out, const void* gamma,
                         void* y_out, void* ws, int64_t M, int64_t H, float eps, void* stream);
int snowverify_dense_gemv(int wt, const void* w, const void* act, void* c, int64_t M, int64_t N,
                          int64_t K, int c_is_bf16, void* stream);
int snowverify_gate_up_swiglu(int fmt, const void* quant, const void* meta, const void* ws,
                              void* act, int64_t M, int64_t F, int64_t K, void* stream);
int64_t snowverify_moe_plan_bytes(void);
int64_t snowverify_moe_max_slots(int64_t M, int64_t topk, int64_t E, int shared);
int snowverify_moe_route_plan(const float* logits, int64_t stride, int64_t M, int64_t E,
                              int64_t topk, float* weights, int32_t* ids, float* shared_w,
                              void* plan, void* stream);
int snowverify_moe_gate_up_down(int fmt, const void* gu_quant, const void* gu_meta,
                                const void* dn_quant, const void* dn_meta,
                                const void* sh_gu_quant, const void* sh_gu_meta,
                                const void* sh_dn_quant, const void* sh_dn_meta, const void* plan,
                                const void* ws, const float* weights, const float* shared_w,
                                void* act, float* pairs, float* shared_out, int64_t M,
                                int64_t max_slots, int64_t E, int64_t H, int64_t F, void* stream);
int snowverify_moe_gate_up(int fmt, const void* gu_quant, const void* gu_meta,
                           const void* sh_gu_quant, const void* sh_gu_meta, const void* plan,
                           const void* ws, void* act, int64_t M, int64_t max_slots, int64_t E,
                           int64_t H, int64_t F, void* stream);
int snowverify_moe_down(int fmt, const void* dn_quant, const void* dn_meta,
                        const void* sh_dn_quant, const void* sh_dn_meta, const void* plan,
                        const void* act, const float* weights, const float* shared_w,
                        float* pairs, float* shared_out, int64_t max_slots, int64_t E, int64_t H,
                        int64_t F, void* stream);
int snowverify_moe_combine(const float* pairs, const float* shared_out, void* out, int64_t M,
                           int64_t topk, int64_t H, void* stream);
int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K);
int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K);
int64_t snowllm_kquant_gguf_bytes(int fmt, int64_t N, int64_t K);
int snowllm_gemm_kquant_shuffle_b(int fmt, const uint8_t* gguf, uint8_t* quant, uint8_t* meta,
                                  int64_t N, int64_t K, void* stream);
int64_t snowverify_dense_bytes(int64_t N, int64_t K);
int snowverify_dense_shuffle(const void* src, void* dst, int64_t N, int64_t K, int wt,
                             void* stream);
int64_t snowverify_paged_attention_scratch_bytes(int64_t batch, int64_t tokens,
                                                 int64_t num_heads, int64_t num_kv_heads,
                                                 int64_t head_size);
int snowverify_paged_attention(const void* q, const void* k_pool, const void* v_pool, void* out,
                               const int32_t* table, const int32_t* lens, const uint64_t* tree,
                               int64_t batch, int64_t tokens, int64_t num_heads,
                               int64_t num_kv_heads, int64_t head_size, int64_t page_size,
                               int64_t table_stride, float scale, void* scratch,
                               int64_t scratch_bytes, void* stream);
}

namespace {

// ---- MoE workspace: operands | logits | routing | plan | activations | pairs | shared rows --
struct MoeWs {
  void* ws;
  float* logits;
  float* weights;
  int32_t* ids;
  float* shared_w;
  void* plan;
  void* act;
  float* pairs;
  float* shared_out;
  size_t bytes;
};

MoeWs moe_ws(void* base, int64_t M) {
  const BuildGeometry& g = active_geometry();
  const int64_t E = g.moe_num_experts, K = g.moe_topk, H = g.hidden, F = g.moe_inter;
  Carve c(base);
  MoeWs w;
  w.ws = c.take((size_t)snowllm_gemm_kquant_a_ws_bytes(M, H));
  w.logits = (float*)c.take((size_t)M * (E + 1) * 4);
  w.weights = (float*)c.take((size_t)M * K * 4);
  w.ids = (int32_t*)c.take((size_t)M * K * 4);
  w.shared_w = (float*)c.take((size_t)M * 4);
  w.plan = c.take((size_t)snowverify_moe_plan_bytes());
  // activation scratch for every slot the plan can take (16 compact rows each)
  w.act = c.take((size_t)snowverify_moe_max_slots(M, K, E, 1) * 16 * F * 2);
  w.pairs = (float*)c.take((size_t)M * K * H * 4);
  w.shared_out = (float*)c.take((size_t)M * H * 4);
  w.bytes = c.used;
  return w;
}

bool moe_geometry_ok() {
  const BuildGeometry& g = active_geometry();
  return g.moe_num_experts > 0 && g.moe_topk > 0 && g.moe_inter > 0;
}

// Router GEMV, routing + plan, experts, combine: out = sum_k w_k expert_k(y) + sigmoid(g) shared(y)
// for the normalised rows y (bf16 `hidden`, operands already in ws.ws).
int moe_body(const Weight* w, const void* hidden, const void* router, void* out, const MoeWs& ws,
             int64_t M, void* s) {
  const BuildGeometry& g = active_geometry();
  const int64_t E = g.moe_num_experts, K = g.moe_topk, H = g.hidden, F = g.moe_inter;
  const bool shared = !absent(&w[2]);
  // experts: gate/up in Q4_K, Q5_K or Q6_K, down in the same or a wider k-quant; the shared
  // expert in the routed experts' formats
  auto efmt = [](int f) { return f == 4 || f == 5 || f == 6; };
  if (!kquant(&w[0]) || !kquant(&w[1]) || !efmt(w[0].fmt) || !efmt(w[1].fmt)) return SV_ENOTSUP;
  if (shared && (!kquant(&w[2]) || !kquant(&w[3]) || w[2].fmt != w[0].fmt ||
                 w[3].fmt != w[1].fmt))
    return SV_ENOTSUP;
  if (shared != (g.moe_shared_expert != 0)) return SV_EINVAL;
  int rc = snowverify_dense_gemv(WT_BF16, router, hidden, ws.logits, M, E + 1, H, 0, s);
  if (rc) return rc;
  rc = snowverify_moe_route_plan(ws.logits, E + 1, M, E, K, ws.weights, ws.ids,
                                 shared ? ws.shared_w : nullptr, ws.plan, s);
  if (rc) return rc;
  const int64_t slots = snowverify_moe_max_slots(M, K, E, shared);
  rc = snowverify_moe_gate_up_down(w[0].fmt | (w[1].fmt << 8), w[0].data[0], w[0].data[1],
                                   w[1].data[0], w[1].data[1],
                                   shared ? w[2].data[0] : nullptr,
                                   shared ? w[2].data[1] : nullptr,
                                   shared ? w[3].data[0] : nullptr,
                                   shared ? w[3].data[1] : nullptr, ws.plan, ws.ws, ws.weights,
                                   ws.shared_w, ws.act, ws.pairs, ws.shared_out, M, slots, E, H,
                                   F, s);
  if (rc) return rc;
  return snowverify_moe_combine(ws.pairs, shared ? ws.shared_out : nullptr, out, M, K, H, s);
}

// ---- dense MLP workspace: x operands | activations | activation operands -----------------
struct MlpWs {
  void* ws_x;
  void* act;
  void* ws_act;
  size_t bytes;
};

MlpWs mlp_ws(void* base, int64_t M) {
  const BuildGeometry& g = active_geometry();
  Carve c(base);
  MlpWs w;
  w.ws_x = c.take((size_t)snowllm_gemm_kquant_a_ws_bytes(M, g.hidden));
  w.act = c.take((size_t)M * g.mlp_inter * 2);
  w.ws_act = c.take((size_t)snowllm_gemm_kquant_a_ws_bytes(M, g.mlp_inter));
  w.bytes = c.used;
  return w;
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

// snowllm/_capi.py:251 -- scratch of snowllm_inference_qkv: the operand workspace of M rows.
SV_API int64_t snowllm_qkv_proj_scratch_bytes(int64_t M) {
  return M <= 0 ? 0 : snowllm_gemm_kquant_a_ws_bytes(M, active_geometry().hidden);
}

// snowllm/_capi.py:688 (ops/inference.py:34-43; QKVProj, models/qwen3_5/layers.py:33-50):
// out [M, qkv_proj_n] bf16 = y W^T with y = RMSNorm(residual += x) * gamma when gamma is given
// (y = RMSNorm(x) * gamma without a residual; y = x without gamma). w[0]: the QKV k-quant
// weight, or with w[1] present the Q|K rows [qkv_off_v, hidden] and w[1] the V rows
// [kv heads * head size, hidden] in their own format (the split of
// models/qwen3_5/qwen3_5_weights.py:95-109: GGUF files keep attn_v wider than attn_q/attn_k);
// w[2] (a bf16 KV) and the indexer are not carried (hipErrorNotSupported).
SV_API int snowllm_inference_qkv(const Weight* w, const void* x, void* residual,
                                 const void* gamma, float eps, void* scratch, void* out,
                                 int64_t M, int path, const void* index_w, void* index_out,
                                 void* stream) {
  (void)path;  // the reference's execution-path hint; one path here
  const BuildGeometry& g = active_geometry();
  if (!w || !kquant(&w[0]) || !absent(&w[2]) || index_w || index_out) return SV_ENOTSUP;
  const bool split = !absent(&w[1]);
  if (split && (!kquant(&w[1]) || g.qkv_off_v + g.num_kv_heads * g.head_size != g.qkv_proj_n))
    return SV_ENOTSUP;
  if (M <= 0 || !x || !out || !scratch) return SV_EINVAL;
  const auto* q = (const uint8_t*)w[0].data[0];
  const auto* m = (const uint8_t*)w[0].data[1];
  if (!split) {
    if (!gamma)
      return snowllm_gemm_kquant_a(w[0].fmt, x, q, m, out, M, g.qkv_proj_n, g.hidden, 1,
                                   scratch, stream);
    int rc = snowverify_norm_prep(x, residual, residual, gamma, nullptr, scratch, M, g.hidden,
                                  eps, stream);
    if (rc) return rc;
    return snowverify_gemm_kquant_a_prepared(w[0].fmt, q, m, out, M, g.qkv_proj_n, g.hidden, 1,
                                          scratch, stream);
  }
  // split: the operands once, then Q|K and V into their columns of out
  int rc = gamma ? snowverify_norm_prep(x, residual, residual, gamma, nullptr, scratch, M,
                                        g.hidden, eps, stream)
                 : snowverify_gemm_kquant_prepare_a(x, M, g.hidden, scratch, stream);
  if (rc) return rc;
  rc = snowverify_gemm_kquant_a_prepared_ld(w[0].fmt, q, m, out, g.qkv_proj_n, M, g.qkv_off_v,
                                            g.hidden, 1, scratch, stream);
  if (rc) return rc;
  return snowverify_gemm_kquant_a_prepared_ld(
      w[1].fmt, (const uint8_t*)w[1].data[0], (const uint8_t*)w[1].data[1],
      (uint16_t*)out + g.qkv_off_v, g.qkv_proj_n, M, g.qkv_proj_n - g.qkv_off_v, g.hidden, 1,
      scratch, stream);
}

// snowllm/_capi.py:254 (bound at import by ops/attention_full.py:512): scratch of the output
// projection of `rows` rows, the projection's operand workspace (as snowllm_attn_output_plan).
SV_API int64_t snowllm_attn_out_scale_oproj_scratch_bytes(int64_t rows) {
  const BuildGeometry& g = active_geometry();
  return rows <= 0 ? 0 : snowllm_gemm_kquant_a_ws_bytes(rows, g.num_heads * g.head_size);
}

// snowllm/_capi.py:300-301 (bound at import by ops/dflash.py:337-338): the draft model's
// attention sizing. The draft model's own layers are not carried here; these answer with the
// decode attention's sizing for the active geometry (one partials region per sequence).
SV_API int64_t snowllm_draft_paged_attn_num_slots(int64_t num_seqs) {
  return num_seqs > 0 ? num_seqs : 0;
}

SV_API int64_t snowllm_draft_paged_attn_workspace_size(int64_t num_slots, int64_t q_tokens) {
  const BuildGeometry& g = active_geometry();
  if (num_slots <= 0 || q_tokens <= 0) return 0;
  return snowverify_paged_attention_scratch_bytes(num_slots, q_tokens, g.num_heads,
                                                  g.num_kv_heads, g.head_size);
}

// snowllm/_capi.py:351 (bound at import by ops/moe.py:279): scratch of the hashed
// (token-id -> expert) router, which this build does not carry (its MoE entry points refuse a
// tid2eid table): 0.
SV_API int64_t snowllm_moe_router_shuffle_bytes(int64_t rows) {
  (void)rows;
  return 0;
}

// snowllm/_capi.py:223 (ops/attention_full.py:54-64): elements of the attention output and the
// scratch bytes of snowllm_attn_output_project for m rows.
SV_API int snowllm_attn_output_plan(int64_t m, int prefill, int kv_int8, int64_t* out) {
  (void)prefill;
  if (kv_int8) return SV_ENOTSUP;
  if (m < 0 || !out) return SV_EINVAL;
  const BuildGeometry& g = active_geometry();
  out[0] = m * g.num_heads * g.head_size;
  out[1] = m > 16 ? snowllm_gemm_kquant_a_ws_bytes(m, g.num_heads * g.head_size) : 0;
  return SV_OK;
}

// snowllm/_capi.py:224 (ops/attention_full.py:67-70): the attention output gate inside the
// projection rows. The geometries of this build carry no output gate.
SV_API void* snowllm_attn_output_gate(const void* proj, int prefill, int kv_int8) {
  (void)proj;
  (void)prefill;
  (void)kv_int8;
  return nullptr;
}

// snowllm/_capi.py:225 (ops/attention_full.py:98-117; OProj, models/qwen3_5/layers.py:53-64):
// out [m, hidden] bf16 = a [m, heads * head_size] Wo^T with the k-quant (quant, meta) weight.
SV_API int snowllm_attn_output_project(const void* a, const void* proj, int64_t proj_stride,
                                       const void* dense, const void* quant, const void* meta,
                                       const void* scale, int fmt, void* scratch, void* out,
                                       int64_t m, int prefill, int kv_int8, void* stream) {
  (void)proj;
  (void)proj_stride;
  (void)prefill;
  if (dense || scale || kv_int8 || active_geometry().qkv_off_scale) return SV_ENOTSUP;
  if (!quant || !meta || !a || !out || m < 0) return SV_EINVAL;
  if (m == 0) return SV_OK;
  const BuildGeometry& g = active_geometry();
  return snowllm_gemm_kquant_a(fmt, a, (const uint8_t*)quant, (const uint8_t*)meta, out, m,
                               g.hidden, g.num_heads * g.head_size, 1, scratch, stream);
}

// snowllm/_capi.py:218-219 (ops/attention_full.py:126-134).
SV_API int64_t snowllm_paged_attention_scratch_bytes(int64_t batch, int64_t tokens, int varlen) {
  if (varlen || batch <= 0 || tokens <= 0) return 0;
  const BuildGeometry& g = active_geometry();
  return snowverify_paged_attention_scratch_bytes(batch, tokens, g.num_heads, g.num_kv_heads,
                                                  g.head_size);
}

// Whether a step runs the varlen (prefill) form. Decode and verify steps -- equal token counts
// per request -- do not; prefill, which this build does not carry, would.
SV_API int snowllm_paged_attention_varlen(int prefill, int64_t tokens, int chunk_decode) {
  (void)tokens;
  (void)chunk_decode;
  return prefill ? 1 : 0;
}

// snowllm/_capi.py:220 (ops/attention_full.py:152-177): the step descriptor's decode/verify
// form -- `tokens` query rows per request, causal within the block, bf16 pools, no gate.
SV_API int snowllm_paged_attention(const PagedAttentionStep* st, void* scratch, int64_t bytes,
                                   void* stream) {
  if (!st) return SV_EINVAL;
  if ((st->varlen & 5) || st->inputs[3] || st->inputs[4] || st->inputs[9]) return SV_ENOTSUP;
  const BuildGeometry& g = active_geometry();
  return snowverify_paged_attention(st->inputs[0], st->inputs[1], st->inputs[2], st->outputs[0],
                                    (const int32_t*)st->inputs[6], (const int32_t*)st->inputs[7],
                                    nullptr, st->batch, st->tokens, g.num_heads, g.num_kv_heads,
                                    g.head_size, st->page_size, st->pages, st->scale, scratch,
                                    bytes, stream);
}

// ---- expert and router repack (snowllm/_capi.py:313-314, 326-331; ops/moe.py:81-86, 136-162)
// The GGUF expert stacks (ffn_gate_exps / ffn_up_exps [E, F, H], ffn_down_exps [E, H, F],
// each expert's rows back to back) become the layout the MoE kernels read: per expert e the
// packed [2F, H] gate/up matrix (gate rows first) at e * its bytes, and the packed [H, F]
// down matrix; each packed matrix is snowllm_gemm_kquant_shuffle_b's (quant, meta), whose
// 16-row tiles are stored in order, so the gate half and the up half are packed separately
// into the two halves. The +4 bytes of the single-matrix quant size come once, at the end.
extern "C" int snowverify_kquant_shuffle_split(int fmt, const uint8_t* top, const uint8_t* bottom,
                                               int64_t n_top, uint8_t* quant, uint8_t* meta,
                                               int64_t N, int64_t K, void* stream);
namespace {
int64_t expert_quant(int fmt, int64_t N, int64_t K) {
  const int64_t q = snowllm_kquant_quant_bytes(fmt, N, K);
  return q < 0 ? -1 : q - 4;
}
bool expert_geometry(int fmt, int64_t E) {
  const BuildGeometry& g = active_geometry();
  return (fmt == 4 || fmt == 5 || fmt == 6 || fmt == 8) && E > 0 && g.moe_inter > 0 && g.hidden > 0 &&
         expert_quant(fmt, g.moe_inter, g.hidden) > 0 && expert_quant(fmt, g.hidden, g.moe_inter) > 0;
}
}  // namespace

SV_API int64_t snowllm_moe_kquant_gate_up_quant_bytes(int fmt, int64_t E) {
  if (!expert_geometry(fmt, E)) return 0;
  const BuildGeometry& g = active_geometry();
  return E * 2 * expert_quant(fmt, g.moe_inter, g.hidden) + 4;
}
SV_API int64_t snowllm_moe_kquant_gate_up_meta_bytes(int fmt, int64_t E) {
  if (!expert_geometry(fmt, E)) return 0;
  const BuildGeometry& g = active_geometry();
  return E * 2 * snowllm_kquant_meta_bytes(fmt, g.moe_inter, g.hidden);
}
SV_API int64_t snowllm_moe_kquant_down_quant_bytes(int fmt, int64_t E) {
  if (!expert_geometry(fmt, E)) return 0;
  const BuildGeometry& g = active_geometry();
  return E * expert_quant(fmt, g.hidden, g.moe_inter) + 4;
}
SV_API int64_t snowllm_moe_kquant_down_meta_bytes(int fmt, int64_t E) {
  if (!expert_geometry(fmt, E)) return 0;
  const BuildGeometry& g = active_geometry();
  return E * snowllm_kquant_meta_bytes(fmt, g.hidden, g.moe_inter);
}

SV_API int snowllm_moe_kquant_shuffle_gate_up(int fmt, const uint8_t* gate, const uint8_t* up,
                                              uint8_t* quant, uint8_t* meta, int64_t E,
                                              void* stream) {
  if (!expert_geometry(fmt, E) || !gate || !up || !quant || !meta) return SV_EINVAL;
  const BuildGeometry& g = active_geometry();
  const int64_t F = g.moe_inter, H = g.hidden;
  const int64_t src = snowllm_kquant_gguf_bytes(fmt, F, H);
  const int64_t q = expert_quant(fmt, 2 * F, H), m = snowllm_kquant_meta_bytes(fmt, 2 * F, H);
  // each expert's [gate; up] as one [2F, H] matrix (gate rows first), read from its two
  // sources; for formats without a per-matrix tail this is the two halves packed one after
  // the other
  for (int64_t e = 0; e < E; ++e) {
    const int rc = snowverify_kquant_shuffle_split(fmt, gate + e * src, up + e * src, F,
                                                   quant + e * q, meta + e * m, 2 * F, H, stream);
    if (rc) return rc;
  }
  return SV_OK;
}

SV_API int snowllm_moe_kquant_shuffle_down(int fmt, const uint8_t* down, uint8_t* quant,
                                           uint8_t* meta, int64_t E, void* stream) {
  if (!expert_geometry(fmt, E) || !down || !quant || !meta) return SV_EINVAL;
  const BuildGeometry& g = active_geometry();
  const int64_t F = g.moe_inter, H = g.hidden;
  const int64_t src = snowllm_kquant_gguf_bytes(fmt, H, F);
  const int64_t q = expert_quant(fmt, H, F), m = snowllm_kquant_meta_bytes(fmt, H, F);
  for (int64_t e = 0; e < E; ++e) {
    const int rc = snowllm_gemm_kquant_shuffle_b(fmt, down + e * src, quant + e * q, meta + e * m,
                                                 H, F, stream);
    if (rc) return rc;
  }
  return SV_OK;
}

// The bf16 router [E + 1, hidden] (the routed experts' rows, then the shared expert's gate row,
// snowllm/models/qwen3_5/qwen3_5_weights.py:333-335) repacked for the router GEMV. A router
// bias is not carried (hipErrorNotSupported).
SV_API int64_t snowllm_moe_shuffle_router_bytes(void) {
  const BuildGeometry& g = active_geometry();
  if (!moe_geometry_ok()) return 0;
  return snowverify_dense_bytes(g.moe_num_experts + 1, g.hidden);
}

SV_API int snowllm_moe_shuffle_router(const void* router, const void* bias, void* out,
                                      void* stream) {
  if (bias) return SV_ENOTSUP;
  if (!router || !out || !moe_geometry_ok()) return SV_EINVAL;
  const BuildGeometry& g = active_geometry();
  return snowverify_dense_shuffle(router, out, g.moe_num_experts + 1, g.hidden, WT_BF16, stream);
}

// snowllm/_capi.py:315 and 690 -- scratch of the MoE block for `rows` rows (flags must be 0).
SV_API int64_t snowllm_moe_workspace_bytes(int64_t rows) {
  if (rows <= 0 || rows > MOE_ROWS || !moe_geometry_ok()) return 0;
  return (int64_t)moe_ws(nullptr, rows).bytes;
}

SV_API int64_t snowllm_inference_moe_workspace_bytes(int64_t rows, int64_t flags) {
  return flags ? 0 : snowllm_moe_workspace_bytes(rows);
}

// snowllm/_capi.py:691 (ops/inference.py:60-76): out [M, hidden] = MoE(x) for normalised x.
// w: experts' gate/up stack, experts' down stack, shared gate/up, shared down (absent when the
// geometry has no shared expert); router: the repacked bf16 [E + 1, hidden] router with the
// shared expert's gate last. x and out may be the same buffer. M <= 64.
SV_API int snowllm_inference_moe(const Weight* w, const void* x, const void* router,
                                 const int64_t* token_ids, const int32_t* tid2eid, void* out,
                                 void* scratch, int64_t capacity, int64_t M, int64_t flags,
                                 void* stream) {
  if (token_ids || tid2eid || flags) return SV_ENOTSUP;
  if (!w || !x || !router || !out || !scratch || M <= 0 || M > MOE_ROWS || !moe_geometry_ok())
    return SV_EINVAL;
  const MoeWs ws = moe_ws(scratch, M);
  if (capacity < (int64_t)ws.bytes) return SV_EINVAL;
  int rc = snowverify_gemm_kquant_prepare_a(x, M, active_geometry().hidden, ws.ws, stream);
  if (rc) return rc;
  return moe_body(w, x, router, out, ws, M, stream);
}

// snowllm/_capi.py:805-807 (ops/inference.py:82-95; FusedMoE with the post-attention norm,
// models/qwen3_5/qwen3_5.py:38-41): residual += x; hidden_row = RMSNorm(residual) * gamma;
// out = MoE(hidden_row). x and out may be the same buffer. M <= 64.
SV_API int snowllm_inference_moe_norm(const Weight* w, const void* x, void* residual,
                                      const void* gamma, float eps, void* hidden_row,
                                      const void* router, void* out, void* scratch,
                                      int64_t capacity, int64_t M, void* stream) {
  if (!w || !x || !residual || !gamma || !hidden_row || !router || !out || !scratch || M <= 0 ||
      M > MOE_ROWS || !moe_geometry_ok())
    return SV_EINVAL;
  const MoeWs ws = moe_ws(scratch, M);
  if (capacity < (int64_t)ws.bytes) return SV_EINVAL;
  int rc = snowverify_norm_prep(x, residual, residual, gamma, hidden_row, ws.ws, M,
                                active_geometry().hidden, eps, stream);
  if (rc) return rc;
  return moe_body(w, hidden_row, router, out, ws, M, stream);
}

// snowllm/_capi.py:599 -- scratch of snowllm_inference_mlp for M rows.
SV_API int64_t snowllm_fused_mlp_workspace_bytes(int64_t M) {
  if (M <= 0 || active_geometry().mlp_inter <= 0) return 0;
  return (int64_t)mlp_ws(nullptr, M).bytes;
}

// snowllm/_capi.py:689 (ops/inference.py:46-51; DenseMLP, models/qwen3_5/layers.py:192-205):
// out [M, hidden] = (silu(x Wg^T) * (x Wu^T)) Wd^T with w[0] the packed [2F, hidden] gate/up
// k-quant weight (gate rows first), w[1] (separate up) absent, w[2] the down weight. M <= 16.
SV_API int snowllm_inference_mlp(const Weight* w, const void* x, void* out, void* scratch,
                                 int64_t M, int decode, void* stream) {
  (void)decode;
  if (!w || !kquant(&w[0]) || !absent(&w[1]) || !kquant(&w[2]) || w[0].fmt != w[2].fmt)
    return SV_ENOTSUP;
  const BuildGeometry& g = active_geometry();
  if (!x || !out || !scratch || M <= 0 || M > MAX_ROWS || g.mlp_inter <= 0) return SV_EINVAL;
  const MlpWs ws = mlp_ws(scratch, M);
  int rc = snowverify_gemm_kquant_prepare_a(x, M, g.hidden, ws.ws_x, stream);
  if (rc) return rc;
  rc = snowverify_gate_up_swiglu(w[0].fmt, w[0].data[0], w[0].data[1], ws.ws_x, ws.act, M,
                                 g.mlp_inter, g.hidden, stream);
  if (rc) return rc;
  return snowllm_gemm_kquant_a(w[2].fmt, ws.act, (const uint8_t*)w[2].data[0],
                               (const uint8_t*)w[2].data[1], out, M, g.hidden, g.mlp_inter, 1,
                               ws.ws_act, stream);
}

// snowllm/_capi.py:355 -- scratch of snowllm_inference_head for M rows.
SV_API int64_t snowllm_lm_head_scratch_bytes(int64_t M) {
  return M <= 0 ? 0 : snowllm_gemm_kquant_a_ws_bytes(M, active_geometry().hidden);
}

// ---- LM head (snowllm/_capi.py:317-321, 354-356, 692; ops/embedding.py:12-16, 44-73;
// ops/inference.py:98-104; LMHead, models/qwen3_5/layers.py:209-228) ------------------------
// A 16-bit head is bf16 [vocab, hidden] repacked by snowllm_lm_head_shuffle_weight; a k-quant
// head is the Q4_K / Q8_0 blocks of [vocab, hidden] repacked by
// snowllm_lm_head_kquant_shuffle_weight (snowllm_gemm_kquant_shuffle_b's layout). Logits f32.

// Bytes a repacked 16-bit weight of `nbytes` source bytes may need: rows are padded to a
// multiple of 16, so at most 15 rows of the widest supported K (65536) are added.
SV_API int64_t snowllm_shuffle_bytes(int64_t nbytes) {
  return nbytes <= 0 ? 0 : nbytes + 15 * 65536 * 2;
}

SV_API int snowllm_lm_head_shuffle_weight(const void* w, void* out, void* stream) {
  const BuildGeometry& g = active_geometry();
  if (!w || !out || g.vocab_size <= 0 || g.hidden <= 0) return SV_EINVAL;
  return snowverify_dense_shuffle(w, out, g.vocab_size, g.hidden, WT_BF16, stream);
}

SV_API int64_t snowllm_lm_head_kquant_gguf_bytes(int fmt) {
  const BuildGeometry& g = active_geometry();
  return snowllm_kquant_gguf_bytes(fmt, g.vocab_size, g.hidden);
}
SV_API int64_t snowllm_lm_head_kquant_quant_bytes(int fmt) {
  const BuildGeometry& g = active_geometry();
  return snowllm_kquant_quant_bytes(fmt, g.vocab_size, g.hidden);
}
SV_API int64_t snowllm_lm_head_kquant_meta_bytes(int fmt) {
  const BuildGeometry& g = active_geometry();
  return snowllm_kquant_meta_bytes(fmt, g.vocab_size, g.hidden);
}
SV_API int snowllm_lm_head_kquant_shuffle_weight(int fmt, const uint8_t* blocks, uint8_t* quant,
                                                 uint8_t* meta, void* stream) {
  const BuildGeometry& g = active_geometry();
  return snowllm_gemm_kquant_shuffle_b(fmt, blocks, quant, meta, g.vocab_size, g.hidden, stream);
}

// bf16 head: x [M, hidden] bf16 rows against the repacked head, 16 rows per launch.
SV_API int snowllm_lm_head(const void* x, const void* w, float* logits, int64_t M, void* scratch,
                           void* stream) {
  (void)scratch;
  const BuildGeometry& g = active_geometry();
  if (!x || !w || !logits || M <= 0) return SV_EINVAL;
  for (int64_t r0 = 0; r0 < M; r0 += 16) {
    const int64_t rows = M - r0 < 16 ? M - r0 : 16;
    const int rc = snowverify_dense_gemv(WT_BF16, w, (const uint16_t*)x + r0 * g.hidden,
                                         logits + r0 * g.vocab_size, rows, g.vocab_size,
                                         g.hidden, 0, stream);
    if (rc) return rc;
  }
  return SV_OK;
}

// k-quant head: scratch holds snowllm_lm_head_scratch_bytes(M).
SV_API int snowllm_lm_head_kquant(int fmt, const void* x, const void* quant, const void* meta,
                                  float* logits, int64_t M, void* scratch, void* stream) {
  const BuildGeometry& g = active_geometry();
  if (!x || !quant || !meta || !logits || !scratch || M <= 0) return SV_EINVAL;
  return snowllm_gemm_kquant_a(fmt, x, (const uint8_t*)quant, (const uint8_t*)meta, logits, M,
                               g.vocab_size, g.hidden, 0, scratch, stream);
}

// The descriptor form: kind 0 = bf16 head, kind 2 / 3 = k-quant head.
SV_API int snowllm_inference_head(const Weight* w, const void* x, float* out, void* scratch,
                                  int64_t M, void* stream) {
  if (!w) return SV_EINVAL;
  if (w->kind == 0 && w->data[0]) return snowllm_lm_head(x, w->data[0], out, M, scratch, stream);
  if (kquant(w)) return snowllm_lm_head_kquant(w->fmt, x, w->data[0], w->data[1], out, M, scratch,
                                              stream);
  return SV_ENOTSUP;
}

// ---- DFlash draft: shape selection and the selector's hidden projection ------------------
// (snowllm/_capi.py:66-90, 227-239, 277, 282; snowllm/ops/dflash.py:21-135;
// models/qwen3_5/dflash_draft.py:187-204). The reference compiles its draft shapes in and
// snowllm_select_draft picks one; here any shape is run-time data. Of the draft's projections
// this build computes the one that feeds the candidate selector: SELECTOR_HIDDEN,
// hp [m, 256] bf16 = hidden [m, draft hidden] W^T, W [256, draft hidden] bf16 (kind 0,
// repacked by snowllm_draft_proj_shuffle_w) or Q4_K / Q8_0 (kind 2, repacked by
// snowllm_draft_proj_shuffle_w_kquant); fp32 accumulate, one bf16 rounding. The backbone's
// projections (FC, CTX_KV, QKV, O, GATE_UP, DOWN, CONV) return hipErrorNotSupported.
struct DraftShape {  // snowllm/_capi.py:67-72
  int64_t hidden, num_layers, num_heads, num_kv_heads, head_size, intermediate, num_taps;
};
namespace {
constexpr int PROJ_SELECTOR_HIDDEN = 7;   // snowllm/ops/dflash.py:29
constexpr int64_t SELECTOR_RANK = 256;    // the selector's codebook rank
DraftShape g_draft;
bool g_draft_set = false;

bool selector_proj(int which) { return which == PROJ_SELECTOR_HIDDEN && g_draft_set; }
}  // namespace

SV_API int snowllm_select_draft(const DraftShape* s) {
  if (!s || s->hidden <= 0 || s->hidden % 256 || s->hidden > 65536) return SV_EINVAL;
  g_draft = *s;
  g_draft_set = true;
  return SV_OK;
}
SV_API int64_t snowllm_draft_count(void) { return g_draft_set ? 1 : 0; }
SV_API int snowllm_draft_shape(int i, DraftShape* out) {
  if (i != 0 || !g_draft_set || !out) return SV_EINVAL;
  *out = g_draft;
  return SV_OK;
}
SV_API int64_t snowllm_draft_name(int i, char* buf, int64_t n) {
  const char* name = (i == 0 && g_draft_set) ? "selected" : "";
  const int64_t len = (int64_t)strlen(name);
  if (buf && n > 0) {
    const int64_t c = len < n - 1 ? len : n - 1;
    memcpy(buf, name, (size_t)c);
    buf[c] = 0;
  }
  return len;
}

SV_API int snowllm_draft_projection_shape(int which, int64_t* nk) {
  if (!nk) return SV_EINVAL;
  if (!selector_proj(which)) return SV_ENOTSUP;
  nk[0] = SELECTOR_RANK;
  nk[1] = g_draft.hidden;
  return SV_OK;
}

// plan = {n, k, scratch bytes} for m rows of the weight storage w (kind, fmt only).
SV_API int snowllm_draft_projection_plan(int which, const Weight* w, int64_t m, int64_t* plan) {
  if (!w || !plan || m <= 0) return SV_EINVAL;
  if (!selector_proj(which)) return SV_ENOTSUP;
  plan[0] = SELECTOR_RANK;
  plan[1] = g_draft.hidden;
  if (w->kind == 0) plan[2] = 0;
  else if (w->kind == 2 && (w->fmt == 4 || w->fmt == 8))
    plan[2] = snowllm_gemm_kquant_a_ws_bytes(m, g_draft.hidden);
  else return SV_ENOTSUP;
  return SV_OK;
}

SV_API int64_t snowllm_draft_projections_workspace_bytes(int64_t m) {
  if (m <= 0 || !g_draft_set) return 0;
  return snowllm_gemm_kquant_a_ws_bytes(m, g_draft.hidden);
}

SV_API int snowllm_draft_projection(int which, const Weight* w, const void* a, void* out,
                                    void* scratch, int64_t capacity, int64_t m, void* stream) {
  if (!w || !a || !out || m <= 0) return SV_EINVAL;
  if (!selector_proj(which)) return SV_ENOTSUP;
  const int64_t K = g_draft.hidden;
  if (w->kind == 0 && w->data[0]) {
    for (int64_t r0 = 0; r0 < m; r0 += 16) {
      const int64_t rows = m - r0 < 16 ? m - r0 : 16;
      const int rc = snowverify_dense_gemv(WT_BF16, w->data[0], (const uint16_t*)a + r0 * K,
                                           (uint16_t*)out + r0 * SELECTOR_RANK, rows,
                                           SELECTOR_RANK, K, 1, stream);
      if (rc) return rc;
    }
    return SV_OK;
  }
  if (w->kind == 2 && w->data[0] && w->data[1]) {
    if (!scratch || capacity < snowllm_gemm_kquant_a_ws_bytes(m, K)) return SV_EINVAL;
    return snowllm_gemm_kquant_a(w->fmt, a, (const uint8_t*)w->data[0],
                                 (const uint8_t*)w->data[1], out, m, SELECTOR_RANK, K, 1,
                                 scratch, stream);
  }
  return SV_ENOTSUP;
}

// bf16 [256, draft hidden] -> the projection's layout (snowllm_shuffle_bytes of its bytes).
SV_API int snowllm_draft_proj_shuffle_w(int which, const void* w, void* out, void* stream) {
  if (!w || !out) return SV_EINVAL;
  if (!selector_proj(which)) return SV_ENOTSUP;
  return snowverify_dense_shuffle(w, out, SELECTOR_RANK, g_draft.hidden, WT_BF16, stream);
}

SV_API int snowllm_draft_proj_shuffle_w_kquant(int which, int fmt, const uint8_t* blocks,
                                               uint8_t* quant, uint8_t* meta, void* stream) {
  if (!blocks || !quant || !meta) return SV_EINVAL;
  if (!selector_proj(which)) return SV_ENOTSUP;
  return snowllm_gemm_kquant_shuffle_b(fmt, blocks, quant, meta, SELECTOR_RANK, g_draft.hidden,
                                       stream);
}
