/*
 * snowverify.h -- C ABI of libsnowverify.so, the gfx950 (MI355X) kernels of SnowLLM's
 * speculative-decoding verify step.
 *
 * Every entry point keeps the name, argument order and meaning of the reference's binding
 * (snowllm/_capi.py) so that the reference's ctypes wrappers (snowllm/ops/*.py) can drive it
 * unchanged. Conventions, as in the reference (snowllm/_capi.py:837-842, ops/_common.py:48-100):
 *   - launches return an int HIP status (0 = success); size queries return int64;
 *   - all pointers are device pointers of caller-allocated, contiguous buffers;
 *   - the HIP stream (hipStream_t as void*) is always the last argument;
 *   - nothing allocates or synchronises inside a launch, so launches can be captured into a
 *     HIP graph. Calls on one device must be stream-ordered (the library keeps small
 *     per-device scratch for argmax and draft_reject, whose reference signatures carry no
 *     workspace).
 */
#ifndef SNOWVERIFY_H
#define SNOWVERIFY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- plumbing ------------------------------------------------------------------------ */

/* ABI version of this library (its own numbering; replaces the libsnowllm ABI check at
 * snowllm/_capi.py:176-194). */
int snowllm_abi_version(void);

/* Text for a status code (snowllm/_capi.py:246, used by check() at :837-842). */
const char* snowllm_error_string(int status);

/* Synchronise a stream (snowllm/_capi.py:247). */
int snowllm_synchronize(void* stream);

/* ---- acceptance ---------------------------------------------------------------------- */

/* Largest top-k width the candidate lists support as "whole vocabulary" (snowllm/_capi.py:245,
 * SAMPLING_MAX_K in snowllm/ops/_common.py:42). Returns 2^19, the vocabulary limit. */
int64_t snowllm_sampling_max_k(void);

/* out[b] = argmax_v logits[b, v]; NaN counts as -inf, ties go to the lowest index
 * (snowllm/_capi.py:590; wrapper snowllm/ops/sampling.py:65-72). */
int snowllm_sampling_argmax(const float* logits, int64_t* out, int64_t B, int64_t V,
                            void* stream);

/* acc[r] = 1 + #leading j with tokens[r, j] == drafts[r, j] (snowllm/_capi.py:579; wrapper
 * snowllm/ops/metadata.py:244-251). Strides are in elements. */
int snowllm_spec_accept(const int64_t* tokens, const int64_t* drafts, int64_t* acc, int64_t b,
                        int64_t t, int64_t tokens_stride, int64_t drafts_stride, void* stream);

/* Bytes of the sampling workspace (snowllm/_capi.py:563; snowllm/ops/sampling.py:28-31). */
int64_t snowllm_sampling_workspace_bytes(int64_t batch, int64_t vocab, int64_t width);

/* Temperature softmax of logits [rows, vocab] into dense [rows, vocab] f32
 * (snowllm/_capi.py:585; snowllm/ops/sampling.py:87-89). `dense` must be the start of a
 * workspace of snowllm_sampling_workspace_bytes(rows, vocab, width) bytes: row statistics are
 * kept behind the dense block. Temperatures <= 0 count as 1. */
int snowllm_sampling_softmax(const float* logits, float* dense, int64_t rows, int64_t vocab,
                             const float* temperature, void* stream);

/* Top-k / top-p candidate lists from dense probabilities (snowllm/_capi.py:586;
 * snowllm/ops/sampling.py:90-91): values f32 [rows, width], ids i64 [rows, width]. Rows whose
 * top_k covers the vocabulary with top_p >= 1 are written in vocabulary order; every other row
 * (any top_k up to the vocabulary, any top_p) is sorted by probability (ties to the lower id),
 * renormalised over its top k and truncated by top-p (entries past the cut keep their id with
 * probability 0); unused slots are (0, -1). `dense` must start a workspace of
 * snowllm_sampling_workspace_bytes(rows, vocab, width) bytes (lists wider than 1024 are sorted
 * behind the dense block). A row whose top_k exceeds `width` cannot be written and comes out
 * as (NaN, -2): callers size the width as the batch's largest top_k, as the reference's do. */
int snowllm_sampling_topk_topp(const float* dense, float* values, int64_t* ids, int64_t rows,
                               int64_t vocab, int64_t width, const int32_t* top_k,
                               const float* top_p, void* stream);

/* Per-row top-k/top-p sample: softmax, candidate list, pick = #(u >= cumsum(values))
 * (snowllm/_capi.py:564; snowllm/ops/sampling.py:34-62). */
int snowllm_sampling_sample(const float* logits, const int32_t* top_k, const float* top_p,
                            const float* temperature, const float* uniform, int64_t* out,
                            void* ws, int64_t ws_bytes, int64_t B, int64_t V, int64_t width,
                            void* stream);

/* Repetition / frequency / presence penalties on one logit row (snowllm/_capi.py:589; wrapper
 * snowllm/ops/sampling.py:94-100): for each of the n listed token ids (unique; the request's
 * prompt and output ids) with output count c, logit = logit > 0 ? logit / repetition :
 * logit * repetition, then logit - frequency * c, then logit - presence (when c > 0). Ids
 * outside [0, vocab) are skipped. */
int snowllm_sampling_penalties(float* logits, const int64_t* ids, const int32_t* counts, int n,
                               int vocab, float presence, float frequency, float repetition,
                               void* stream);

/* Rejection sampling of a draft prefix plus residual/bonus resample (snowllm/_capi.py:289;
 * wrapper snowllm/ops/dflash.py:201-219; semantics tests/test_dflash_sampling.py:94-119).
 * p/ids [b*width, p_width], drafts [b, width-1], cand/q [S, width-1, q_width], slots/valid
 * [b], uniform [b, width] -> out [b, width] (-1 padded), accepted [b]. Candidate rows must not
 * repeat an id (as produced by snowllm_sampling_topk_topp and the draft selector). */
int snowllm_draft_reject(const float* p, const int64_t* ids, const int64_t* drafts,
                         const int64_t* cand, const float* q, const int32_t* slots,
                         const int32_t* valid, const float* uniform, int64_t* out,
                         int64_t* accepted, int64_t b, int64_t width, int64_t p_width,
                         int64_t q_width, void* stream);

/* Extension: the acceptance straight from the target logits, for requests whose candidate
 * lists are the whole vocabulary in vocabulary order (top-k >= vocab, top-p 1) -- the DFlash
 * verify's rejection branch (snowllm/engine/dflash_sampling.py:61-69) with the arithmetic, and
 * so the bits, of snowllm_sampling_softmax + snowllm_sampling_topk_topp + snowllm_draft_reject,
 * in three launches that never materialise the probabilities and never wait on one another's
 * workgroups. logits [b*width, vocab] f32, temperature [b*width] (NULL: 1; <= 0 counts as 1);
 * the rest as snowllm_draft_reject. b*width <= 256, width <= 64 (larger shapes return
 * hipErrorNotSupported with nothing launched: the caller then takes snowllm_sampling_softmax +
 * snowllm_sampling_topk_topp + snowllm_draft_reject). Calls on one device must be
 * stream-ordered (library-owned statistics). */
int snowverify_accept_reject(const float* logits, const float* temperature,
                             const int64_t* drafts, const int64_t* cand, const float* q,
                             const int32_t* slots, const int32_t* valid, const float* uniform,
                             int64_t* out, int64_t* accepted, int64_t b, int64_t width,
                             int64_t vocab, int64_t q_width, void* stream);
/* Extension: the greedy branch (snowllm/engine/dflash_sampling.py:56-59; spec_decode.py:
 * 196-207) in one launch: tokens [b, width] = argmax of each logit row (as
 * snowllm_sampling_argmax), accepted [b] = 1 + leading matches with drafts [b, width-1] (as
 * snowllm_spec_accept). Limits as snowverify_accept_reject. */
int snowverify_accept_greedy(const float* logits, const int64_t* drafts, int64_t* tokens,
                             int64_t* accepted, int64_t b, int64_t width, int64_t vocab,
                             void* stream);

/* ---- DFlash 2 candidate selector (snowllm/ops/dflash.py:164-198; semantics
 * tests/test_dflash_sampling.py:44-75, tests/test_dflash_selector_topk.py:42-61) ------------
 * Per position: the 16 largest logits (stable descending, NaN as -inf), scores = values +
 * the codebook correction pred[prev] . hp[row] . succ[cand], then the first argmax (greedy)
 * or a pick from softmax(scores / T) with uniform[b, j]; prev = the pick. hp bf16
 * [b*ell, 256], logits f32 [b*ell, v] (16 <= v <= 262144), pred/succ bf16 [v, 256], anchor
 * i64 [b], path i64 [b, ell] (ell <= 32). */
/* Scratch bytes for n = b * ell rows (snowllm/_capi.py:285). */
int64_t snowllm_draft_select_scratch_bytes(int64_t n);
/* Greedy walk, path only (snowllm/_capi.py:286-287). */
int snowllm_draft_select(const void* hp, const float* logits, const void* pred, const void* succ,
                         const int64_t* anchor, int64_t* path, void* scratch, int64_t b,
                         int64_t ell, int64_t v, void* stream);
/* Per-row greedy (temperature <= 0) or sampling walk; writes candidate_ids i64 and
 * probabilities f32 [S, ell, 16] at row slots[b] (snowllm/_capi.py:288). top_k must be 16. */
int snowllm_draft_sample(const void* hp, const float* logits, const void* pred, const void* succ,
                         const int64_t* anchor, const float* temperature, const float* uniform,
                         const int32_t* slots, int64_t* path, int64_t* candidate_ids,
                         float* probabilities, void* scratch, int64_t b, int64_t ell, int64_t v,
                         int64_t top_k, void* stream);
/* Extension, no counterpart in the reference: the selector at codebook rank `rank` (64, 128,
 * 256 or 512); temperature == NULL is snowllm_draft_select. */
int snowverify_draft_select(const void* hp, const float* logits, const void* pred,
                            const void* succ, const int64_t* anchor, const float* temperature,
                            const float* uniform, const int32_t* slots, int64_t* path,
                            int64_t* candidate_ids, float* probabilities, void* scratch,
                            int64_t b, int64_t ell, int64_t v, int64_t rank, void* stream);

/* ---- GGUF k-quant GEMV ----------------------------------------------------------------- */
/* Format ids as in the reference (snowllm/ops/moe.py:189-190, checkpoint/gguf/source.py:33):
 * 4 = Q4_K, 5 = Q5_K, 6 = Q6_K, 8 = Q8_0. */

/* Sizes of the GGUF blocks and of the packed (quant, meta) pair for an [N, K] weight
 * (snowllm/_capi.py:323-325; snowllm/ops/gemm.py:130-133). quant - 4 + meta == gguf.
 * N must be a multiple of 16 and K of 256; -1 otherwise. */
int64_t snowllm_kquant_gguf_bytes(int fmt, int64_t N, int64_t K);
int64_t snowllm_kquant_quant_bytes(int fmt, int64_t N, int64_t K);
int64_t snowllm_kquant_meta_bytes(int fmt, int64_t N, int64_t K);

/* 1 if the format is implemented (snowllm/_capi.py:780-781). */
int snowllm_kquant_supported(int fmt);

/* Repack GGUF blocks into the MFMA lane layout (snowllm/_capi.py:619;
 * snowllm/ops/gemm.py:136-147). */
int snowllm_gemm_kquant_shuffle_b(int fmt, const uint8_t* gguf, uint8_t* quant, uint8_t* meta,
                                  int64_t N, int64_t K, void* stream);
/* Extension, no counterpart in the reference: repack two GGUF tensors of one format, `top`
 * (rows 0 .. n_top - 1) and `bottom` (rows n_top .. N - 1), as one [N, K] matrix -- an expert's
 * [gate; up] from its two stacks (snowllm_gemm_kquant_shuffle_b is the single-tensor case). */
int snowverify_kquant_shuffle_split(int fmt, const uint8_t* top, const uint8_t* bottom,
                                    int64_t n_top, uint8_t* quant, uint8_t* meta, int64_t N,
                                    int64_t K, void* stream);

/* Activation workspace bytes for gemm_kquant_a (snowllm/_capi.py:620). */
int64_t snowllm_gemm_kquant_a_ws_bytes(int64_t M, int64_t K);

/* C[M, N] = A[M, K] (bf16) x W[N, K]^T, W dequantised on the fly, fp32 accumulate; C is bf16
 * when c_is_bf16 else f32 (snowllm/_capi.py:621-622; snowllm/ops/gemm.py:150-163). */
int snowllm_gemm_kquant_a(int fmt, const void* a, const uint8_t* quant, const uint8_t* meta,
                          void* c, int64_t M, int64_t N, int64_t K, int c_is_bf16, void* ws,
                          void* stream);

/* Extension (tuning knob), no counterpart in the reference: force a GEMV tile shape,
 * 0 = automatic. Process-global. */
void snowverify_gemv_variant(int v);

/* Extension, no counterpart in the reference: fill the gemm_kquant_a operand workspace from
 * bf16 activations A[M, K] once, so that several weights sharing one input reuse it. */
int snowverify_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws, void* stream);

/* Extension, no counterpart in the reference: gemm_kquant_a on a prepared workspace. */
int snowverify_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta, void* c,
                                   int64_t M, int64_t N, int64_t K, int c_is_bf16,
                                   const void* ws, void* stream);

/* Extension, no counterpart in the reference: snowverify_gemm_kquant_a_prepared writing row m
 * of the result at c + m * ldc elements (N <= ldc < 2^31), so that weights of different
 * formats fill the column ranges of one output: the Q|K and V rows of an attention projection
 * whose GGUF tensors differ in format (snowllm_inference_qkv's split form). Same bits per
 * element as the contiguous form. */
int snowverify_gemm_kquant_a_prepared_ld(int fmt, const uint8_t* quant, const uint8_t* meta,
                                         void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                         int c_is_bf16, const void* ws, void* stream);

/* No counterpart in the reference: snowllm_gemm_kquant_a for callers that cannot allocate
 * (code under HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc). It
 * allocates nothing and takes no workspace: up to 16 rows the GEMV converts the activations
 * itself; above that the operand workspace is a device array inside the library, 2,244,608
 * bytes per GPU for the life of the process. M <= 64 and K <= 16384, larger sizes return
 * hipErrorInvalidValue. Calls on one GPU share that array: calls that overlap on one device
 * (different streams) race. */
int snowverify_gemm_kquant_a_noalloc(int fmt, const void* a, const uint8_t* quant,
                                     const uint8_t* meta, void* c, int64_t M, int64_t N,
                                     int64_t K, int c_is_bf16, void* stream);

/* ---- paged attention --------------------------------------------------------------- */

/* Scratch bytes of snowverify_paged_attention (split-KV partials). */
int64_t snowverify_paged_attention_scratch_bytes(int64_t batch, int64_t tokens, int64_t num_heads,
                                                 int64_t num_kv_heads, int64_t head_size);

/* GQA attention of `tokens` query rows per request against the paged bf16 KV cache, with the
 * shapes passed explicitly (the reference's snowllm_paged_attention, snowllm/_capi.py:220 and
 * snowllm/ops/attention_full.py:120-177, reads them from its compiled-in geometry).
 * q/out bf16 [batch*tokens, num_heads, head_size]; pools in the reference layouts
 * K [blocks, Hkv, d/16, page, 16], V [blocks, Hkv, page/4, d, 4] (tests/test_lfm2_dspark_
 * reference.py:30-36); table i32 [batch, table_stride]; lens i32 [batch] = context + tokens.
 * Row t sees the context and, of the block, the rows whose bits are set in tree[b*tokens + t]
 * (u64), or rows 0..t when tree is null (causal, tests/test_lfm2_long_attention.py:40-44).
 * head_size 128 or 256, page_size 16, tokens <= 64. */
int snowverify_paged_attention(const void* q, const void* k_pool, const void* v_pool, void* out,
                               const int32_t* table, const int32_t* lens, const uint64_t* tree,
                               int64_t batch, int64_t tokens, int64_t num_heads,
                               int64_t num_kv_heads, int64_t head_size, int64_t page_size,
                               int64_t table_stride, float scale, void* scratch,
                               int64_t scratch_bytes, void* stream);

/* Extension, no counterpart in the reference (which runs snowllm_qk_norm_rope_cache, then
 * snowllm_paged_attention): both in the attention's launches. Its workgroups normalise and
 * rotate their query rows from the raw projection rows, and the workgroup whose split holds a
 * block row's cache position writes that row's K (normalised, rotated) and V into the pools
 * first -- the same bits as the separate writer. proj [batch*tokens, proj_stride] bf16 (q head
 * hq at hq * q_head_stride, k / v head h at k_off / v_off + h * head_size); cos/sin rows
 * cs_stride apart (first `half` used, half a multiple of 32 and at most 64, wider returns
 * hipErrorNotSupported); slots [batch*tokens] the cache
 * slot of each block row (position lens[b] - tokens + t); q_out [batch*tokens, Hq, D] or NULL. */
int snowverify_paged_attention_qk(const void* proj, int64_t proj_stride, int64_t q_head_stride,
                                  int64_t k_off, int64_t v_off, const void* q_gamma,
                                  const void* k_gamma, const float* cos_in, const float* sin_in,
                                  int64_t cs_stride, int64_t half, float eps,
                                  const int32_t* slots, void* q_out, void* k_pool, void* v_pool,
                                  void* out, const int32_t* table, const int32_t* lens,
                                  const uint64_t* tree, int64_t batch, int64_t tokens,
                                  int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
                                  int64_t page_size, int64_t table_stride, float scale,
                                  void* scratch, int64_t scratch_bytes, void* stream);
/* Extension, no counterpart in the reference: snowverify_paged_attention_qk that also writes
 * the output projection's operand workspace out_ws (as snowverify_gemm_kquant_prepare_a would
 * from `out` viewed as [batch*tokens, num_heads*head_size]; snowllm_gemm_kquant_a_ws_bytes of
 * that shape), so the projection runs snowverify_gemm_kquant_a_prepared with the same bits as
 * snowllm_gemm_kquant_a on `out`. head_size 256 only (hipErrorNotSupported otherwise). */
int snowverify_paged_attention_qk_ws(const void* proj, int64_t proj_stride,
                                     int64_t q_head_stride, int64_t k_off, int64_t v_off,
                                     const void* q_gamma, const void* k_gamma,
                                     const float* cos_in, const float* sin_in, int64_t cs_stride,
                                     int64_t half, float eps, const int32_t* slots, void* q_out,
                                     void* k_pool, void* v_pool, void* out,
                                     const int32_t* table, const int32_t* lens,
                                     const uint64_t* tree, int64_t batch, int64_t tokens,
                                     int64_t num_heads, int64_t num_kv_heads, int64_t head_size,
                                     int64_t page_size, int64_t table_stride, float scale,
                                     void* scratch, int64_t scratch_bytes, void* out_ws,
                                     void* stream);

/* Extension, no counterpart in the reference (a tuning knob): pages per context split of
 * snowverify_paged_attention; 0 = automatic. Returns the previous value. */
int snowverify_attention_pages_per_split(int pages);
/* Extension, no counterpart in the reference (a tuning knob): waves per 16-row tile of the
 * attention's split kernel, 1 or 2 (two split the head's output columns), or 3 (eight waves,
 * one or two per tile, for five to seven tiles); 0 = automatic. Returns the previous value. */
int snowverify_attention_d_split(int dh);
/* Extension, no counterpart in the reference (a tuning knob): pages in the attention split
 * kernel's LDS ring, 4 or 8; 0 = automatic. Returns the previous value. */
int snowverify_attention_ring(int pages);
/* Extension, no counterpart in the reference (a tuning knob): row groups of the attention split
 * kernel's one-wave-per-tile form, 1 or 2 (two workgroups per context split, each with half of
 * the row tiles, on one XCD); 0 = automatic. Returns the previous value. */
int snowverify_attention_row_groups(int groups);

/* ---- geometry-driven operator entry points (reference signatures) ---------------------
 * Shapes from the active geometry (see below); weights in the reference's _Weight descriptor
 * (snowllm/ops/inference.py:10-22) holding this library's repacked layouts: k-quant (quant,
 * meta) from snowllm_gemm_kquant_shuffle_b as kind 2 (kind 3: an expert stack, the experts'
 * packed matrices back to back), 16-bit dense matrices (router, LM head) repacked by
 * snowverify_dense_shuffle as kind 0. Features the verify path of this build does not carry
 * (int8 KV, gated attention output, split Q/KV weights, fp8 dense scales, the DSA indexer,
 * hashed routing, varlen prefill) return hipErrorNotSupported. */
typedef struct SnowllmWeight {
  void* data[3];
  void* scale;
  int kind; /* -1 absent, 0 dense, 1 dense + scale, 2 k-quant, 3 k-quant expert stack */
  int fmt;  /* 4 = Q4_K, 8 = Q8_0 */
} SnowllmWeight;

/* snowllm/ops/attention_full.py:120-123. inputs: q, k_pool, v_pool, k_scale, v_scale,
 * cu_seqlens, table, lens, qmap, gate; outputs: out, plan, workspace. */
typedef struct PagedAttentionStep {
  void* inputs[10];
  void* outputs[3];
  int64_t batch, pages, q_blocks, slots, tokens, page_size, gate_stride, gate_row0;
  float scale;
  int varlen; /* bit 0 varlen, bit 1 host lengths, bit 2 prepared metadata */
} PagedAttentionStep;

/* QKV projection with the input norm fused (snowllm/_capi.py:688; ops/inference.py:34-43):
 * out [M, qkv_proj_n] bf16 = RMSNorm(residual += x) * gamma . W^T (no residual: RMSNorm(x);
 * no gamma: x). w[3]: the QKV k-quant weight, then an optional split V (w[0] then holds the
 * Q|K rows [qkv_off_v, hidden] and w[1] the V rows in its own format), then a bf16 KV (absent:
 * hipErrorNotSupported). */
int64_t snowllm_qkv_proj_scratch_bytes(int64_t M);                     /* _capi.py:251 */
/* Sizing queries the reference's hot-path ops modules bind at import: the O projection's
 * scratch (snowllm/_capi.py:254; ops/attention_full.py:512); the draft model's attention
 * sizing (snowllm/_capi.py:300-301; ops/dflash.py:337-338), answered with the decode
 * attention's for the active geometry -- the draft's layers are not carried; the hashed
 * router's scratch (snowllm/_capi.py:351; ops/moe.py:279), 0: hashed routing is refused. */
int64_t snowllm_attn_out_scale_oproj_scratch_bytes(int64_t rows);
int64_t snowllm_draft_paged_attn_num_slots(int64_t num_seqs);
int64_t snowllm_draft_paged_attn_workspace_size(int64_t num_slots, int64_t q_tokens);
int64_t snowllm_moe_router_shuffle_bytes(int64_t rows);
int snowllm_inference_qkv(const SnowllmWeight* w, const void* x, void* residual,
                          const void* gamma, float eps, void* scratch, void* out, int64_t M,
                          int path, const void* index_w, void* index_out, void* stream);
/* Attention output projection (snowllm/_capi.py:223-225; ops/attention_full.py:54-117):
 * plan -> {elements of the attention output, scratch bytes}; the gate is NULL (no output gate
 * in these geometries); out [m, hidden] bf16 = a [m, heads * head_size] . Wo^T (k-quant). */
int snowllm_attn_output_plan(int64_t m, int prefill, int kv_int8, int64_t* out);
void* snowllm_attn_output_gate(const void* proj, int prefill, int kv_int8);
int snowllm_attn_output_project(const void* a, const void* proj, int64_t proj_stride,
                                const void* dense, const void* quant, const void* meta,
                                const void* scale, int fmt, void* scratch, void* out, int64_t m,
                                int prefill, int kv_int8, void* stream);
/* Paged attention through the step descriptor (snowllm/_capi.py:218-220; ops/attention_full.py:
 * 126-177): the decode/verify form (tokens query rows per request, causal in the block). */
int64_t snowllm_paged_attention_scratch_bytes(int64_t batch, int64_t tokens, int varlen);
int snowllm_paged_attention_varlen(int prefill, int64_t tokens, int chunk_decode);
int snowllm_paged_attention(const PagedAttentionStep* step, void* scratch, int64_t bytes,
                            void* stream);
/* Prepared attention metadata (snowllm/_capi.py:808-812; ops/attention_full.py:136-150):
 * none is needed, so the size is 0 (the reference's wrapper then passes no prepared buffer and
 * its runner skips the decode plan, engine/qwen_runner.py:202-208); prepare checks its
 * arguments and launches nothing. */
int64_t snowllm_paged_attention_prepared_bytes(int64_t batch, int64_t tokens, int64_t slots,
                                               int varlen);
int snowllm_paged_attention_prepare(const int32_t* lens, void* result, int64_t batch,
                                    int64_t tokens, int64_t slots, int64_t block_size,
                                    void* stream);
/* Split-KV decode attention and its plan (snowllm/_capi.py:358, 371-373, 506-509; read at
 * import by ops/attention_full.py:516-518, 565; called at :1147-1161, 1232-1238). The context
 * splits are sized at launch from the block-table width and the kernels read the lengths
 * themselves, so the plan is one int32 that nothing writes and the plan call only checks its
 * arguments. A slot is one sequence's partials region. max_q_tokens: T * G <= 128 and
 * T <= 64 for the active geometry. q rows are q_pitch elements apart (0: heads * head_size)
 * from row q_row0; out [num_seqs * q_tokens, heads, head_size]; ws sized by
 * snowllm_paged_decode_workspace_size(num_slots, q_tokens), num_slots >= num_seqs. */
int64_t snowllm_paged_decode_max_q_tokens(void);
int64_t snowllm_paged_decode_num_slots(int64_t num_seqs);
int64_t snowllm_paged_decode_workspace_size(int64_t num_slots, int64_t q_tokens);
int64_t snowllm_paged_decode_plan_elems(int64_t num_seqs, int64_t num_slots);
int snowllm_paged_attn_decode_plan(const int32_t* seq_lens, int32_t* plan, int64_t num_seqs,
                                   int64_t num_slots, int64_t block_size, int uniform,
                                   void* stream);
int snowllm_paged_attn_decode(const void* q, const int32_t* seq_lens, const void* k_cache,
                              const void* v_cache, void* out, const int32_t* block_tables,
                              const int32_t* plan, int64_t num_seqs, int64_t max_blocks,
                              int64_t num_slots, void* ws, float scale, int64_t q_tokens,
                              int64_t block_size, int64_t q_pitch, int64_t q_row0, void* stream);
/* Query-block map of a varlen batch, host arithmetic on host arrays (snowllm/_capi.py:364-365;
 * ops/attention_full.py:539-547): blocks of 16 query rows; the map holds (sequence, first row
 * of the block in the sequence) int32 pairs. */
int64_t snowllm_prefill_q_blocks(const int32_t* lens, int64_t B);
void snowllm_prefill_q_block_map(const int32_t* lens, int64_t B, int32_t* map);
/* Page sizes of the KV pools (snowllm/_capi.py:243; read at import by ops/_common.py:35-43):
 * writes up to n to out (if not NULL) and returns their count (one: 16). */
int64_t snowllm_kv_block_sizes(int64_t* out, int64_t n);
/* MoE block (snowllm/_capi.py:315, 690-691, 805-807; ops/inference.py:54-95): w[4] = experts'
 * gate/up stack, experts' down stack, shared gate/up, shared down; router: repacked bf16
 * [E+1, hidden], the shared expert's gate last. The _norm form first sets residual += x and
 * hidden_row = RMSNorm(residual) * gamma. x and out may alias. M <= 64 (the workspace query
 * returns 0 above). */
int64_t snowllm_moe_workspace_bytes(int64_t rows);
int64_t snowllm_inference_moe_workspace_bytes(int64_t rows, int64_t flags);
int snowllm_inference_moe(const SnowllmWeight* w, const void* x, const void* router,
                          const int64_t* token_ids, const int32_t* tid2eid, void* out,
                          void* scratch, int64_t capacity, int64_t M, int64_t flags,
                          void* stream);
int snowllm_inference_moe_norm(const SnowllmWeight* w, const void* x, void* residual,
                               const void* gamma, float eps, void* hidden_row,
                               const void* router, void* out, void* scratch, int64_t capacity,
                               int64_t M, void* stream);
/* Expert and router repack from the GGUF layout (snowllm/_capi.py:313-314, 326-331;
 * ops/moe.py:81-86, 136-162), over the active geometry (F = moe_inter, H = hidden): gate and
 * up are the ffn_gate_exps / ffn_up_exps blocks [E, F, H], down the ffn_down_exps blocks
 * [E, H, F] (fmt 4 = Q4_K, 8 = Q8_0; the MoE entry points compute Q4_K). Expert e's packed
 * [2F, H] gate/up (gate rows first) and [H, F] down sit at e times their packed size, as
 * snowllm_inference_moe reads them (kind 3). The router is bf16 [E + 1, H], shared gate last;
 * a router bias returns hipErrorNotSupported. */
int64_t snowllm_moe_kquant_gate_up_quant_bytes(int fmt, int64_t E);
int64_t snowllm_moe_kquant_gate_up_meta_bytes(int fmt, int64_t E);
int64_t snowllm_moe_kquant_down_quant_bytes(int fmt, int64_t E);
int64_t snowllm_moe_kquant_down_meta_bytes(int fmt, int64_t E);
int snowllm_moe_kquant_shuffle_gate_up(int fmt, const uint8_t* gate, const uint8_t* up,
                                       uint8_t* quant, uint8_t* meta, int64_t E, void* stream);
int snowllm_moe_kquant_shuffle_down(int fmt, const uint8_t* down, uint8_t* quant, uint8_t* meta,
                                    int64_t E, void* stream);
int64_t snowllm_moe_shuffle_router_bytes(void);
int snowllm_moe_shuffle_router(const void* router, const void* bias, void* out, void* stream);
/* Dense SwiGLU MLP (snowllm/_capi.py:599, 689; ops/inference.py:46-51): w[3] = packed [2F, H]
 * gate/up (gate rows first), separate up (absent), down. M <= 16. */
int64_t snowllm_fused_mlp_workspace_bytes(int64_t M);
int snowllm_inference_mlp(const SnowllmWeight* w, const void* x, void* out, void* scratch,
                          int64_t M, int decode, void* stream);
/* LM head (snowllm/_capi.py:317-321, 354-356, 692; ops/embedding.py:12-16, 44-73;
 * ops/inference.py:98-104): logits [M, vocab] f32 for the normalised bf16 rows x. A 16-bit head
 * is bf16 [vocab, hidden] repacked by snowllm_lm_head_shuffle_weight into
 * snowllm_shuffle_bytes(vocab * hidden * 2) bytes (descriptor kind 0); a k-quant head is the
 * GGUF Q4_K / Q8_0 blocks repacked by snowllm_lm_head_kquant_shuffle_weight (kind 2 or 3). */
int64_t snowllm_shuffle_bytes(int64_t nbytes);
int snowllm_lm_head_shuffle_weight(const void* w, void* out, void* stream);
int64_t snowllm_lm_head_kquant_gguf_bytes(int fmt);
int64_t snowllm_lm_head_kquant_quant_bytes(int fmt);
int64_t snowllm_lm_head_kquant_meta_bytes(int fmt);
int snowllm_lm_head_kquant_shuffle_weight(int fmt, const uint8_t* blocks, uint8_t* quant,
                                          uint8_t* meta, void* stream);
int64_t snowllm_lm_head_scratch_bytes(int64_t M);
int snowllm_lm_head(const void* x, const void* w, float* logits, int64_t M, void* scratch,
                    void* stream);
int snowllm_lm_head_kquant(int fmt, const void* x, const void* quant, const void* meta,
                           float* logits, int64_t M, void* scratch, void* stream);
int snowllm_inference_head(const SnowllmWeight* w, const void* x, float* out, void* scratch,
                           int64_t M, void* stream);

/* ---- DSpark Markov head (snowllm/_capi.py:567-573; snowllm/ops/dspark.py:10-16, 53-77;
 * semantics tests/test_lfm2_dspark_reference.py:143-152) ----------------------------------
 * Per request r and block row j: latent = w1[prev] (prev = anchor[r], then the previous row's
 * pick; a prev outside [0, v) gives a zero latent), bias = w2 latent summed exactly and rounded
 * once to bf16 (fp32 with fp32_bias), out[r, j] = argmax fp32(base + bias) (NaN as -inf, ties
 * to the lowest index), confidence[r, j] = sigmoid([pre_head row, latent] . conf_weight +
 * conf_bias). base f32 rows of stride base_stride; w2 packed by snowllm_dspark_pack_weight;
 * b <= 16, rank % 8 == 0, rank <= 512, b * rank <= 4096; one launch per block row. Calls on one device must be
 * stream-ordered (library-owned arrival counter). */
int64_t snowllm_dspark_weight_bytes(int64_t n, int64_t k);
int snowllm_dspark_pack_weight(const void* raw, void* packed, int64_t n, int64_t k, void* stream);
int64_t snowllm_dspark_markov_workspace_bytes(int64_t b, int64_t v, int64_t rank, int64_t block);
int snowllm_dspark_markov(const void* base, const void* w1, const void* w2, const int64_t* anchor,
                          const void* pre_head, const float* conf_weight, const float* conf_bias,
                          int64_t* out, float* confidence, void* workspace, int64_t b, int64_t v,
                          int64_t rank, int64_t block, int64_t base_stride, int64_t h, int64_t ps,
                          int64_t workspace_bytes, int fp32_bias, void* stream);

/* ---- DFlash draft shape and the selector's hidden projection (snowllm/_capi.py:66-90,
 * 227-239, 277, 282; snowllm/ops/dflash.py:21-135; models/qwen3_5/dflash_draft.py:187-204) --
 * Any draft shape is accepted (hidden % 256 == 0). Projection `which` 7 (SELECTOR_HIDDEN):
 * hp [m, 256] bf16 = hidden [m, draft hidden] W^T, fp32 accumulate, W bf16 (descriptor kind
 * 0, repacked by snowllm_draft_proj_shuffle_w into snowllm_shuffle_bytes of its bytes) or
 * Q4_K / Q8_0 (kind 2). The backbone's projections (0-6) return hipErrorNotSupported. */
typedef struct DraftShape {
  int64_t hidden, num_layers, num_heads, num_kv_heads, head_size, intermediate, num_taps;
} DraftShape;
int snowllm_select_draft(const DraftShape* shape);
int64_t snowllm_draft_count(void);
int snowllm_draft_shape(int i, DraftShape* out);
int64_t snowllm_draft_name(int i, char* buf, int64_t n);
int snowllm_draft_projection_shape(int which, int64_t* nk);
int snowllm_draft_projection_plan(int which, const SnowllmWeight* w, int64_t m, int64_t* plan);
int64_t snowllm_draft_projections_workspace_bytes(int64_t m);
int snowllm_draft_projection(int which, const SnowllmWeight* w, const void* a, void* out,
                             void* scratch, int64_t capacity, int64_t m, void* stream);
int snowllm_draft_proj_shuffle_w(int which, const void* w, void* out, void* stream);
int snowllm_draft_proj_shuffle_w_kquant(int which, int fmt, const uint8_t* blocks, uint8_t* quant,
                                        uint8_t* meta, void* stream);

/* ---- geometry ------------------------------------------------------------------------ */
/* The reference compiles its shapes in (snowllm/_capi.py:44-113); here they are run-time
 * data. BuildGeometry has the reference's 37 int64 fields in the same order. */
typedef struct BuildGeometry BuildGeometry;

/* Current geometry (snowllm/_capi.py:50-53). */
void snowllm_model_config(BuildGeometry* out);
/* Select a geometry: 0 = Qwen3.6-35B-A3B shape (BASELINE configs 4/5), 100 = dense 8B shape
 * (snowllm/_capi.py:94-103). */
int snowllm_select_geometry(int geo);
int snowllm_active_geometry(void);                                     /* _capi.py:106-107 */
int64_t snowllm_geometry_name(int geo, char* buf, int64_t n);          /* _capi.py:110-113 */
/* Extension, no counterpart in the reference: install arbitrary shapes (geometry id 1000). */
int snowverify_define_geometry(const BuildGeometry* g);

/* ---- layer plumbing --------------------------------------------------------------------- */
/* Embedding gather (snowllm/_capi.py:375; snowllm/ops/embedding.py:18-25): bf16 table of the
 * current geometry. The extension takes an fp16 (table_f16 = 1) or bf16 table [V, H]. */
int snowllm_gather_embedding(const int64_t* ids, const void* table, void* out, int64_t M,
                             void* stream);
int snowverify_gather_embedding(const int64_t* ids, const void* table, void* out, int64_t M,
                                int64_t V, int64_t H, int table_f16, void* stream);
/* Embedding gather from a Q4_K table (snowllm/_capi.py:726; ops/embedding.py:27-41): weight
 * [vocab, hidden / 256 * 144] bytes of GGUF blocks -> bf16 [rows, hidden], each value
 * fp32(d sc) q - fp32(dmin m) rounded once to bf16. hidden % 256 == 0. */
int snowllm_gather_embedding_q4_k(const int64_t* ids, const void* weight, void* out, int64_t rows,
                                  int64_t vocab, int64_t hidden, void* stream);

/* RMSNorm y = x rsqrt(mean(x^2) + eps) gamma (snowllm/_capi.py:376, 381; ops/norm.py:66-97);
 * the residual form first sets residual = x + residual. */
int snowllm_rmsnorm(const void* x, const void* gamma, void* out, int64_t M, float eps,
                    void* stream);
int snowllm_rmsnorm_residual(const void* x, void* residual, const void* gamma, void* out,
                             int64_t M, float eps, void* stream);
int snowverify_rmsnorm(const void* x, void* residual, const void* gamma, void* out, int64_t M,
                       int64_t H, float eps, void* stream);

/* RoPE tables cos/sin [M, 64] of pos * inv_freq[32] (snowllm/ops/rope.py:11-24, the plain
 * form): the reference's rotary dimension 64, the 32 values repeated in columns 32..63. */
int snowllm_rope_cos_sin(const int64_t* pos, const float* inv_freq, float* cos_out,
                         float* sin_out, int64_t M, void* stream);
/* Extension: RoPE tables cos/sin [M, half] of pos * inv_freq (any rotary width). */
int snowverify_rope_cos_sin(const int64_t* pos, const float* inv_freq, float* cos_out,
                            float* sin_out, int64_t M, int64_t half, void* stream);

/* QK-norm + RoPE + paged KV write (snowllm/_capi.py:397-399; ops/attention_full.py:736-784),
 * shapes from the active geometry: q heads of proj [m, n] at the geometry's q head stride, K
 * rows at kp (stride ks), V rows at v (stride vs); cos/sin [m, 64]; q [m, Hq, D]; K/V into the
 * bf16 pools at slots[m] (negative: skipped). k_scale and v_scale must be NULL (no int8 KV). */
int snowllm_qk_norm_rope_cache(const void* proj, int64_t n, const void* kp, int64_t ks,
                               const void* v, int64_t vs, const void* q_gamma,
                               const void* k_gamma, const float* cos_in, const float* sin_in,
                               void* q, void* k_cache, void* v_cache, const void* k_scale,
                               const void* v_scale, const int32_t* slots, int64_t m, float eps,
                               int64_t block_size, void* stream);
/* Extension: the same with explicit shapes: proj [M, stride] = q|k|v bf16 -> q_out [M, Hq, D];
 * cos/sin [M, half]. D in {64, 128, 256}; half a multiple of 32 with 2 half <= D. */
int snowverify_qk_norm_rope_cache(const void* proj, int64_t stride, const void* q_gamma,
                                  const void* k_gamma, const float* cos_in, const float* sin_in,
                                  void* q_out, void* k_pool, void* v_pool, const int32_t* slots,
                                  int64_t M, int64_t Hq, int64_t Hkv, int64_t D, int64_t half,
                                  int64_t page, float eps, void* stream);

/* slot = table[seq, pos / page] * page + pos % page (snowllm/_capi.py:361; ops/cache.py:40-53;
 * spec_decode.py:183). Rows with a negative seq or pos, a page past the table's width or a
 * negative (padding) table entry get slot -1, which the cache writers skip. */
int snowllm_resolve_slots(const int32_t* table, int64_t stride, const int32_t* seq,
                          const int32_t* pos, int32_t* out, int64_t M, int64_t page, void* stream);

/* K/V pool bytes for num_blocks pages of the current geometry (snowllm/_capi.py:359). */
void snowllm_kv_pool_bytes(int64_t num_blocks, int64_t block_size, int kv_int8, int64_t* k,
                           int64_t* v);

/* Extensions: SwiGLU over a [M, 2F] gate|up block, bf16 add, and MoE routing (softmax over E
 * routed logits, top-k, renormalised; sigmoid of column E as the shared-expert gate). */
int snowverify_swiglu(const void* gate_up, int64_t stride, void* out, int64_t M, int64_t F,
                      void* stream);
int snowverify_add_bf16(const void* a, const void* b, void* out, int64_t n, void* stream);
int snowverify_moe_route(const float* logits, int64_t stride, int64_t M, int64_t E, int64_t topk,
                         float* weights, int32_t* ids, float* shared_w, void* stream);

/* ---- feed-forward (extensions; the reference reaches these through snowllm_inference_*,
 * snowllm/_capi.py:687-692, whose weight descriptors and workspaces are internal) ------------ */
/* res_out = x + res_in; y = RMSNorm(res_out) * gamma into the k-quant operand workspace ws (and
 * y_out if given). H <= 8192; res_out and y_out may alias x or res_in (in place). */
int snowverify_norm_prep(const void* x, const void* res_in, void* res_out, const void* gamma,
                         void* y_out, void* ws, int64_t M, int64_t H, float eps, void* stream);
/* snowverify_norm_prep on the MoE layer's output, combined in the same launch: x = bf16(sum_k
 * pairs[r*topk + k] + shared_out[r]) (snowverify_moe_combine's order), written to x_out if
 * given. pairs [M*topk, H] f32, shared_out [M, H] f32 or NULL. */
int snowverify_norm_prep_moe(const float* pairs, const float* shared_out, int64_t topk,
                             void* x_out, const void* res_in, void* res_out, const void* gamma,
                             void* y_out, void* ws, int64_t M, int64_t H, float eps,
                             void* stream);
/* The post-attention block of a MoE layer up to the experts in one launch, with the bits of
 * snowverify_norm_prep (res_out, y_out, ws) + snowverify_dense_gemv (bf16 router [E (+1), H]
 * repacked by snowverify_dense_shuffle; f32 logits [M, E (+1)]) + snowverify_moe_route_plan
 * (weights/ids [M, topk], shared_w [M] or NULL for no shared expert, plan). res_out must not
 * alias x or res_in. M <= 16; H a multiple of 512, <= 4096, M * (H + 8) * 2 <= 131072; E <= 256;
 * topk <= 16. Library-owned counter: calls on one device must be stream-ordered. */
int snowverify_norm_router_plan(const void* x, const void* res_in, void* res_out,
                                const void* gamma, float eps, void* ws, void* y_out,
                                const void* router, float* logits, int64_t M, int64_t H,
                                int64_t E, int64_t topk, float* weights, int32_t* ids,
                                float* shared_w, void* plan, void* stream);
/* 16-bit weight GEMV: repack size, repack (wt 1 = fp16, 2 = bf16), and C = A W^T (fp16 weights
 * take the operand workspace, bf16 weights bf16 activations). M <= 256; each workgroup loads a
 * weight tile once for up to four 16-row tiles. */
int64_t snowverify_dense_bytes(int64_t N, int64_t K);
int snowverify_dense_shuffle(const void* src, void* dst, int64_t N, int64_t K, int wt,
                             void* stream);
int snowverify_dense_gemv(int wt, const void* w, const void* act, void* c, int64_t M, int64_t N,
                          int64_t K, int c_is_bf16, void* stream);
/* act[M, F] = silu(x Wg^T) * (x Wu^T), gate_up the packed [2F, K] k-quant weight. */
int snowverify_gate_up_swiglu(int fmt, const void* quant, const void* meta, const void* ws,
                              void* act, int64_t M, int64_t F, int64_t K, void* stream);
/* MoE: plan of the experts the block touches (device side), then the experts of one layer.
 * A plan holds up to 64 block rows (M * topk <= 512): each expert the block touches takes one
 * slot per 16 of its rows (its rows in ascending order), experts in ascending id, then the
 * shared expert ceil(M / 16) slots; snowverify_moe_max_slots(M, topk, E, shared) bounds the
 * slots (the expert launches' max_slots and their activation scratch [slots, 16, F]; 0 past
 * the limits). */
int64_t snowverify_moe_plan_bytes(void);
int64_t snowverify_moe_max_slots(int64_t M, int64_t topk, int64_t E, int shared);
int snowverify_moe_plan(const int32_t* ids, int64_t M, int64_t topk, int64_t E, int shared,
                        void* plan, void* stream);
/* snowverify_moe_route and snowverify_moe_plan in one launch (shared slot iff shared_w). */
int snowverify_moe_route_plan(const float* logits, int64_t stride, int64_t M, int64_t E,
                              int64_t topk, float* weights, int32_t* ids, float* shared_w,
                              void* plan, void* stream);
/* The three stages of snowverify_moe_experts, for callers that schedule them separately:
 * gate/up + SwiGLU over max_slots plan slots (compact activation rows), the down GEMV into
 * pre-weighted pairs / shared rows, and the fixed-order combine. */
int snowverify_moe_gate_up(int fmt, const void* gu_quant, const void* gu_meta,
                           const void* sh_gu_quant, const void* sh_gu_meta, const void* plan,
                           const void* ws, void* act, int64_t M, int64_t max_slots, int64_t E,
                           int64_t H, int64_t F, void* stream);
int snowverify_moe_down(int fmt, const void* dn_quant, const void* dn_meta,
                        const void* sh_dn_quant, const void* sh_dn_meta, const void* plan,
                        const void* act, const float* weights, const float* shared_w,
                        float* pairs, float* shared_out, int64_t max_slots, int64_t E, int64_t H,
                        int64_t F, void* stream);
/* Extension, no counterpart in the reference (whose expert stages are internal to
 * snowllm_inference_moe): snowverify_moe_gate_up then snowverify_moe_down in one launch, same
 * outputs and bits; a down item starts as soon as its slot's gate/up items are done. Uses
 * library-owned flags, so calls on one device must be stream-ordered. */
int snowverify_moe_gate_up_down(int fmt, const void* gu_quant, const void* gu_meta,
                                const void* dn_quant, const void* dn_meta,
                                const void* sh_gu_quant, const void* sh_gu_meta,
                                const void* sh_dn_quant, const void* sh_dn_meta, const void* plan,
                                const void* ws, const float* weights, const float* shared_w,
                                void* act, float* pairs, float* shared_out, int64_t M,
                                int64_t max_slots, int64_t E, int64_t H, int64_t F, void* stream);
/* Non-zero once a snowverify_moe_gate_up_down launch has timed out waiting for its own
 * activations (never expected; reading it synchronises the device). */
int snowverify_moe_sync_error(void);
int snowverify_moe_combine(const float* pairs, const float* shared_out, void* out, int64_t M,
                           int64_t topk, int64_t H, void* stream);
int snowverify_moe_experts(int fmt, const void* gu_quant, const void* gu_meta,
                           const void* dn_quant, const void* dn_meta, const void* sh_gu_quant,
                           const void* sh_gu_meta, const void* sh_dn_quant,
                           const void* sh_dn_meta, const void* plan, const void* ws,
                           const float* weights, const float* shared_w, void* act, float* pairs,
                           float* shared_out, void* out, int64_t M, int64_t topk, int64_t E,
                           int64_t H, int64_t F, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SNOWVERIFY_H */
