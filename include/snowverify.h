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
 * top_k covers the vocabulary with top_p >= 1 are written in vocabulary order; rows with
 * top_k <= 1024 are sorted by probability (ties to the lower id), renormalised and truncated
 * by top-p; unused slots are (0, -1). Other rows are written as (NaN, -2). */
int snowllm_sampling_topk_topp(const float* dense, float* values, int64_t* ids, int64_t rows,
                               int64_t vocab, int64_t width, const int32_t* top_k,
                               const float* top_p, void* stream);

/* Per-row top-k/top-p sample: softmax, candidate list, pick = #(u >= cumsum(values))
 * (snowllm/_capi.py:564; snowllm/ops/sampling.py:34-62). */
int snowllm_sampling_sample(const float* logits, const int32_t* top_k, const float* top_p,
                            const float* temperature, const float* uniform, int64_t* out,
                            void* ws, int64_t ws_bytes, int64_t B, int64_t V, int64_t width,
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

/* ---- GGUF k-quant GEMV ----------------------------------------------------------------- */
/* Format ids as in the reference (snowllm/ops/moe.py:189-190): 4 = Q4_K, 8 = Q8_0. */

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
int snowllm_gemm_kquant_prepare_a(const void* a, int64_t M, int64_t K, void* ws, void* stream);

/* Extension, no counterpart in the reference: gemm_kquant_a on a prepared workspace. */
int snowllm_gemm_kquant_a_prepared(int fmt, const uint8_t* quant, const uint8_t* meta, void* c,
                                   int64_t M, int64_t N, int64_t K, int c_is_bf16,
                                   const void* ws, void* stream);

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

#ifdef __cplusplus
}
#endif

#endif /* SNOWVERIFY_H */
