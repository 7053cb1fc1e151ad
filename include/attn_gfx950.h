/*
 * Attention-block entry points of libmoe_gfx950 (MI355X, gfx950): the gpt-oss
 * AttentionBlock around the MoE block, with its paged KV cache.
 *
 * The reference builds the block from Relax ops and mlc-llm's PagedKVCache
 * (model/attention.py:182-256): RMSNorm, a fused QKV nn.Linear, YaRN RoPE on
 * q and k, append_mha_kv, self_attention (prefill) / cross_attention (decode)
 * / both merged (extend), the sink scaling, the output nn.Linear and the
 * residual add.  The dense projections (QKV, output, unembedding) are
 * library GEMMs on the host side for prefill-sized inputs and the GEMV entry
 * points below (with their epilogues fused) for decode-sized ones.
 * The conventions of moe_gfx950.h hold: caller-owned device buffers, nothing
 * allocated, no host synchronisation, the stream last, MOE_OK or a negative
 * MOE_ERR_* code (no launch on error).
 *
 * Shapes fixed by gpt-oss: head_dim 64, 64 query heads, 8 key/value heads,
 * 16 tokens per page.  KV cache of one layer: bf16
 * [num_pages, 2 (k, v), 8, 16, 64] (mlc-llm's page layout, 32 KB per page).
 * A sequence's pages are listed in page_indices[page_indptr[b] ..
 * page_indptr[b+1]); its token at position p lives in page p / 16, slot
 * p % 16.  kv_len[b] counts the sequence's tokens including the ones this
 * forward appends.  Page ids outside [0, num_pages) and positions past a
 * sequence's listed pages are clamped (wrong keys, no fault): the caller
 * keeps the tables consistent.
 */
#ifndef ATTN_GFX950_H_
#define ATTN_GFX950_H_

#include "moe_gfx950.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RMSNorm, out = bf16(fp32(x r) w), r = 1/sqrt(mean(x^2) + eps).
 * Replaces nn.RMSNorm at model/attention.py:80 (block pre-norm) and
 * model/transformer.py:49,63 (final norm).  x, out [n, H] bf16; H % 8 == 0. */
MOE_API int attn_rms_norm(const uint16_t* x, int64_t n, int64_t H, const uint16_t* w, float eps,
                          uint16_t* out, moe_stream_t stream);

/* The QKV epilogue and the cache append: qkv [n, 5120] is the bf16 matmul
 * output t @ W_qkv^T (model/attention.py:204, without its bias); this adds the
 * bias (a second bf16 rounding, nn.Linear), applies YaRN RoPE to q and k at
 * positions[i] (model/attention.py:94-178: inv_freq [32] fp32 and the
 * concentration 0.1 ln(factor) + 1 come from the caller), writes q [n, 64,
 * 64] bf16 to q_out and appends k and v at cache slot slots[i] = page * 16 +
 * offset (PagedKVCache.append_mha_kv, tvm_fix.patch:14-33).  Slots outside
 * [0, 16 num_pages) are not written. */
MOE_API int attn_qkv_rope_append(const uint16_t* qkv, const uint16_t* qkv_bias, int64_t n,
                                 const int32_t* positions, const int32_t* slots,
                                 const float* inv_freq, float concentration, void* kv_cache,
                                 int64_t num_pages, uint16_t* q_out, moe_stream_t stream);

/* Workspace of attn_decode for `batch` sequences attending to at most
 * max_span keys each (min(kv_len, window) for sliding layers).  Its first
 * 32 x batch bytes are arrival counts that must be zero before the first call
 * on the workspace; every call leaves them zero (zero the whole workspace
 * once when it is allocated). */
MOE_API size_t attn_decode_workspace_bytes(int64_t batch, int64_t max_span);

/* Decode attention: one query token per sequence, q [batch, 64, 64] bf16 at
 * position kv_len[b] - 1, over the sequence's cached keys (all of them, or
 * the last `window` when window > 0), scaled by sm_scale, softmax in fp32,
 * then the sink scaling bf16(o) * bf16(sigmoid(lse - sinks[h])) of
 * model/attention.py:235-245.  out [batch, 64, 64] bf16.  Replaces
 * PagedKVCache.cross_attention at model/attention.py:219-222.  max_span bounds
 * every sequence's attended span; a sequence beyond it gets NaN outputs. */
MOE_API int attn_decode(const uint16_t* q, int64_t batch, const void* kv_cache, int64_t num_pages,
                        const int32_t* page_indptr, const int32_t* page_indices,
                        const int32_t* kv_len, int64_t max_span, int32_t window, float sm_scale,
                        const uint16_t* sinks, uint16_t* out, void* workspace,
                        size_t workspace_bytes, moe_stream_t stream);

/* Prefill / extend attention: sequence b's queries are q rows [q_indptr[b],
 * q_indptr[b+1]) at positions kv_len[b] - q_len .. kv_len[b] - 1 (already
 * appended to the cache); each attends causally to the cached keys, within
 * `window` when window > 0 (the mask of tvm_fix.patch:36-47), then the sink
 * scaling as in attn_decode.  Replaces PagedKVCache.self_attention (prefill,
 * an empty cache before the chunk) and self + cross attention merged
 * (extend), model/attention.py:216-232.  Scores and softmax in fp32; the
 * probabilities enter the bf16 MFMA as two bf16 pieces (about 16 bits).
 * max_q_len bounds every q_len. */
MOE_API int attn_prefill(const uint16_t* q, const int32_t* q_indptr, int64_t batch,
                         int64_t max_q_len, const void* kv_cache, int64_t num_pages,
                         const int32_t* page_indptr, const int32_t* page_indices,
                         const int32_t* kv_len, int32_t window, float sm_scale,
                         const uint16_t* sinks, uint16_t* out, moe_stream_t stream);

/* out = bf16(x + bf16(y + bias)): the output nn.Linear's bias add and the
 * residual of model/attention.py:254-256.  x, y, out [n, H]; H % 4 == 0. */
MOE_API int attn_bias_residual(const uint16_t* x, const uint16_t* y, const uint16_t* bias,
                               int64_t n, int64_t H, uint16_t* out, moe_stream_t stream);

/* Embedding gather, out[i] = table[ids[i]] (nn.Embedding,
 * model/transformer.py:39,101-105); ids outside [0, vocab) give zero rows.
 * H % 8 == 0. */
MOE_API int attn_embedding(const int32_t* ids, int64_t n, const uint16_t* table, int64_t vocab,
                           int64_t H, uint16_t* out, moe_stream_t stream);

/* Decode-sized dense projection (nn.Linear's matmul for M <= 8 tokens):
 * out[m][n] = bf16(sum_k t[m][k] W[n][k]), fp32 accumulation, one bf16
 * rounding, where t = x, or t = RMSNorm(x) with weight norm_w and eps when
 * norm_w is not NULL (the same arithmetic as attn_rms_norm).  x [M, K], W [N,
 * K], out [M, N] bf16; K % 8 == 0, K <= 4096.  Replaces the final norm and
 * the unembedding nn.Linear at decode (model/transformer.py:63,95-100). */
MOE_API int attn_gemv(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W, int64_t N,
                      const uint16_t* norm_w, float eps, uint16_t* out, moe_stream_t stream);

/* The attention output nn.Linear at decode with its bias and the residual
 * (model/attention.py:254-256): out = bf16(residual + bf16(bf16(x W^T) +
 * bias)); residual, out [M, N]. */
MOE_API int attn_gemv_bias_residual(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W,
                                    int64_t N, const uint16_t* bias, const uint16_t* residual,
                                    uint16_t* out, moe_stream_t stream);

/* The block's pre-norm (when norm_w is not NULL), the fused QKV nn.Linear at
 * decode (model/attention.py:80,204) and attn_qkv_rope_append in one kernel:
 * W [5120, K], then the bias, YaRN RoPE, q_out and the cache append exactly
 * as attn_qkv_rope_append does. */
MOE_API int attn_qkv_gemv_rope_append(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W,
                                      const uint16_t* norm_w, float eps,
                                      const uint16_t* qkv_bias, const int32_t* positions,
                                      const int32_t* slots, const float* inv_freq,
                                      float concentration, void* kv_cache, int64_t num_pages,
                                      uint16_t* q_out, moe_stream_t stream);

/* Workspace of attn_sample_top_p: 256 KB per sequence.  It must be zero
 * before the first call (e.g. hipMemset once after allocation); every call
 * leaves it zero again. */
MOE_API size_t attn_sample_workspace_bytes(int64_t batch);

/* Top-p sampling of one token per sequence from bf16 logits [batch, vocab]
 * (the unembedding's bf16 output, model/transformer.py:95-100), replacing
 * TVM's vm.builtin.sample_top_p_from_logits (engine.py:39-40,165-167):
 * argmax if temperature < 1e-6; else e = exp((l - max) / temperature), the
 * top-p mass is the cumulative mass in descending-logit order up to and
 * including the element at which it reaches top_p, and the first element whose
 * cumulative mass exceeds uniform x that mass is chosen (equal logits in index
 * order; past the mass: the first maximum).  exp is rounded once to fp32 and
 * the masses are summed exactly (fp64) where TVM adds fp32 values serially.
 * out_ids [batch] int32. */
MOE_API int attn_sample_top_p(const uint16_t* logits, int64_t batch, int64_t vocab,
                              float temperature, float top_p, float uniform, int32_t* out_ids,
                              void* workspace, size_t workspace_bytes, moe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTN_GFX950_H_ */
