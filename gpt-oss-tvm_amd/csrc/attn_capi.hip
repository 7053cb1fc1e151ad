// C ABI of the attention-block entry points: argument validation, then the
// launchers of attn_kernels.hip.  Declarations and reference citations:
// include/attn_gfx950.h.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/attn_gfx950.h"

extern "C" {
int attn_launch_rms_norm(const void* x, int n, int H, const void* w, float eps, void* out,
                         hipStream_t s);
int attn_launch_qkv_rope_append(const void* qkv, const void* bias, int n, const int* positions,
                                const int* slots, const float* inv_freq, float conc, void* cache,
                                int num_pages, void* q_out, hipStream_t s);
int attn_launch_decode(const void* q, int batch, const void* cache, const int* page_indptr,
                       const int* page_indices, int num_pages, const int* kv_len, int window,
                       float sm_scale, const void* sinks, int splits, int cps, float* part_o,
                       float* part_ml, int* arrive, void* out, hipStream_t s);
int attn_launch_prefill(const void* q, const int* q_indptr, int batch, int max_q_len,
                        const void* cache, const int* page_indptr, const int* page_indices,
                        int num_pages, const int* kv_len, int window, float sm_scale,
                        const void* sinks, void* out, hipStream_t s);
int attn_launch_bias_residual(const void* x, const void* y, const void* bias, int64_t n, int H,
                              void* out, hipStream_t s);
int attn_launch_embedding(const int* ids, int n, const void* table, int vocab, int H, void* out,
                          hipStream_t s);
size_t attn_sample_state_bytes();
int attn_launch_gemv(const void* x, int M, int K, const void* W, int N, void* out,
                     const void* norm_w, float eps, const void* bias, const void* res,
                     hipStream_t s);
int attn_launch_qkv_gemv(const void* x, int M, int K, const void* W, const void* norm_w,
                         float eps, const void* bias, const int* positions, const int* slots,
                         const float* inv_freq, float conc, void* cache, int num_pages,
                         void* q_out, hipStream_t s);
int attn_launch_sample(const void* logits, int batch, int V, float temperature, float top_p,
                       float uniform, int* out, void* state, hipStream_t s);
}

namespace {

constexpr int64_t kHeadDim = 64, kQHeads = 64, kKvHeads = 8, kPage = 16;
constexpr int64_t kDecChunk = 128;     // keys per chunk of a decode workgroup
constexpr int64_t kMaxTokens = 1 << 24;
constexpr int64_t kMaxPages = ((int64_t)1 << 31) / kPage;

inline bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool a4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
inline hipStream_t as_stream(moe_stream_t s) { return (hipStream_t)s; }
inline int status(int launch_rc) { return launch_rc == 0 ? MOE_OK : MOE_ERR_LAUNCH; }

// Chunks of 128 keys per decode workgroup: more with larger batches, where
// there are workgroups enough (a workgroup's fixed costs, the page-table
// reads before its first loads and the published partial after its last
// chunk, then spread over more keys).  It depends on the batch only (the
// kernel makes a span of at most two chunks one split), so a call's results
// do not depend on the span bound (a captured graph fixes the
// bound at the pool's capacity).
int64_t decode_cps(int64_t batch) { return batch >= 32 ? 8 : batch >= 8 ? 4 : batch >= 2 ? 2 : 1; }
int64_t decode_splits(int64_t batch, int64_t max_span) {
  const int64_t keys = kDecChunk * decode_cps(batch);
  return (max_span + keys - 1) / keys;
}

}  // namespace

extern "C" {

int attn_rms_norm(const uint16_t* x, int64_t n, int64_t H, const uint16_t* w, float eps,
                  uint16_t* out, moe_stream_t stream) {
  if (n < 0 || n > kMaxTokens || H <= 0 || H % 8 || H > 65536) return MOE_ERR_SHAPE;
  if (n == 0) return MOE_OK;
  if (!x || !w || !out) return MOE_ERR_NULL;
  if (!a16(x) || !a16(w) || !a16(out)) return MOE_ERR_ALIGN;
  return status(attn_launch_rms_norm(x, (int)n, (int)H, w, eps, out, as_stream(stream)));
}

int attn_qkv_rope_append(const uint16_t* qkv, const uint16_t* qkv_bias, int64_t n,
                         const int32_t* positions, const int32_t* slots, const float* inv_freq,
                         float concentration, void* kv_cache, int64_t num_pages, uint16_t* q_out,
                         moe_stream_t stream) {
  if (n < 0 || n > kMaxTokens || num_pages <= 0 || num_pages > kMaxPages) return MOE_ERR_SHAPE;
  if (n == 0) return MOE_OK;
  if (!qkv || !qkv_bias || !positions || !slots || !inv_freq || !kv_cache || !q_out)
    return MOE_ERR_NULL;
  if (!a16(qkv) || !a16(qkv_bias) || !a16(kv_cache) || !a16(q_out) || !a4(positions) ||
      !a4(slots) || !a4(inv_freq))
    return MOE_ERR_ALIGN;
  return status(attn_launch_qkv_rope_append(qkv, qkv_bias, (int)n, positions, slots, inv_freq,
                                            concentration, kv_cache, (int)num_pages, q_out,
                                            as_stream(stream)));
}

// Workspace of attn_decode: the arrival counts [batch][8] (int32, padded to
// 256 bytes; zero before the first call, left zero by every call), then the
// split partials o [batch][64][splits][64] and (m, l) [batch][64][splits][2].
static size_t decode_counts_bytes(int64_t batch) {
  return ((size_t)batch * kKvHeads * 4 + 255) & ~(size_t)255;
}

size_t attn_decode_workspace_bytes(int64_t batch, int64_t max_span) {
  if (batch <= 0 || max_span <= 0) return 0;
  const size_t parts = (size_t)batch * kQHeads * (size_t)decode_splits(batch, max_span);
  return decode_counts_bytes(batch) + parts * (kHeadDim + 2) * sizeof(float) + 256;
}

int attn_decode(const uint16_t* q, int64_t batch, const void* kv_cache, int64_t num_pages,
                const int32_t* page_indptr, const int32_t* page_indices, const int32_t* kv_len,
                int64_t max_span, int32_t window, float sm_scale, const uint16_t* sinks,
                uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  if (batch < 0 || batch > 65535 || num_pages <= 0 || num_pages > kMaxPages) return MOE_ERR_SHAPE;
  if (batch == 0) return MOE_OK;
  if (max_span <= 0 || max_span > kMaxPages * kPage) return MOE_ERR_SHAPE;
  if (!q || !kv_cache || !page_indptr || !page_indices || !kv_len || !sinks || !out || !workspace)
    return MOE_ERR_NULL;
  if (!a16(q) || !a16(kv_cache) || !a16(out) || !a16(workspace) || !a4(page_indptr) ||
      !a4(page_indices) || !a4(kv_len) || ((uintptr_t)sinks & 1u))
    return MOE_ERR_ALIGN;
  if (workspace_bytes < attn_decode_workspace_bytes(batch, max_span)) return MOE_ERR_WORKSPACE;
  const int64_t splits = decode_splits(batch, max_span);
  if (splits > 65535) return MOE_ERR_SHAPE;
  int* arrive = (int*)workspace;
  float* part_o = (float*)((char*)workspace + decode_counts_bytes(batch));
  float* part_ml = part_o + (size_t)batch * kQHeads * splits * kHeadDim;
  return status(attn_launch_decode(q, (int)batch, kv_cache, page_indptr, page_indices,
                                   (int)num_pages, kv_len, window, sm_scale, sinks, (int)splits,
                                   (int)decode_cps(batch), part_o, part_ml, arrive, out,
                                   as_stream(stream)));
}

int attn_prefill(const uint16_t* q, const int32_t* q_indptr, int64_t batch, int64_t max_q_len,
                 const void* kv_cache, int64_t num_pages, const int32_t* page_indptr,
                 const int32_t* page_indices, const int32_t* kv_len, int32_t window,
                 float sm_scale, const uint16_t* sinks, uint16_t* out, moe_stream_t stream) {
  if (batch < 0 || max_q_len < 0 || max_q_len > kMaxTokens || num_pages <= 0 ||
      num_pages > kMaxPages)
    return MOE_ERR_SHAPE;
  if (batch == 0 || max_q_len == 0) return MOE_OK;
  const int64_t tiles = (max_q_len + 63) / 64;
  if (tiles * batch >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  if (!q || !q_indptr || !kv_cache || !page_indptr || !page_indices || !kv_len || !sinks || !out)
    return MOE_ERR_NULL;
  if (!a16(q) || !a16(kv_cache) || !a16(out) || !a4(q_indptr) || !a4(page_indptr) ||
      !a4(page_indices) || !a4(kv_len) || ((uintptr_t)sinks & 1u))
    return MOE_ERR_ALIGN;
  return status(attn_launch_prefill(q, q_indptr, (int)batch, (int)max_q_len, kv_cache,
                                    page_indptr, page_indices, (int)num_pages, kv_len, window,
                                    sm_scale, sinks, out, as_stream(stream)));
}

int attn_bias_residual(const uint16_t* x, const uint16_t* y, const uint16_t* bias, int64_t n,
                       int64_t H, uint16_t* out, moe_stream_t stream) {
  if (n < 0 || n > kMaxTokens || H <= 0 || H % 4 || H > 65536) return MOE_ERR_SHAPE;
  if (n == 0) return MOE_OK;
  if (!x || !y || !bias || !out) return MOE_ERR_NULL;
  if (((uintptr_t)x & 7u) || ((uintptr_t)y & 7u) || ((uintptr_t)bias & 7u) || ((uintptr_t)out & 7u))
    return MOE_ERR_ALIGN;
  return status(attn_launch_bias_residual(x, y, bias, n, (int)H, out, as_stream(stream)));
}

int attn_embedding(const int32_t* ids, int64_t n, const uint16_t* table, int64_t vocab, int64_t H,
                   uint16_t* out, moe_stream_t stream) {
  if (n < 0 || n > kMaxTokens || vocab <= 0 || vocab >= ((int64_t)1 << 31) || H <= 0 || H % 8 ||
      H > 65536)
    return MOE_ERR_SHAPE;
  if (n == 0) return MOE_OK;
  if (!ids || !table || !out) return MOE_ERR_NULL;
  if (!a4(ids) || !a16(table) || !a16(out)) return MOE_ERR_ALIGN;
  return status(attn_launch_embedding(ids, (int)n, table, (int)vocab, (int)H, out,
                                      as_stream(stream)));
}

size_t attn_sample_workspace_bytes(int64_t batch) {
  return batch > 0 ? (size_t)batch * attn_sample_state_bytes() : 0;
}

int attn_sample_top_p(const uint16_t* logits, int64_t batch, int64_t vocab, float temperature,
                      float top_p, float uniform, int32_t* out_ids, void* workspace,
                      size_t workspace_bytes, moe_stream_t stream) {
  if (batch < 0 || batch > 65535 || vocab <= 0 || vocab >= ((int64_t)1 << 30)) return MOE_ERR_SHAPE;
  if (batch == 0) return MOE_OK;
  if (!(temperature >= 0.0f) || !(top_p > 0.0f) || !(uniform >= 0.0f)) return MOE_ERR_UNSUPPORTED;
  if (!logits || !out_ids || !workspace) return MOE_ERR_NULL;
  if (!a16(logits) || !a4(out_ids) || !a16(workspace)) return MOE_ERR_ALIGN;
  if (workspace_bytes < attn_sample_workspace_bytes(batch)) return MOE_ERR_WORKSPACE;
  return status(attn_launch_sample(logits, (int)batch, (int)vocab, temperature, top_p, uniform,
                                   out_ids, workspace, as_stream(stream)));
}

namespace {
int check_gemv(const void* x, int64_t M, int64_t K, const void* W, int64_t N, const void* out) {
  if (M < 1 || M > 8 || K <= 0 || K % 8 || K > 4096 || N <= 0 || N >= ((int64_t)1 << 31))
    return MOE_ERR_SHAPE;
  if (!x || !W || !out) return MOE_ERR_NULL;
  if (!a16(x) || !a16(W) || ((uintptr_t)out & 1u)) return MOE_ERR_ALIGN;
  return MOE_OK;
}
}  // namespace

int attn_gemv(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W, int64_t N,
              const uint16_t* norm_w, float eps, uint16_t* out, moe_stream_t stream) {
  int rc = check_gemv(x, M, K, W, N, out);
  if (rc) return rc;
  if (norm_w && ((uintptr_t)norm_w & 1u)) return MOE_ERR_ALIGN;
  return status(attn_launch_gemv(x, (int)M, (int)K, W, (int)N, out, norm_w, eps, nullptr,
                                 nullptr, as_stream(stream)));
}

int attn_gemv_bias_residual(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W, int64_t N,
                            const uint16_t* bias, const uint16_t* residual, uint16_t* out,
                            moe_stream_t stream) {
  int rc = check_gemv(x, M, K, W, N, out);
  if (rc) return rc;
  if (!bias || !residual) return MOE_ERR_NULL;
  if (((uintptr_t)bias & 1u) || ((uintptr_t)residual & 1u)) return MOE_ERR_ALIGN;
  return status(attn_launch_gemv(x, (int)M, (int)K, W, (int)N, out, nullptr, 0.0f, bias,
                                 residual, as_stream(stream)));
}

int attn_qkv_gemv_rope_append(const uint16_t* x, int64_t M, int64_t K, const uint16_t* W,
                              const uint16_t* norm_w, float eps, const uint16_t* qkv_bias,
                              const int32_t* positions, const int32_t* slots,
                              const float* inv_freq, float concentration, void* kv_cache,
                              int64_t num_pages, uint16_t* q_out, moe_stream_t stream) {
  int rc = check_gemv(x, M, K, W, kHeadDim * (kQHeads + 2 * kKvHeads), q_out);
  if (rc) return rc;
  if (num_pages <= 0 || num_pages > kMaxPages) return MOE_ERR_SHAPE;
  if (!qkv_bias || !positions || !slots || !inv_freq || !kv_cache) return MOE_ERR_NULL;
  if (!a16(kv_cache) || !a4(positions) || !a4(slots) || !a4(inv_freq) ||
      ((uintptr_t)qkv_bias & 1u) || (norm_w && ((uintptr_t)norm_w & 1u)))
    return MOE_ERR_ALIGN;
  return status(attn_launch_qkv_gemv(x, (int)M, (int)K, W, norm_w, eps, qkv_bias, positions,
                                     slots, inv_freq, concentration, kv_cache, (int)num_pages,
                                     q_out, as_stream(stream)));
}

}  // extern "C"
