// C ABI of libmoe_gfx950: argument validation, workspace layout and the
// block-level chain.  Declarations and reference citations: include/moe_gfx950.h.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "../../include/moe_gfx950.h"

extern "C" {
int moe_launch_dequant(const void* blocks, const void* scales, void* out, int64_t rows, int fast,
                       hipStream_t stream);
int moe_launch_router(const void* x, const void* norm_w, const void* gate_w, const void* gate_b,
                      int n, int H, int E, int k, float eps, void* t_out, void* idx_out,
                      void* w_out, hipStream_t stream);
int moe_launch_router_pieces(const void* x, const void* norm_w, const void* gate_w,
                             const void* gate_b, int n, int H, int E, int k, float eps,
                             void* t_out, void* idx_out, void* w_out, void* pq, void* pqs,
                             hipStream_t stream);
int moe_launch_permute(const void* idx, int nk, int k, int E, void* indptr, void* sorted_pairs,
                       void* token_indices, void* expert_ids, void* pair_pos, hipStream_t stream);
int moe_launch_router_logits(const void* x, const void* norm_w, const void* gate_w,
                             const void* gate_b, int n, int H, int E, float eps, void* t_out,
                             float* logits, void* pq, void* pqs, void* zero_e,
                             hipStream_t stream);
int moe_select_chunks(int n);
int moe_launch_select_group(const float* logits, int n, int E, int k, void* idx_out, void* w_out,
                            void* counts, void* indptr, void* sorted_pairs, void* token_indices,
                            void* expert_ids, void* pair_pos, int zero_ints, hipStream_t stream);
int moe_launch_router_select(const void* x, const void* norm_w, const void* gate_w,
                             const void* gate_b, int n, int H, int E, int k, float eps, void* t_out,
                             float* logits, void* pq, void* pqs, void* zero_e, void* idx_out,
                             void* w_out, void* indptr, void* sorted_pairs, void* token_indices,
                             void* expert_ids, void* pair_pos, void* zero, int zero_ints,
                             void* arrive, hipStream_t stream);
size_t moe_pieces_q_bytes(int64_t rows, int64_t K, int pieces);
size_t moe_pieces_total_bytes(int64_t rows, int64_t K, int pieces);
int moe_launch_pieces(const void* x, int x_is_f32, int rows, int K, int pieces, void* packed,
                      hipStream_t stream);
int moe_launch_mx_gemv(const void* packed, int rows, int pieces, const void* indptr,
                       const void* sorted_pairs, int k_top, int arow_mode, int orow_mode,
                       const void* blocks, const void* scales, const void* bias, int E, int N,
                       int K, int max_tokens, int rows_active, int swiglu, float alpha,
                       float limit, void* out, int out_ld, hipStream_t stream);
int moe_launch_mx_gemm(const void* packed, int rows, int pieces, const void* indptr,
                       const void* sorted_pairs, int k_top, int arow_mode, int orow_mode,
                       const void* blocks, const void* scales, const void* bias, int E, int N,
                       int K, int rows_active, int swiglu, float alpha, float limit, void* out,
                       int out_ld, void* out_qs, hipStream_t stream);
int moe_launch_gating(const void* y, const void* w, const void* x, int n, int k, int N, void* out,
                      const void* status, hipStream_t stream);
int moe_mx_decode_check(int E, int H, int I, int nk);
int moe_decode_spin_limit_exchange(int polls);
int moe_launch_mx_decode(const void* t_packed, int n, const void* indptr,
                         const void* sorted_pairs, int k_top, const void* blocks1,
                         const void* scales1, const void* bias1, const void* blocks2,
                         const void* scales2, const void* bias2, int E, int H, int I, int nk,
                         float alpha, float limit, void* act_packed, void* y, void* done,
                         void* status, const void* w, const void* x, void* out, void* arrive,
                         const void* logits, void* idx, void* route_w, void* const* route,
                         hipStream_t stream);
int moe_mx_token1_check(int E, int k, int H, int I);
int moe_launch_mx_token1_mlp1(const void* t_packed, const void* logits, int E,
                              void* const* route, const void* blocks, const void* scales,
                              const void* bias, int k, int H, int I, float alpha, float limit,
                              void* act_packed, hipStream_t stream);
int moe_launch_mx_token1_mlp2(const void* act_packed, const void* logits, int E, const void* x,
                              const void* blocks, const void* scales, const void* bias, int k,
                              int H, int I, void* out, hipStream_t stream);
int moe_launch_swiglu(const void* x, int64_t pairs, float alpha, float limit, void* out,
                      hipStream_t stream);
int moe_launch_hbm_read(const void* src, size_t bytes, int grid, int unroll, uint32_t* sink,
                        hipStream_t stream);
}

namespace {

constexpr int64_t kMaxK = 3072;  // reduction length limit (24 MFMA chunks of 128)

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline hipStream_t as_stream(moe_stream_t s) { return (hipStream_t)s; }

// Common shape checks of the block: see the header's "Supported shapes".
int check_dims(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I) {
  if (n < 0 || H <= 0 || I <= 0) return MOE_ERR_SHAPE;
  if (H % 64 || I % 32 || H > kMaxK || I > kMaxK) return MOE_ERR_SHAPE;
  if (k < 1 || k > 8 || E < k || E > 256) return MOE_ERR_UNSUPPORTED;
  if (n * k >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  return MOE_OK;
}

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Expert matmul dispatch (model/mlp_optimized.py:94-107 picks prefill or
// decode kernels by token count): the tiled GEMM once the experts average
// kGemmMinTokens or more tokens (each weight tile then serves many tokens),
// the grouped GEMV below that or when N is not a multiple of its tile.
constexpr int64_t kGemmMinTokens = 48;

// The decode launch combines a token's k mlp2 rows itself (the last of its k
// tiles to arrive sums them) up to this many tokens; above it a separate
// gating kernel is faster: the combine's device-scope round trips (arrival
// count, then the y rows) sit at the launch's tail.
constexpr int64_t kFusedCombineMaxTokens = 32;

// The decode launch (mlp1, act's encoding and mlp2 in one persistent launch)
// from this many tokens up.  One token takes separate launches (mlp1 GEMV,
// mlp2 GEMV encoding act while staging it, gating kernel): its mlp1 is a
// few tiles per workgroup, so the launch's chain of device-scope round trips
// (act stored, count published, count polled, act staged) costs more than a
// kernel boundary (block 32.0 us against 34.5; two tokens 42.9 against 43.2,
// three 52.1 against 50.4, the launch ahead from there on).
constexpr int64_t kDecodeLaunchMinTokens = 2;

// moe_block_forward_marked: the caller's hipEvents recorded on the block's
// stream before its first launch and after each stage (MOE_STAGE_*).
constexpr int kMaxMarks = 8;
struct Marks {
  hipEvent_t const* ev;
  int used;
  int32_t stage[kMaxMarks];
};

inline int mark(Marks* m, int stage, hipStream_t s) {
  if (!m) return MOE_OK;
  if (m->used >= kMaxMarks) return MOE_ERR_SHAPE;
  if (hipEventRecord(m->ev[m->used], s) != hipSuccess) return MOE_ERR_LAUNCH;
  m->stage[m->used++] = stage;
  return MOE_OK;
}

int expert_matmul(const void* packed, int rows, int pieces, const int32_t* indptr,
                  const int32_t* sorted_pairs, int k_top, int arow_mode, int orow_mode,
                  const void* blocks, const void* scales, const void* bias, int E, int N, int K,
                  int max_tokens, int pairs, int swiglu, float alpha, float limit, void* out,
                  int out_ld, hipStream_t s) {
  // the GEMM stores 16-byte row pieces and loads the bias 16 bytes at a time
  if ((int64_t)pairs >= kGemmMinTokens * E && ((uintptr_t)out & 15u) == 0 && out_ld % 4 == 0 &&
      ((uintptr_t)bias & 15u) == 0) {
    const int rc = moe_launch_mx_gemm(packed, rows, pieces, indptr, sorted_pairs, k_top,
                                      arow_mode, orow_mode, blocks, scales, bias, E, N, K, pairs,
                                      swiglu, alpha, limit, out, out_ld, nullptr, s);
    if (rc != MOE_ERR_UNSUPPORTED) return rc;
  }
  return moe_launch_mx_gemv(packed, rows, pieces, indptr, sorted_pairs, k_top, arow_mode,
                            orow_mode, blocks, scales, bias, E, N, K, max_tokens, pairs, swiglu,
                            alpha, limit, out, out_ld, s);
}

// Bytes [0, kCounterBytes) of the block workspace, at the same place for
// every n: counters that are zero before the first call and that every call
// leaves at zero (int 0: the router launch's finished workgroups).
constexpr size_t kCounterBytes = 256;
constexpr int kCounterRouter = 0;

constexpr int kNumRegions = 15;
constexpr int kRegionSync = 14;  // decode launch: E completion counts, then the status word
constexpr int kPiecesT = 2;    // fp8 pieces of the bf16 normalised tokens (exact)
// fp8 pieces of the fp32 SwiGLU output act, mlp2's operand: three carry
// about 12 significant bits (relative to each 32-block's largest magnitude),
// adding ~2e-5 of max |y| to y and far less than the bf16 rounding of the
// block output, while mlp2 stages and multiplies a quarter less than with
// four.  moe_einsum_fused keeps four pieces for fp32 x (about 16 bits).
constexpr int kPiecesAct = 3;
constexpr int kPiecesF32 = 4;

// The fp32 act rows have a region of their own only where mlp2 reads them
// while writing y (at most two pairs per expert: the GEMV encodes act while
// staging it).  Otherwise act, when a path writes it at all, is last read by
// the pieces kernel before mlp2 starts, and shares y's bytes (y holds
// max(H, I) columns' worth).
void layout(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I, size_t off[kNumRegions],
            size_t* total) {
  const size_t nk = (size_t)n * (size_t)k;
  const bool own_act = (int64_t)nk <= 2 * E;
  const size_t sizes[kNumRegions] = {
      (size_t)n * H * 2,      // t        bf16 [n, H]
      nk * 4,                 // idx      int32 [n, k]
      nk * 2,                 // w        bf16 [n, k]
      (size_t)(E + 1) * 4,    // indptr   int32 [E+1]
      nk * 4,                 // sorted_pairs
      nk * 4,                 // token_indices
      nk * 4,                 // expert_ids
      nk * 4,                 // pair_pos
      moe_pieces_total_bytes(n, H, kPiecesT),          // t_pieces
      own_act ? nk * (size_t)I * 4 : 0,                // act      fp32 [n*k, I]
      moe_pieces_total_bytes((int64_t)nk, I, kPiecesAct),  // act_pieces
      nk * (size_t)std::max(H, I) * 4,                 // y        fp32 [n*k, H]
      (size_t)n * E * 4,      // logits   fp32 [n, E] (bf16 values)
      // counts int32: [chunks of 16 tokens, E] (the grouping above 128
      // tokens), or [n, H / 16] (the decode launch's arrival counts)
      std::max((size_t)moe_select_chunks((int)n) * E,
               n <= kFusedCombineMaxTokens ? (size_t)n * (H / 16) : 0) * 4,
      // sync int32 [E + 1]: the decode launch's per-expert mlp1 completion
      // counts and its status word (zeroed by the logits kernel)
      (size_t)(E + 1) * 4,
  };
  size_t o = kCounterBytes;
  for (int i = 0; i < kNumRegions; ++i) {
    off[i] = o;
    o = round_up(o + sizes[i], 256);
  }
  if (!own_act) off[9] = off[11];
  *total = o;
}

// mlp1 + SwiGLU with act written as its three fp8 pieces (rows by sorted
// position).  With the tiled GEMM (48 or more pairs per expert on average)
// the epilogue encodes act directly (a 192-column tile holds whole
// 32-element blocks of act): no fp32 act round trip and no encoding pass.
// Otherwise the grouped GEMV writes fp32 act and the pieces kernel encodes it.
int mlp1_pieces(const void* t_pk, int64_t n, int64_t k, int64_t E, int64_t H, int64_t I,
                const int32_t* indptr, const int32_t* sp, const void* blocks, const void* scales,
                const void* bias, float alpha, float limit, float* act, void* act_pk,
                hipStream_t s) {
  const int nk = (int)(n * k);
  int rc;
  if ((int64_t)nk >= kGemmMinTokens * E && ((uintptr_t)bias & 15u) == 0) {
    rc = moe_launch_mx_gemm(t_pk, (int)n, kPiecesT, indptr, sp, (int)k, 0, 1, blocks, scales,
                            bias, (int)E, (int)(2 * I), (int)H, nk, 2, alpha, limit, act_pk,
                            (int)I, (char*)act_pk + moe_pieces_q_bytes(nk, I, kPiecesAct), s);
    if (rc != MOE_ERR_UNSUPPORTED) return rc;
  }
  if ((rc = expert_matmul(t_pk, (int)n, kPiecesT, indptr, sp, (int)k, 0, 1, blocks, scales, bias,
                          (int)E, (int)(2 * I), (int)H, (int)n, nk, 1, alpha, limit, act, (int)I,
                          s)))
    return rc;
  return moe_launch_pieces(act, 1, nk, (int)I, kPiecesAct, act_pk, s);
}

}  // namespace

extern "C" {

int moe_version(void) { return 200; }

const char* moe_status_string(int status) {
  switch (status) {
    case MOE_OK: return "ok";
    case MOE_ERR_NULL: return "null pointer";
    case MOE_ERR_SHAPE: return "unsupported or inconsistent shape";
    case MOE_ERR_ALIGN: return "pointer not 16-byte aligned";
    case MOE_ERR_UNSUPPORTED: return "unsupported parameter value";
    case MOE_ERR_LAUNCH: return "kernel launch failed";
    case MOE_ERR_WORKSPACE: return "workspace too small";
    case MOE_ERR_TOO_LARGE:
      return "n too large for moe_block_forward_noalloc's static scratch (48 MiB)";
    case MOE_ERR_INCOMPLETE:
      return "the decode launch's bounded wait gave up: outputs are NaN";
    default: return "unknown status";
  }
}

static int dequant_common(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                          int64_t rows, int fast, moe_stream_t stream) {
  if (rows < 0 || rows > ((int64_t)1 << 36)) return MOE_ERR_SHAPE;
  if (rows == 0) return MOE_OK;
  if (!blocks || !scales || !out) return MOE_ERR_NULL;
  if (!aligned16(blocks) || !aligned16(out)) return MOE_ERR_ALIGN;
  return moe_launch_dequant(blocks, scales, out, rows, fast, as_stream(stream));
}

int moe_dequant_mxfp4(const uint8_t* blocks, const uint8_t* scales, uint16_t* out, int64_t rows,
                      moe_stream_t stream) {
  return dequant_common(blocks, scales, out, rows, 0, stream);
}

int moe_dequant_mxfp4_fast(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                           int64_t rows, moe_stream_t stream) {
  return dequant_common(blocks, scales, out, rows, 1, stream);
}

int moe_router_topk(const uint16_t* x, const uint16_t* norm_w, const uint16_t* gate_w,
                    const uint16_t* gate_b, int64_t n, int64_t H, int64_t E, int64_t k, float eps,
                    uint16_t* t, int32_t* idx, uint16_t* w, moe_stream_t stream) {
  if (n < 0 || H <= 0 || H % 8 || H > 4096 || n >= ((int64_t)1 << 31) / 8) return MOE_ERR_SHAPE;
  if (k < 1 || k > 8 || E < k || E > 256) return MOE_ERR_UNSUPPORTED;
  if (n == 0) return MOE_OK;
  if (!x || !norm_w || !gate_w || !gate_b || !t || !idx || !w) return MOE_ERR_NULL;
  if (!aligned16(x) || !aligned16(norm_w) || !aligned16(gate_w) || !aligned16(t))
    return MOE_ERR_ALIGN;
  return moe_launch_router(x, norm_w, gate_w, gate_b, (int)n, (int)H, (int)E, (int)k, eps, t, idx,
                           w, as_stream(stream));
}

int moe_permute(const int32_t* idx, int64_t n, int64_t k, int64_t E, int32_t* indptr,
                int32_t* sorted_pairs, int32_t* token_indices, int32_t* expert_ids,
                int32_t* pair_pos, moe_stream_t stream) {
  if (n < 0 || k < 1 || k > 8 || n * k >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  if (E < 1 || E > 256) return MOE_ERR_UNSUPPORTED;
  if (!indptr) return MOE_ERR_NULL;
  if (n > 0 && (!idx || !sorted_pairs || !token_indices || !expert_ids || !pair_pos))
    return MOE_ERR_NULL;
  return moe_launch_permute(idx, (int)(n * k), (int)k, (int)E, indptr, sorted_pairs, token_indices,
                            expert_ids, pair_pos, as_stream(stream));
}

static size_t einsum_grouping_bytes(int64_t n, int64_t k, int64_t E) {
  const size_t nk = (size_t)n * (size_t)k;
  return round_up((size_t)(E + 1) * 4, 256) + 4 * round_up(nk * 4, 256);
}

size_t moe_einsum_workspace_bytes(int64_t n, int64_t k, int64_t E, int64_t K, int x_is_3d_f32) {
  if (n < 0 || k < 1 || E < 1 || K < 0) return 0;
  const int64_t rows = x_is_3d_f32 ? n * k : n;
  return einsum_grouping_bytes(n, k, E) +
         moe_pieces_total_bytes(rows, K, x_is_3d_f32 ? kPiecesF32 : kPiecesT);
}

// Output rows per expert matmul come in 16-row tiles.
static int check_matmul(int64_t n, int64_t k, int64_t E, int64_t N, int64_t K) {
  if (n < 0 || N <= 0 || K <= 0 || N % 16 || K % 32 || K > kMaxK) return MOE_ERR_SHAPE;
  if (k < 1 || k > 8 || E < k || E > 256) return MOE_ERR_UNSUPPORTED;
  if (n * k >= ((int64_t)1 << 31) || N * E >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  return MOE_OK;
}

int moe_einsum_fused(const void* x, int x_is_3d_f32, const int32_t* expert_indices, int64_t n,
                     int64_t k, int64_t E, int64_t N, int64_t K, const uint8_t* blocks,
                     const uint8_t* scales, const uint16_t* bias, float* out, void* workspace,
                     size_t workspace_bytes, moe_stream_t stream) {
  int rc = check_matmul(n, k, E, N, K);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!x || !expert_indices || !blocks || !scales || !bias || !out || !workspace) return MOE_ERR_NULL;
  if (!aligned16(x) || !aligned16(blocks) || !aligned16(scales) || !aligned16(out) ||
      !aligned16(workspace))
    return MOE_ERR_ALIGN;
  if (workspace_bytes < moe_einsum_workspace_bytes(n, k, E, K, x_is_3d_f32))
    return MOE_ERR_WORKSPACE;
  const size_t nk = (size_t)n * (size_t)k;
  char* ws = (char*)workspace;
  int32_t* indptr = (int32_t*)ws;
  ws += round_up((size_t)(E + 1) * 4, 256);
  const size_t seg = round_up(nk * 4, 256);
  int32_t* sp = (int32_t*)ws;
  int32_t* ti = (int32_t*)(ws + seg);
  int32_t* ei = (int32_t*)(ws + 2 * seg);
  int32_t* pp = (int32_t*)(ws + 3 * seg);
  void* packed = ws + 4 * seg;
  hipStream_t s = as_stream(stream);
  rc = moe_launch_permute(expert_indices, (int)nk, (int)k, (int)E, indptr, sp, ti, ei, pp, s);
  if (rc) return rc;
  // mlp1-style: bf16 rows per token; mlp2-style: fp32 rows per pair
  const int rows = x_is_3d_f32 ? (int)nk : (int)n;
  const int pieces = x_is_3d_f32 ? kPiecesF32 : kPiecesT;
  if ((rc = moe_launch_pieces(x, x_is_3d_f32, rows, (int)K, pieces, packed, s))) return rc;
  return expert_matmul(packed, rows, pieces, indptr, sp, (int)k, x_is_3d_f32 ? 1 : 0, 0, blocks,
                       scales, bias, (int)E, (int)N, (int)K, (int)nk, (int)nk, 0, 0.f, 0.f, out,
                       (int)N, s);
}

size_t moe_pieces_bytes(int64_t rows, int64_t K, int pieces) {
  if (rows < 0 || K <= 0 || K % 32 || K > kMaxK || pieces < 2 || pieces > 4) return 0;
  return moe_pieces_total_bytes(rows, K, pieces);
}

int moe_quantize_pieces(const void* x, int x_is_f32, int64_t rows, int64_t K, int pieces,
                        void* packed, moe_stream_t stream) {
  if (rows < 0 || K <= 0 || K % 32 || K > kMaxK || rows >= ((int64_t)1 << 31) / 96)
    return MOE_ERR_SHAPE;
  if (pieces < 2 || pieces > 4 || (pieces == 3 && !x_is_f32)) return MOE_ERR_UNSUPPORTED;
  if (rows == 0) return MOE_OK;
  if (!x || !packed) return MOE_ERR_NULL;
  if (!aligned16(x) || !aligned16(packed)) return MOE_ERR_ALIGN;
  return moe_launch_pieces(x, x_is_f32, (int)rows, (int)K, pieces, packed, as_stream(stream));
}

int moe_mlp1_swiglu(const void* t_pieces, const int32_t* indptr, const int32_t* sorted_pairs,
                    int64_t n, int64_t k, int64_t E, int64_t H, int64_t I, const uint8_t* blocks,
                    const uint8_t* scales, const uint16_t* bias, float alpha, float limit,
                    float* act, moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!t_pieces || !indptr || !sorted_pairs || !blocks || !scales || !bias || !act)
    return MOE_ERR_NULL;
  if (!aligned16(t_pieces) || !aligned16(blocks) || ((uintptr_t)act & 3u)) return MOE_ERR_ALIGN;
  return expert_matmul(t_pieces, (int)n, kPiecesT, indptr, sorted_pairs, (int)k, 0, 1, blocks,
                       scales, bias, (int)E, (int)(2 * I), (int)H, (int)(n * k), (int)(n * k), 1,
                       alpha, limit, act, (int)I, as_stream(stream));
}

int moe_mlp1_swiglu_pieces(const void* t_pieces, const int32_t* indptr,
                           const int32_t* sorted_pairs, int64_t n, int64_t k, int64_t E,
                           int64_t H, int64_t I, const uint8_t* blocks, const uint8_t* scales,
                           const uint16_t* bias, float alpha, float limit, float* act,
                           void* act_pieces, moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!t_pieces || !indptr || !sorted_pairs || !blocks || !scales || !bias || !act ||
      !act_pieces)
    return MOE_ERR_NULL;
  if (!aligned16(t_pieces) || !aligned16(blocks) || !aligned16(act) || !aligned16(act_pieces))
    return MOE_ERR_ALIGN;
  return mlp1_pieces(t_pieces, n, k, E, H, I, indptr, sorted_pairs, blocks, scales, bias, alpha,
                     limit, act, act_pieces, as_stream(stream));
}

int moe_mlp2(const void* act_pieces, const int32_t* indptr, const int32_t* sorted_pairs, int64_t n,
             int64_t k, int64_t E, int64_t H, int64_t I, const uint8_t* blocks,
             const uint8_t* scales, const uint16_t* bias, float* y, moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!act_pieces || !indptr || !sorted_pairs || !blocks || !scales || !bias || !y)
    return MOE_ERR_NULL;
  if (!aligned16(act_pieces) || !aligned16(blocks) || ((uintptr_t)y & 3u)) return MOE_ERR_ALIGN;
  return expert_matmul(act_pieces, (int)(n * k), kPiecesAct, indptr, sorted_pairs, (int)k, 2, 0,
                       blocks, scales, bias, (int)E, (int)H, (int)I, (int)(n * k), (int)(n * k), 0,
                       0.f, 0.f, y, (int)H, as_stream(stream));
}

int moe_mlp_decode(const void* t_pieces, const int32_t* indptr, const int32_t* sorted_pairs,
                   int64_t n, int64_t k, int64_t E, int64_t H, int64_t I,
                   const uint8_t* mlp1_blocks, const uint8_t* mlp1_scales,
                   const uint16_t* mlp1_bias, const uint8_t* mlp2_blocks,
                   const uint8_t* mlp2_scales, const uint16_t* mlp2_bias, float alpha,
                   float limit, void* act_pieces, int32_t* done, float* y,
                   moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (n > 128) return MOE_ERR_UNSUPPORTED;
  if (!t_pieces || !indptr || !sorted_pairs || !mlp1_blocks || !mlp1_scales || !mlp1_bias ||
      !mlp2_blocks || !mlp2_scales || !mlp2_bias || !act_pieces || !done || !y)
    return MOE_ERR_NULL;
  if (!aligned16(t_pieces) || !aligned16(mlp1_blocks) || !aligned16(mlp1_scales) ||
      !aligned16(mlp2_blocks) || !aligned16(mlp2_scales) || !aligned16(act_pieces) ||
      ((uintptr_t)y & 3u) || ((uintptr_t)done & 3u))
    return MOE_ERR_ALIGN;
  return moe_launch_mx_decode(t_pieces, (int)n, indptr, sorted_pairs, (int)k, mlp1_blocks,
                              mlp1_scales, mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias, (int)E,
                              (int)H, (int)I, (int)(n * k), alpha, limit, act_pieces, y, done,
                              done + E, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                              nullptr, nullptr, as_stream(stream));
}

int moe_gemv_gating(const float* y, const uint16_t* w, const uint16_t* x, int64_t n, int64_t k,
                    int64_t N, uint16_t* out, moe_stream_t stream) {
  if (n < 0 || k < 1 || k > 8 || N <= 0 || N % 4 || n >= ((int64_t)1 << 31) / 8 ||
      N >= ((int64_t)1 << 28))
    return MOE_ERR_SHAPE;
  if (n == 0) return MOE_OK;
  if (!y || !w || !out) return MOE_ERR_NULL;
  if (!aligned16(y) || ((uintptr_t)out & 7u) || (x && ((uintptr_t)x & 7u))) return MOE_ERR_ALIGN;
  return moe_launch_gating(y, w, x, (int)n, (int)k, (int)N, out, nullptr, as_stream(stream));
}

int moe_swiglu(const float* x, int64_t rows, int64_t d, float alpha, float limit, float* out,
               moe_stream_t stream) {
  if (rows < 0 || d < 0) return MOE_ERR_SHAPE;
  if (rows == 0 || d == 0) return MOE_OK;
  if (!x || !out) return MOE_ERR_NULL;
  if ((uintptr_t)x & 7u) return MOE_ERR_ALIGN;
  return moe_launch_swiglu(x, rows * d, alpha, limit, out, as_stream(stream));
}

size_t moe_workspace_bytes(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I) {
  if (check_dims(n, E, k, H, I)) return 0;
  size_t off[kNumRegions], total;
  layout(n, E, k, H, I, off, &total);
  return total;
}

int moe_workspace_layout(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I,
                         size_t offsets[15]) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (!offsets) return MOE_ERR_NULL;
  size_t total;
  layout(n, E, k, H, I, offsets, &total);
  return MOE_OK;
}

}  // extern "C"

namespace {

static int block_forward_impl(const uint16_t* x, int64_t n, int64_t E, int64_t k, int64_t H,
                              int64_t I, const uint16_t* norm_w, const uint16_t* gate_w,
                              const uint16_t* gate_b, const uint8_t* mlp1_blocks,
                              const uint8_t* mlp1_scales, const uint16_t* mlp1_bias,
                              const uint8_t* mlp2_blocks, const uint8_t* mlp2_scales,
                              const uint16_t* mlp2_bias, float eps, float alpha, float limit,
                              uint16_t* out, void* workspace, size_t workspace_bytes,
                              moe_stream_t stream, Marks* m) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!x || !norm_w || !gate_w || !gate_b || !mlp1_blocks || !mlp1_scales || !mlp1_bias ||
      !mlp2_blocks || !mlp2_scales || !mlp2_bias || !out || !workspace)
    return MOE_ERR_NULL;
  if (!aligned16(x) || !aligned16(norm_w) || !aligned16(gate_w) || !aligned16(mlp1_blocks) ||
      !aligned16(mlp1_scales) || !aligned16(mlp2_blocks) || !aligned16(mlp2_scales) ||
      ((uintptr_t)out & 7u) || ((uintptr_t)workspace & 255u))
    return MOE_ERR_ALIGN;
  size_t off[kNumRegions], total;
  layout(n, E, k, H, I, off, &total);
  if (workspace_bytes < total) return MOE_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  uint16_t* t = (uint16_t*)(ws + off[0]);
  int32_t* idx = (int32_t*)(ws + off[1]);
  uint16_t* w = (uint16_t*)(ws + off[2]);
  int32_t* indptr = (int32_t*)(ws + off[3]);
  int32_t* sp = (int32_t*)(ws + off[4]);
  int32_t* ti = (int32_t*)(ws + off[5]);
  int32_t* ei = (int32_t*)(ws + off[6]);
  int32_t* pp = (int32_t*)(ws + off[7]);
  void* t_pk = ws + off[8];
  float* act = (float*)(ws + off[9]);
  void* act_pk = ws + off[10];
  float* y = (float*)(ws + off[11]);
  hipStream_t s = as_stream(stream);
  const int nk = (int)(n * k);
  float* logits = (float*)(ws + off[12]);
  int32_t* counts = (int32_t*)(ws + off[13]);
  int32_t* sync = (int32_t*)(ws + off[kRegionSync]);  // [E] counts, [E] status
  const bool gemm = (int64_t)nk >= kGemmMinTokens * E;
  // norm, t, its pieces and the logits (and sync[0..E] = 0: the decode
  // launch's counts and status); then top-k, softmax and grouping
  void* t_qs = (char*)t_pk + moe_pieces_q_bytes(n, H, kPiecesT);
  if ((rc = mark(m, MOE_STAGE_START, s))) return rc;
  // the decode launch's arrival counts (fused combine) zeroed by the selection
  const bool decode = !gemm && n >= kDecodeLaunchMinTokens && n <= 128;
  const bool fuse = decode && n <= kFusedCombineMaxTokens;
  const int zero_ints = fuse ? (int)(n * (H / 16)) : 0;
  // One token (the shape permitting): the logits launch, then mlp1 and mlp2
  // with the gated combine, each wave on one weight tile; mlp1 writes act as
  // mlp2's three fp8 pieces (act_pk, rows slot 3 + piece); both route the
  // token themselves from its logits, and mlp1's first workgroup writes idx,
  // w and the grouping.
  if (n == 1 && !gemm && moe_mx_token1_check((int)E, (int)k, (int)H, (int)I) == MOE_OK) {
    void* const route[7] = {idx, w, indptr, sp, ti, ei, pp};
    if ((rc = moe_launch_router_logits(x, norm_w, gate_w, gate_b, (int)n, (int)H, (int)E, eps, t,
                                       logits, t_pk, t_qs, nullptr, s)) ||
        (rc = mark(m, MOE_STAGE_ROUTER_LOGITS, s)) ||
        (rc = moe_launch_mx_token1_mlp1(t_pk, logits, (int)E, route, mlp1_blocks, mlp1_scales,
                                        mlp1_bias, (int)k, (int)H, (int)I, alpha, limit, act_pk,
                                        s)) ||
        (rc = mark(m, MOE_STAGE_MLP1, s)) ||
        (rc = moe_launch_mx_token1_mlp2(act_pk, logits, (int)E, x, mlp2_blocks, mlp2_scales,
                                        mlp2_bias, (int)k, (int)H, (int)I, out, s)))
      return rc;
    return mark(m, MOE_STAGE_MLP2, s);
  }
  // From kFusedCombineMaxTokens + 1 to 128 tokens (E <= 32, the launch
  // fitting the device) the decode launch routes itself: the logits launch,
  // the decode launch (each workgroup ranks the logits and groups the pairs;
  // workgroup 0 writes idx, w and the grouping), the gating launch.
  if (decode && !fuse && E <= 32 && n * E <= 4096 && nk <= 512 &&
      moe_mx_decode_check((int)E, (int)H, (int)I, nk) == MOE_OK) {
    void* const grouping[3] = {ti, ei, pp};
    if ((rc = moe_launch_router_logits(x, norm_w, gate_w, gate_b, (int)n, (int)H, (int)E, eps, t,
                                       logits, t_pk, t_qs, sync, s)) ||
        (rc = mark(m, MOE_STAGE_ROUTER_LOGITS, s)) ||
        (rc = moe_launch_mx_decode(t_pk, (int)n, indptr, sp, (int)k, mlp1_blocks, mlp1_scales,
                                   mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias, (int)E,
                                   (int)H, (int)I, nk, alpha, limit, act_pk, y, sync, sync + E,
                                   nullptr, x, nullptr, counts, logits, idx, w, grouping, s)) ||
        (rc = mark(m, MOE_STAGE_DECODE, s)) ||
        (rc = moe_launch_gating(y, w, x, (int)n, (int)k, (int)H, out, sync + E, s)))
      return rc;
    return mark(m, MOE_STAGE_GATING, s);
  }
  // other decode sizes: the logits launch's last workgroup runs the selection
  // and grouping (one launch); otherwise two launches
  rc = MOE_ERR_UNSUPPORTED;
  if (!gemm && n <= 128) {
    int32_t* arrive = (int32_t*)ws + kCounterRouter;
    rc = moe_launch_router_select(x, norm_w, gate_w, gate_b, (int)n, (int)H, (int)E, (int)k, eps,
                                  t, logits, t_pk, t_qs, sync, idx, w, indptr, sp, ti, ei, pp,
                                  counts, zero_ints, arrive, s);
    if (rc == MOE_OK && (rc = mark(m, MOE_STAGE_ROUTER, s))) return rc;
  }
  if (rc == MOE_ERR_UNSUPPORTED) {
    if ((rc = moe_launch_router_logits(x, norm_w, gate_w, gate_b, (int)n, (int)H, (int)E, eps, t,
                                       logits, t_pk, t_qs, sync, s)) ||
        (rc = mark(m, MOE_STAGE_ROUTER_LOGITS, s)))
      return rc;
    if ((rc = moe_launch_select_group(logits, (int)n, (int)E, (int)k, idx, w, counts, indptr, sp,
                                      ti, ei, pp, zero_ints, s)) ||
        (rc = mark(m, MOE_STAGE_SELECT, s)))
      return rc;
  } else if (rc) {
    return rc;
  }
  // Decode (2 to 128 tokens, the shape and device fit): mlp1, the encoding of
  // act and mlp2 in one launch.
  if (decode) {
    // up to kFusedCombineMaxTokens with the gated combine: the last of a
    // token's k mlp2 tiles to arrive writes its 16 columns of out (NaN if a
    // wait gave up); above, the gating kernel (NaN rows after a give-up)
    rc = moe_launch_mx_decode(t_pk, (int)n, indptr, sp, (int)k, mlp1_blocks, mlp1_scales,
                              mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias, (int)E, (int)H,
                              (int)I, nk, alpha, limit, act_pk, y, sync, sync + E,
                              fuse ? w : nullptr, x, fuse ? out : nullptr, counts, nullptr,
                              nullptr, nullptr, nullptr, s);
    if (rc == MOE_OK && (rc = mark(m, MOE_STAGE_DECODE, s))) return rc;
    if (rc == MOE_OK && !fuse) {
      if ((rc = moe_launch_gating(y, w, x, (int)n, (int)k, (int)H, out, sync + E, s))) return rc;
      return mark(m, MOE_STAGE_GATING, s);
    }
    if (rc != MOE_ERR_UNSUPPORTED) return rc;
  }
  if (gemm) {
    if ((rc = mlp1_pieces(t_pk, n, k, E, H, I, indptr, sp, mlp1_blocks, mlp1_scales, mlp1_bias,
                          alpha, limit, act, act_pk, s)))
      return rc;
  } else if ((rc = expert_matmul(t_pk, (int)n, kPiecesT, indptr, sp, (int)k, 0, 1, mlp1_blocks,
                                 mlp1_scales, mlp1_bias, (int)E, (int)(2 * I), (int)H, (int)n, nk,
                                 1, alpha, limit, act, (int)I, s))) {
    return rc;
  }
  if ((rc = mark(m, MOE_STAGE_MLP1, s))) return rc;
  if (gemm) {
    if ((rc = expert_matmul(act_pk, nk, kPiecesAct, indptr, sp, (int)k, 2, 0, mlp2_blocks,
                            mlp2_scales, mlp2_bias, (int)E, (int)H, (int)I, (int)n, nk, 0, 0.f, 0.f,
                            y, (int)H, s)))
      return rc;
  } else if ((int64_t)nk <= 2 * E) {
    // at most two pairs per expert on average: the GEMV encodes the fp32 act
    // rows itself while staging them (one kernel less; with more tokens per
    // expert the encoding would lengthen each staging more than it saves)
    if ((rc = moe_launch_mx_gemv(act, nk, kPiecesAct, indptr, sp, (int)k, 2, 0, mlp2_blocks,
                                 mlp2_scales, mlp2_bias, (int)E, (int)H, (int)I, (int)n, nk, 2, 0.f,
                                 0.f, y, (int)H, s)))
      return rc;
  } else {
    if ((rc = moe_launch_pieces(act, 1, nk, (int)I, kPiecesAct, act_pk, s)) ||
        (rc = mark(m, MOE_STAGE_ACT_PIECES, s)))
      return rc;
    if ((rc = moe_launch_mx_gemv(act_pk, nk, kPiecesAct, indptr, sp, (int)k, 2, 0, mlp2_blocks,
                                 mlp2_scales, mlp2_bias, (int)E, (int)H, (int)I, (int)n, nk, 0, 0.f,
                                 0.f, y, (int)H, s)))
      return rc;
  }
  if ((rc = mark(m, MOE_STAGE_MLP2, s)) ||
      (rc = moe_launch_gating(y, w, x, (int)n, (int)k, (int)H, out, nullptr, s)))
    return rc;
  return mark(m, MOE_STAGE_GATING, s);
}

}  // namespace

extern "C" {

int moe_block_forward(const uint16_t* x, int64_t n, int64_t E, int64_t k, int64_t H, int64_t I,
                      const uint16_t* norm_w, const uint16_t* gate_w, const uint16_t* gate_b,
                      const uint8_t* mlp1_blocks, const uint8_t* mlp1_scales,
                      const uint16_t* mlp1_bias, const uint8_t* mlp2_blocks,
                      const uint8_t* mlp2_scales, const uint16_t* mlp2_bias, float eps,
                      float alpha, float limit, uint16_t* out, void* workspace,
                      size_t workspace_bytes, moe_stream_t stream) {
  return block_forward_impl(x, n, E, k, H, I, norm_w, gate_w, gate_b, mlp1_blocks, mlp1_scales,
                            mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias, eps, alpha, limit, out,
                            workspace, workspace_bytes, stream, nullptr);
}

int moe_block_forward_marked(const uint16_t* x, int64_t n, int64_t E, int64_t k, int64_t H,
                             int64_t I, const uint16_t* norm_w, const uint16_t* gate_w,
                             const uint16_t* gate_b, const uint8_t* mlp1_blocks,
                             const uint8_t* mlp1_scales, const uint16_t* mlp1_bias,
                             const uint8_t* mlp2_blocks, const uint8_t* mlp2_scales,
                             const uint16_t* mlp2_bias, float eps, float alpha, float limit,
                             uint16_t* out, void* workspace, size_t workspace_bytes,
                             void* const* events, int n_events, int32_t* stages, int32_t* n_marks,
                             moe_stream_t stream) {
  if (!events || !stages || !n_marks) return MOE_ERR_NULL;
  if (n_events < kMaxMarks) return MOE_ERR_SHAPE;
  Marks m{(hipEvent_t const*)events, 0, {}};
  const int rc = block_forward_impl(x, n, E, k, H, I, norm_w, gate_w, gate_b, mlp1_blocks,
                                    mlp1_scales, mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias,
                                    eps, alpha, limit, out, workspace, workspace_bytes, stream, &m);
  for (int i = 0; i < m.used; ++i) stages[i] = m.stage[i];
  *n_marks = m.used;
  return rc;
}

int moe_set_decode_spin_limit(int polls) { return moe_decode_spin_limit_exchange(polls); }

int moe_hbm_read(const void* src, size_t bytes, int grid, int unroll, uint32_t* sink,
                 moe_stream_t stream) {
  if (!src || !sink) return MOE_ERR_NULL;
  if (bytes < 16 || bytes % 16 || grid < 1 || grid > (1 << 20)) return MOE_ERR_SHAPE;
  if (!aligned16(src)) return MOE_ERR_ALIGN;
  if (unroll != 4 && unroll != 8 && unroll != 16) return MOE_ERR_UNSUPPORTED;
  return moe_launch_hbm_read(src, bytes, grid, unroll, sink, as_stream(stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// moe_block_forward_noalloc: the block with its workspace in a static device
// array instead of a caller buffer, for callers that cannot allocate.  Each
// GPU the library runs on holds its own copy of `scratch` (48 MiB) until the
// process ends.  In host code the array's name is not a device address: the
// address of this device's copy comes from hipGetSymbolAddress, looked up
// once per device with that device current, and only that address is ever
// handed to kernels.
namespace {

constexpr size_t kScratchBytes = (size_t)48 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<uintptr_t> g_scratch_addr[kMaxDevices];  // 0: not looked up yet

// Zeroes the workspace counters (a kernel, not a memset: the first call may
// be captured in a graph).
__global__ void zero_counters_kernel(uint32_t* p) { p[threadIdx.x] = 0u; }

// Device address of the current device's scratch; the first lookup on a
// device also zeroes the scratch's counters on `s`, ahead of the call's
// kernels.
int scratch_address(void** out, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MOE_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return MOE_ERR_UNSUPPORTED;
  uintptr_t a = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (a == 0) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return MOE_ERR_LAUNCH;
    hipLaunchKernelGGL(zero_counters_kernel, dim3(1), dim3(kCounterBytes / 4), 0, s,
                       (uint32_t*)p);
    if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    a = (uintptr_t)p;
    g_scratch_addr[dev].store(a, std::memory_order_release);  // same value if raced
  }
  *out = (void*)a;
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_block_forward_noalloc(const uint16_t* x, int64_t n, int64_t E, int64_t k, int64_t H,
                              int64_t I, const uint16_t* norm_w, const uint16_t* gate_w,
                              const uint16_t* gate_b, const uint8_t* mlp1_blocks,
                              const uint8_t* mlp1_scales, const uint16_t* mlp1_bias,
                              const uint8_t* mlp2_blocks, const uint8_t* mlp2_scales,
                              const uint16_t* mlp2_bias, float eps, float alpha, float limit,
                              uint16_t* out, moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  size_t off[kNumRegions], total;
  layout(n, E, k, H, I, off, &total);
  if (total > kScratchBytes) return MOE_ERR_TOO_LARGE;
  void* ws = nullptr;
  if ((rc = scratch_address(&ws, as_stream(stream)))) return rc;
  // every region the kernels read is written earlier in the same call (the
  // per-call counters are zeroed by the first kernel, the persistent ones are
  // left at zero by every call), so stale contents of the last call do no harm
  return moe_block_forward(x, n, E, k, H, I, norm_w, gate_w, gate_b, mlp1_blocks, mlp1_scales,
                           mlp1_bias, mlp2_blocks, mlp2_scales, mlp2_bias, eps, alpha, limit, out,
                           ws, kScratchBytes, stream);
}

int moe_block_status(const void* workspace, int64_t n, int64_t E, int64_t k, int64_t H,
                     int64_t I, moe_stream_t stream) {
  int rc = check_dims(n, E, k, H, I);
  if (rc) return rc;
  if (n == 0) return MOE_OK;
  if (!workspace) return MOE_ERR_NULL;
  size_t off[kNumRegions], total;
  layout(n, E, k, H, I, off, &total);
  int32_t status = 0;
  hipStream_t s = as_stream(stream);
  if (hipMemcpyAsync(&status, (const char*)workspace + off[kRegionSync] + (size_t)E * 4, 4,
                     hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return MOE_ERR_LAUNCH;
  return status == 0 ? MOE_OK : MOE_ERR_INCOMPLETE;
}

}  // extern "C"
