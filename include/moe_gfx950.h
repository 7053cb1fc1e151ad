/*
 * libmoe_gfx950 -- C ABI of the MI355X (gfx950) MXFP4 mixture-of-experts block.
 *
 * Every entry point replaces one operator of the reference MoE path
 * (brekkylab/gpt-oss-tvm); the citation above each declaration names the
 * reference operator and where it is defined or called.  The reference's
 * operators are destination-passing TIR prim_funcs called through
 * nn.tensor_ir_op: the caller (Relax VM) owns every output and the kernel
 * allocates nothing.  These entry points keep that contract:
 *
 *   - all buffers are caller-owned device pointers; outputs come last but one;
 *   - nothing is allocated and the host never waits on the device, so every
 *     call can be captured in a HIP graph;
 *   - the last argument is the HIP stream (hipStream_t) to launch on, NULL for
 *     the default stream;
 *   - the return value is MOE_OK or a negative MOE_ERR_* code; on error no
 *     kernel was launched and no output was written.  Nothing throws across
 *     the ABI.  One failure can only be seen after the kernels ran: the
 *     decode launch (moe_mlp_decode, and moe_block_forward for n <= 128)
 *     waits for other workgroups of its own launch, and if that bounded wait
 *     gives up it reports so in a device status word; the block then writes
 *     NaN to the output (every element above 32 tokens; up to 32 tokens, where
 *     the launch combines each token's rows itself as they complete, every
 *     element combined after the give-up, which includes every element that
 *     the given-up work fed) and moe_block_status() returns
 *     MOE_ERR_INCOMPLETE: treat the whole output as invalid.
 *
 * Tensor conventions: bf16 tensors are uint16_t bit patterns, row-major,
 * 16-byte aligned.  MXFP4 weights stay in the checkpoint layout of
 * model/mlp.py:100-144: blocks uint8 [E, N, K/32, 16] (element 2j of a block
 * in the low nibble of byte j), scales uint8 E8M0 [E, N, K/32], bias bf16
 * [E, N].  H = hidden size, I = intermediate size, E = experts, k = experts
 * per token, n = tokens.
 *
 * Supported shapes: H % 64 == 0, I % 32 == 0, H <= 3072, I <= 3072,
 * 1 <= k <= 8, k <= E <= 256, 0 <= n and n*k < 2^31.
 *
 * Threading: stateless and re-entrant; calls on one stream execute in order.
 */
#ifndef MOE_GFX950_H_
#define MOE_GFX950_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_NULL (-1)        /* a required pointer is NULL */
#define MOE_ERR_SHAPE (-2)       /* unsupported or inconsistent shape */
#define MOE_ERR_ALIGN (-3)       /* a pointer is not 16-byte aligned */
#define MOE_ERR_UNSUPPORTED (-4) /* valid but unsupported parameter value */
#define MOE_ERR_LAUNCH (-5)      /* the HIP runtime rejected a launch */
#define MOE_ERR_WORKSPACE (-6)   /* workspace smaller than moe_workspace_bytes() */
#define MOE_ERR_INCOMPLETE (-7)  /* the decode launch's bounded wait gave up (outputs are NaN) */
#define MOE_ERR_TOO_LARGE (-8)   /* beyond moe_block_forward_noalloc's static scratch */

typedef void* moe_stream_t; /* a hipStream_t */

#if defined(__GNUC__)
#define MOE_API __attribute__((visibility("default")))
#else
#define MOE_API
#endif

/* Library version (major*10000 + minor*100 + patch). */
MOE_API int moe_version(void);

/* Static description of a status code. */
MOE_API const char* moe_status_string(int status);

/*
 * Standalone MXFP4 -> bf16 dequantisation.
 * Replaces: dequant_mxfp4, model/mlp.py:172-234 (MLPBlock.__dequantize_mxfp4_weight,
 * mlp.py:146-236).  blocks [rows, 16] u8, scales [rows] u8 E8M0 (the raw byte;
 * the reference subtracts 127 before the call, mlp.py:155), out [rows, 32] bf16.
 * Bit-exact for all 256 x 256 (byte, scale) pairs.
 */
MOE_API int moe_dequant_mxfp4(const uint8_t* blocks, const uint8_t* scales, uint16_t* out, int64_t rows,
                      moe_stream_t stream);

/*
 * The same dequantisation through the hardware conversion used inside the
 * expert matmuls (v_cvt_scalef32_pk_bf16_fp4); exposed so the fused path's
 * dequantisation can be compared with moe_dequant_mxfp4.
 * Replaces: the in-kernel LUT dequant of mxfp4_moe_mlp*_{prefill,decode},
 * model/mlp_optimized.py:324-331, 441-446, 549-554, 644-647.
 */
MOE_API int moe_dequant_mxfp4_fast(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                           int64_t rows, moe_stream_t stream);

/*
 * RMSNorm + router linear + top-k + softmax.
 * Replaces: model/mlp.py:375-382 (self.norm, self.gate, nn.op.topk, nn.op.softmax);
 * mlc-llm gating_softmax_topk as called at model/mlp_optimized.py:118,187.
 * x [n, H] bf16, norm_w [H], gate_w [E, H], gate_b [E] bf16 ->
 * t [n, H] bf16 (normalised tokens), idx [n, k] int32 (descending logit,
 * lower index on ties), w [n, k] bf16 (softmax over the k selected logits).
 */
MOE_API int moe_router_topk(const uint16_t* x, const uint16_t* norm_w, const uint16_t* gate_w,
                    const uint16_t* gate_b, int64_t n, int64_t H, int64_t E, int64_t k, float eps,
                    uint16_t* t, int32_t* idx, uint16_t* w, moe_stream_t stream);

/*
 * Expert grouping: stable counting sort of the n*k (token, slot) pairs by expert.
 * Replaces: mlc-llm moe_cumsum + get_indices + get_indptr(inclusive=False) and the
 * moe_expand_indptr prim_func, model/mlp_optimized.py:119-148.
 * idx [n, k] int32 -> indptr [E+1], sorted_pairs [n*k] (sorted position -> pair
 * p = token*k + slot), token_indices [n*k] (-> token), expert_ids [n*k]
 * (-> expert), pair_pos [n*k] (pair -> sorted position, -1 if idx was out of range).
 */
MOE_API int moe_permute(const int32_t* idx, int64_t n, int64_t k, int64_t E, int32_t* indptr,
                int32_t* sorted_pairs, int32_t* token_indices, int32_t* expert_ids,
                int32_t* pair_pos, moe_stream_t stream);

/*
 * Raw expert matmul: out[s, r, c] = bias[e, c] + sum_i x[s, (r,) i] * W_e[c, i],
 * e = expert_indices[s, r], fp32 out [n, k, N].
 * Replaces: moe_einsum_fused, model/mlp.py:267-326 (MLPBlock.run_einsum, mlp.py:238-326).
 * x is bf16 [n, K] when x_is_3d_f32 == 0 (the mlp1 call, mlp.py:387) or fp32
 * [n, k, K] when 1 (the mlp2 call, mlp.py:395).  workspace holds the grouping
 * and the fp8 pieces of x (2 for bf16 x, 4 for fp32 x, see moe_quantize_pieces):
 * at least moe_einsum_workspace_bytes(n, k, E, K, x_is_3d_f32) bytes, 16-byte
 * aligned.  N % 16 == 0, K % 32 == 0, K <= 3072.
 */
MOE_API size_t moe_einsum_workspace_bytes(int64_t n, int64_t k, int64_t E, int64_t K,
                                          int x_is_3d_f32);
MOE_API int moe_einsum_fused(const void* x, int x_is_3d_f32, const int32_t* expert_indices,
                             int64_t n, int64_t k, int64_t E, int64_t N, int64_t K,
                             const uint8_t* blocks, const uint8_t* scales, const uint16_t* bias,
                             float* out, void* workspace, size_t workspace_bytes,
                             moe_stream_t stream);

/*
 * Activation operand encoding of the expert matmuls ("pieces").  No reference
 * counterpart: the reference multiplies bf16 activations by dequantised bf16
 * weights (model/mlp_optimized.py:324-331); here the weights stay MXFP4 and
 * the matmul is gfx950's block-scaled fp4 x fp8 MFMA, whose activation
 * operand is fp8 e4m3 with one E8M0 scale per 32 elements.  Each row of x is
 * written as the sum of `pieces` fp8 rows, each quantising (round to nearest
 * even) what the earlier ones left, with the smallest scale that keeps the
 * block's codes below 256.  pieces = 2 reproduces bf16 input to within
 * 2^-14 of each 32-block's largest magnitude (exactly when a block spans at
 * most 6 binades); pieces = 3 (fp32 input only) carries about 12 significant
 * bits and pieces = 4 about 16.  x [rows, K] bf16 (x_is_f32 == 0) or fp32;
 * packed: moe_pieces_bytes(rows, K, pieces) bytes, 16-byte aligned.
 * K % 32 == 0, K <= 3072, pieces 2 or 4 (bf16 or fp32) or 3 (fp32).
 */
MOE_API size_t moe_pieces_bytes(int64_t rows, int64_t K, int pieces);
MOE_API int moe_quantize_pieces(const void* x, int x_is_f32, int64_t rows, int64_t K, int pieces,
                                void* packed, moe_stream_t stream);

/*
 * mlp1 with the interleaved clamped SwiGLU epilogue, over grouped pairs.
 * Replaces: mxfp4_moe_mlp1_{prefill,decode}, model/mlp_optimized.py:214-571, with
 * the fp32 semantics of model/mlp.py:387-390 (run_einsum + swiglu(out_dtype=float32)).
 * t_pieces: moe_quantize_pieces(t, 0, n, H, 2) of the normalised tokens t [n, H];
 * indptr/sorted_pairs from moe_permute; weights [E, 2I, H/32, 16], [E, 2I, H/32],
 * bias [E, 2I] -> act [n*k, I] fp32, row = sorted position.
 */
MOE_API int moe_mlp1_swiglu(const void* t_pieces, const int32_t* indptr,
                            const int32_t* sorted_pairs, int64_t n, int64_t k, int64_t E,
                            int64_t H, int64_t I, const uint8_t* blocks, const uint8_t* scales,
                            const uint16_t* bias, float alpha, float limit, float* act,
                            moe_stream_t stream);

/*
 * mlp1 with the SwiGLU epilogue, its output act written as the three fp8 pieces
 * moe_mlp2 takes (moe_quantize_pieces(act, 1, n*k, I, 3), rows by sorted
 * position), as moe_block_forward runs it at prefill: with 48 or more pairs
 * per expert on average the tiled GEMM's epilogue encodes act directly (act
 * is not written); below that the grouped GEMV writes act, fp32 [n*k, I]
 * (caller-owned scratch), and the encoding follows.
 * Replaces: mxfp4_moe_mlp1_prefill, model/mlp_optimized.py:214-351 (its bf16
 * act output becomes fp8 pieces here), with the fp32 semantics of
 * model/mlp.py:387-390.  act_pieces: moe_pieces_bytes(n*k, I, 3) bytes.
 */
MOE_API int moe_mlp1_swiglu_pieces(const void* t_pieces, const int32_t* indptr,
                                   const int32_t* sorted_pairs, int64_t n, int64_t k, int64_t E,
                                   int64_t H, int64_t I, const uint8_t* blocks,
                                   const uint8_t* scales, const uint16_t* bias, float alpha,
                                   float limit, float* act, void* act_pieces,
                                   moe_stream_t stream);

/*
 * mlp2 over grouped pairs.
 * Replaces: mxfp4_moe_mlp2_{prefill,decode}, model/mlp_optimized.py:353-460, 573-660,
 * with the fp32 semantics of model/mlp.py:395.
 * act_pieces: moe_quantize_pieces(act, 1, n*k, I, 3) of moe_mlp1_swiglu's output;
 * weights [E, H, I/32, 16], [E, H, I/32], bias [E, H] -> y [n*k, H] fp32,
 * row = pair p = token*k + slot.
 */
MOE_API int moe_mlp2(const void* act_pieces, const int32_t* indptr, const int32_t* sorted_pairs,
                     int64_t n, int64_t k, int64_t E, int64_t H, int64_t I,
                     const uint8_t* blocks, const uint8_t* scales, const uint16_t* bias,
                     float* y, moe_stream_t stream);

/*
 * Decode chain: mlp1 with the SwiGLU epilogue, the encoding of act and mlp2 in
 * one launch (the results of moe_mlp1_swiglu -> moe_quantize_pieces(act, 1, n*k,
 * I, 3) -> moe_mlp2, bit for bit), for n <= 128.
 * Replaces: mxfp4_moe_mlp1_decode + swiglu + mxfp4_moe_mlp2_decode,
 * model/mlp_optimized.py:214-660 (fp32 semantics of model/mlp.py:387-395).
 * t_pieces, indptr, sorted_pairs and the weights as for moe_mlp1_swiglu and
 * moe_mlp2; act_pieces: moe_pieces_bytes(n*k, I, 3) bytes, written with the
 * pieces moe_mlp2 takes; done: E + 1 int32, zero on entry (left holding the
 * per-expert tile counts in done[0..E) and the status word in done[E]) ->
 * y [n*k, H] fp32, row = pair.  MOE_ERR_UNSUPPORTED unless H == I
 * (2817..2944), n <= 128, the device has 256 or more CUs, one workgroup of the
 * launch fits on a CU, and the shape's batches fit the launch (always at
 * gpt-oss-20b's E = 32); the caller then runs the three calls.  The launch keeps
 * one workgroup on each of 256 CUs and its mlp2 phase waits for the other
 * workgroups' mlp1 results: work running on the device at the same time delays
 * it.  The wait is bounded (about a second, moe_set_decode_spin_limit); a
 * workgroup that gives up adds 1 to done[E], and the y rows it wrote are then
 * wrong: done[E] == 0 after the launch means y is complete.
 */
MOE_API int moe_mlp_decode(const void* t_pieces, const int32_t* indptr,
                           const int32_t* sorted_pairs, int64_t n, int64_t k, int64_t E,
                           int64_t H, int64_t I, const uint8_t* mlp1_blocks,
                           const uint8_t* mlp1_scales, const uint16_t* mlp1_bias,
                           const uint8_t* mlp2_blocks, const uint8_t* mlp2_scales,
                           const uint16_t* mlp2_bias, float alpha, float limit,
                           void* act_pieces, int32_t* done, float* y, moe_stream_t stream);

/*
 * Gate-weighted sum of the k expert outputs, plus the residual when x != NULL.
 * Replaces: moe_gemv_gating, model/mlp.py:340-369 (MLPBlock.run_gating, mlp.py:328-369)
 * and the residual add of mlp.py:402; the prefill combine scatter_output * w +
 * moe_sum + x of model/mlp_optimized.py:168-172.
 * y [n, k, N] fp32, w [n, k] bf16, x [n, N] bf16 or NULL -> out [n, N] bf16.
 * N % 4 == 0.
 */
MOE_API int moe_gemv_gating(const float* y, const uint16_t* w, const uint16_t* x, int64_t n, int64_t k,
                    int64_t N, uint16_t* out, moe_stream_t stream);

/*
 * Interleaved clamped SwiGLU, fp32: x [rows, 2d] -> out [rows, d].
 * Replaces: swiglu, model/mlp.py:29-60 (out_dtype float32 as called at mlp.py:390).
 */
MOE_API int moe_swiglu(const float* x, int64_t rows, int64_t d, float alpha, float limit, float* out,
               moe_stream_t stream);

/*
 * Whole block: out = x + MoE(RMSNorm(x)).
 * Replaces: MLPBlock.forward, model/mlp.py:371-402 (and model/mlp_optimized.py:94-107).
 * x [n, H] bf16 and the nine parameters in checkpoint layout (model/mlp.py:63-144)
 * -> out [n, H] bf16.  workspace: at least moe_workspace_bytes(n, E, k, H, I)
 * bytes, 256-byte aligned; its layout is given by moe_workspace_layout().
 * Its first 256 bytes hold counters that must be zero before the first call
 * (allocate the workspace zero-filled); every call leaves them at zero, so a
 * workspace can serve calls of any n, in order on one stream.  (From 2 to 32
 * tokens the router's logits launch counts its finished workgroups there and
 * the last one runs the top-k, softmax and grouping; at one token and from 33
 * to 128 tokens the launches after the logits launch route themselves.)
 */
MOE_API size_t moe_workspace_bytes(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I);

/* Byte offsets of the intermediates inside the block workspace (after the
 * 256 bytes of counters), in this order:
 * t, idx, w, indptr, sorted_pairs, token_indices, expert_ids, pair_pos,
 * t_pieces, act (fp32 [n*k, I]; where n*k > 2E it shares y's offset: its
 * last reader runs before y is written; not written by the one-token and
 * decode launches), act_pieces (at one token: rows by slot, written by the
 * mlp1 launch), y (fp32 [n*k, H], in a
 * region of n*k*max(H, I) floats), logits (fp32 [n, E], bf16 values), counts
 * (int32 [ceil(n / 16), E], expert histogram per 16-token chunk, n > 128; or
 * int32 [n, H / 16], the decode launch's arrivals per token and 16-column
 * tile of y, n <= 32), sync (int32 [E + 1]: the decode launch's per-expert
 * counts, then its status word). */
MOE_API int moe_workspace_layout(int64_t n, int64_t E, int64_t k, int64_t H, int64_t I,
                                 size_t offsets[15]);

MOE_API int moe_block_forward(const uint16_t* x, int64_t n, int64_t E, int64_t k, int64_t H, int64_t I,
                      const uint16_t* norm_w, const uint16_t* gate_w, const uint16_t* gate_b,
                      const uint8_t* mlp1_blocks, const uint8_t* mlp1_scales,
                      const uint16_t* mlp1_bias, const uint8_t* mlp2_blocks,
                      const uint8_t* mlp2_scales, const uint16_t* mlp2_bias, float eps,
                      float alpha, float limit, uint16_t* out, void* workspace,
                      size_t workspace_bytes, moe_stream_t stream);

/* Stages of moe_block_forward, in launch order; which ones run depends on n. */
#define MOE_STAGE_START 0         /* before the first launch */
#define MOE_STAGE_ROUTER_LOGITS 1 /* RMSNorm, t and its pieces, router logits */
#define MOE_STAGE_SELECT 2        /* top-k, softmax and the grouping */
#define MOE_STAGE_DECODE 3        /* mlp1 + SwiGLU + act pieces + mlp2 in one launch (+ combine, n <= 32) */
#define MOE_STAGE_MLP1 4          /* mlp1 + SwiGLU (prefill GEMM: act pieces in its epilogue) */
#define MOE_STAGE_ACT_PIECES 5    /* act's fp8 pieces (GEMV path above 2 pairs per expert) */
#define MOE_STAGE_MLP2 6          /* mlp2 (one token: with the gated combine) */
#define MOE_STAGE_GATING 7        /* gated combine + residual */
#define MOE_STAGE_ROUTER 8        /* ROUTER_LOGITS + SELECT in one launch (decode sizes) */

/*
 * moe_block_forward with the caller's hipEvents (hipEvent_t, created by the
 * caller, at least 8) recorded on `stream`: events[0] before the block's
 * first launch, then one after each stage.  stages[i] (int32, 8 entries)
 * receives the MOE_STAGE_* that events[i] closes and *n_marks the number of
 * events recorded, so the elapsed time between events[i - 1] and events[i]
 * is stage stages[i].  The launches and results are those of
 * moe_block_forward; only the event records are added.
 * No reference counterpart: a measurement hook for the block's own kernels
 * (the reference's operators are timed by TVM's profiler).
 */
MOE_API int moe_block_forward_marked(const uint16_t* x, int64_t n, int64_t E, int64_t k,
                                     int64_t H, int64_t I, const uint16_t* norm_w,
                                     const uint16_t* gate_w, const uint16_t* gate_b,
                                     const uint8_t* mlp1_blocks, const uint8_t* mlp1_scales,
                                     const uint16_t* mlp1_bias, const uint8_t* mlp2_blocks,
                                     const uint8_t* mlp2_scales, const uint16_t* mlp2_bias,
                                     float eps, float alpha, float limit, uint16_t* out,
                                     void* workspace, size_t workspace_bytes,
                                     void* const* events, int n_events, int32_t* stages,
                                     int32_t* n_marks, moe_stream_t stream);

/*
 * moe_block_forward without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  No reference counterpart: the reference's Relax VM
 * allocates every intermediate itself.  The workspace is a static device
 * array of 48 MiB held by each GPU the library runs on until the process
 * ends; nothing is allocated (no hipMalloc/hipFree) by this call.  Limit:
 * moe_workspace_bytes(n, E, k, H, I) <= 48 MiB (n <= 530 tokens at
 * gpt-oss-20b's shape, n <= 528 at 120b's), else MOE_ERR_TOO_LARGE with no
 * launch.  Same results as moe_block_forward.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams or host
 * threads) race and give wrong results; calls in order on one stream are
 * safe.  The array keeps the last call's contents, and nothing in it needs to
 * start at zero.  moe_block_status does not apply (the status word lives in
 * the static array; the outputs are NaN, as for moe_block_forward, if the
 * decode launch gave up).
 */
MOE_API int moe_block_forward_noalloc(const uint16_t* x, int64_t n, int64_t E, int64_t k,
                                      int64_t H, int64_t I, const uint16_t* norm_w,
                                      const uint16_t* gate_w, const uint16_t* gate_b,
                                      const uint8_t* mlp1_blocks, const uint8_t* mlp1_scales,
                                      const uint16_t* mlp1_bias, const uint8_t* mlp2_blocks,
                                      const uint8_t* mlp2_scales, const uint16_t* mlp2_bias,
                                      float eps, float alpha, float limit, uint16_t* out,
                                      moe_stream_t stream);

/*
 * Status of the last moe_block_forward that used this workspace (same shape
 * arguments): MOE_OK, or MOE_ERR_INCOMPLETE when its decode launch's bounded
 * wait gave up (the outputs of that call are NaN).  Unlike every other entry
 * point this one waits: it synchronises `stream` to read the status word.
 * No reference counterpart: TVM's kernels have no cross-workgroup waits
 * (model/mlp_optimized.py:214-660 launches each stage separately).
 */
MOE_API int moe_block_status(const void* workspace, int64_t n, int64_t E, int64_t k, int64_t H,
                             int64_t I, moe_stream_t stream);

/*
 * Bound of the decode launch's wait in polls (about 1 us each; default 2^20,
 * a negative value restores it).  Returns the previous bound.  Process-wide;
 * meant for tests, which set 0 to make every wait give up at once and check
 * that the failure is reported.  No reference counterpart (as above).
 */
MOE_API int moe_set_decode_spin_limit(int polls);

/*
 * Streaming read of `bytes` (a multiple of 16, 16-byte aligned) at src by
 * `grid` workgroups of 256 threads, each thread `unroll` (4, 8 or 16)
 * 16-byte loads in flight per iteration; sink: `grid` uint32 (written only in
 * the unlikely case the data fold to a fixed constant).  No reference
 * counterpart: the achievable-HBM-bandwidth calibration the kernels' HBM
 * fractions are read against.
 */
MOE_API int moe_hbm_read(const void* src, size_t bytes, int grid, int unroll, uint32_t* sink,
                         moe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_GFX950_H_ */
