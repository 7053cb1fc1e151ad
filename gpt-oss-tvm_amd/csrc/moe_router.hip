// Fused RMSNorm + router GEMV + top-k + softmax, and the expert-grouping pass.
//
// Router: model/mlp.py:375-382 (norm -> gate -> topk -> softmax); the decode
// variant's gating_softmax_topk call is model/mlp_optimized.py:187.
// Grouping: mlc-llm moe_cumsum / get_indices / get_indptr / moe_expand_indptr
// as called at model/mlp_optimized.py:119-148.
#include <algorithm>
#include <climits>
#include <cstdlib>

#include "moe_common.h"
#include "moe_select.h"

namespace moe {

// Unpack the eight bf16 of a 16-byte chunk to fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = bf2f((uint16_t)(v[d] & 0xFFFFu));
    f[2 * d + 1] = bf2f((uint16_t)(v[d] >> 16));
  }
}

// Router: TT consecutive tokens per workgroup of W waves.  Wave w owns experts
// e = w, w + W, ... and needs no other wave until the top-k:
//  1  every lane issues its loads at once: chunks c = lane + 64 i (i < S) of
//     the TT token rows and the norm weight, and the first KE gate rows it
//     owns;
//  2  per token, fp64 sum of squares per lane, fixed-order wave tree (each
//     wave computes the norms itself); r = fp32(1 / sqrt(ss / H + eps));
//     t = bf16(x * r * w), kept packed; wave 0 writes t;
//  3  the (token, chunk slot) pairs are shared out over the waves for the
//     two fp8 pieces of t: the four lanes of a 32-element block share its
//     maximum by lane exchange (same encoding as moe_pieces_kernel);
//  4  per owned expert and token, the dot of t and the gate row: every
//     product of two bf16 values is exact in fp32 and is added in fp64, per
//     lane, then by a fixed-order wave tree (the next batch of gate rows loads
//     meanwhile); logit = bf16(bf16(fp32(dot)) + bias) into LDS;
//  5  wave j < TT ranks token j's logits by (value descending, expert
//     ascending); the k winners' fp64 exponentials are summed in rank order
//     and normalised.
// A product below 2^-126 in magnitude is rounded to an fp32 subnormal; no
// logit above 2^-100 can change by it.
template <bool kPieces, int S, int W, int TT, int KE>
__global__ __launch_bounds__(64 * W) void moe_router_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
    const uint16_t* __restrict__ gate_w, const uint16_t* __restrict__ gate_b, int n, int H, int E,
    int k, float eps, uint16_t* __restrict__ t_out, int32_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out, uint8_t* __restrict__ pq, uint8_t* __restrict__ pqs) {
  __shared__ float logit[TT][256];
  __shared__ double topv[TT][8];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok0 = blockIdx.x * TT;
  const int ntok = min(TT, n - tok0);
  const int H8 = H >> 3;
  const int NC = (H + 127) >> 7;
  const u32x4* nr = (const u32x4*)norm_w;

  // rows past n repeat the last token (computed, never stored)
  u32x4 xv[TT][S], wv[S];
#pragma unroll
  for (int i = 0; i < S; ++i) wv[i] = nr[min(lane + 64 * i, H8 - 1)];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const u32x4* xr = (const u32x4*)(x + (size_t)min(tok0 + tt, n - 1) * H);
#pragma unroll
    for (int i = 0; i < S; ++i) xv[tt][i] = xr[min(lane + 64 * i, H8 - 1)];
  }
  const int nown = (E - wave + W - 1) / W;  // experts owned by this wave (may be 0)
  const int Epad = (E + 31) & ~31;
  for (int u = threadIdx.x; u < TT * 256; u += 64 * W) {
    const int e = u & 255;
    if (e >= E && e < Epad) logit[u >> 8][e] = -INFINITY;
  }
  u32x4 gv[KE][S];
  auto load_gate = [&](int eb) {
#pragma unroll
    for (int b = 0; b < KE; ++b) {
      // a wave owning no expert still issues the batch (a valid row)
      const int e = max(0, min(wave + W * min(eb + b, nown - 1), E - 1));
      const u32x4* gr = (const u32x4*)(gate_w + (size_t)e * H);
#pragma unroll
      for (int i = 0; i < S; ++i) gv[b][i] = gr[min(lane + 64 * i, H8 - 1)];
    }
  };
  load_gate(0);  // in flight during the norms

  u32x4 tp[TT][S];  // t, packed bf16 (zero past H)
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (lane + 64 * i < H8) {
        float f[8];
        unpack8(xv[tt][i], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
      }
    }
    ss = wave_sum_f64(ss);
    const float rn = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
    const int tok = tok0 + tt;
    // unpack x again below rather than holding 8 S floats across the tree
#pragma unroll
    for (int i = 0; i < S; ++i) asm volatile("" : "+v"(xv[tt][i]));
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int c = lane + 64 * i;
      float f[8], g[8];
      unpack8(xv[tt][i], f);
      unpack8(wv[i], g);
      u32x4 o;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint16_t lo = f2bf(__fmul_rn(__fmul_rn(f[2 * d], rn), g[2 * d]));
        const uint16_t hi = f2bf(__fmul_rn(__fmul_rn(f[2 * d + 1], rn), g[2 * d + 1]));
        o[d] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      const bool in = c < H8;
#pragma unroll
      for (int d = 0; d < 4; ++d) tp[tt][i][d] = in ? o[d] : 0u;
      if (wave == 0 && in && tt < ntok) ((u32x4*)(t_out + (size_t)tok * H))[c] = o;
      if constexpr (kPieces) {
        // a quad (32-element block) lies wholly inside or outside [0, 16 * NC)
        // because H % 32 == 0
        if ((tt * S + i) % W == wave && tt < ntok && c < 16 * NC) {
          const int blk = c >> 2, quarter = c & 3;
          const int ch = blk >> 2, gg = blk & 3;
          const int Kp = NC * 128;
          float rr[8];
          unpack8(tp[tt][i], rr);
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(rr[q]));
            amax = fmaxf(amax, lane_xor1(amax));
            amax = fmaxf(amax, lane_xor2(amax));
            const uint32_t sc = e8m0_for_amax(amax);
            const float inv = __uint_as_float((254u - sc) << 23);
            const float scf = sc ? __uint_as_float(sc << 23) : __uint_as_float(0x00400000u);
            uint32_t lo, hi;
            e4m3_piece8(rr, inv, scf, lo, hi);
            const size_t prow = (size_t)tok * 2 + p;
            *(uint2*)(pq + prow * Kp + c * 8) = make_uint2(lo, hi);
            if (quarter == 0) {
              uint8_t* run = pqs + prow * 112 + gg * 28;
              run[ch] = (uint8_t)sc;
              if (ch == NC - 1)
                for (int z = NC; z < 28; ++z) run[z] = 0;
            }
          }
        }
      }
    }
  }

  for (int eb = 0; eb < nown; eb += KE) {
    // t stays packed: the opaque copy keeps its unpacking inside the loop
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int i = 0; i < S; ++i) asm volatile("" : "+v"(tp[tt][i]));
    double acc[KE][TT];
#pragma unroll
    for (int b = 0; b < KE; ++b) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = 0.0;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        float gf[8];
        unpack8(gv[b][i], gf);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          float tf[8];
          unpack8(tp[tt][i], tf);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[b][tt] += (double)__fmul_rn(tf[q], gf[q]);
        }
      }
    }
    if (eb + KE < nown) load_gate(eb + KE);  // next rows load during the trees
#pragma unroll
    for (int b = 0; b < KE; ++b)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[b][tt] = wave_sum_f64(acc[b][tt]);
    // lane b * TT + tt stores expert (eb + b)'s logit for token tt
    if (lane < KE * TT) {
      const int b = lane / TT, tt = lane - b * TT;
      double a = acc[0][0];
#pragma unroll
      for (int bb = 0; bb < KE; ++bb)
#pragma unroll
        for (int t2 = 0; t2 < TT; ++t2) a = lane == bb * TT + t2 ? acc[bb][t2] : a;
      if (eb + b < nown) {
        const int e = wave + W * (eb + b);
        const float d = bf2f(f64_to_bf16_via_f32(a));
        logit[tt][e] = bf2f(f2bf(__fadd_rn(d, bf2f(gate_b[e]))));
      }
    }
  }
  __syncthreads();

  if (wave < ntok) {
    const int tok = tok0 + wave;
    const float* lg = logit[wave];
    // rank of each logit: how many others come first (logits past E are
    // -inf and never do)
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const float v = e < E ? lg[e] : 0.0f;
      int rank = 0;
      for (int o0 = 0; o0 < E; o0 += 32) {
        float ov[32];
#pragma unroll
        for (int o = 0; o < 32; ++o) ov[o] = lg[o0 + o];
#pragma unroll
        for (int o = 0; o < 32; ++o)
          rank += (ov[o] > v || (ov[o] == v && o0 + o < e)) ? 1 : 0;
      }
      if (e < E && rank < k) {
        idx_out[(size_t)tok * k + rank] = e;
        topv[wave][rank] = (double)v;
      }
    }
  }
  __syncthreads();
  if (wave < ntok) {
    const int tok = tok0 + wave;
    double ex = 0.0;
    if (lane < k) ex = exp(topv[wave][lane] - topv[wave][0]);
    // summed in rank order, as a single lane would
    auto lane_f64 = [&](int j) {
      const uint64_t u = __builtin_bit_cast(uint64_t, ex);
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, j);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
      return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    };
    double sum = lane_f64(0);
    for (int j = 1; j < k; ++j) sum += lane_f64(j);
    if (lane < k) w_out[(size_t)tok * k + lane] = f64_to_bf16_via_f32(ex / sum);
  }
}

// Router logits: workgroup (bx, by) of W waves computes the logits of tokens
// [TT bx, TT bx + TT) for experts [W epw by, W epw (by + 1)): wave w takes
// experts W (epw by + i) + w, i < epw, one after another (the next gate row
// loads while the current one's dots run).  Up to 1024 tokens epw = 1: the
// experts spread over several workgroups per token.
//  1  the threads load the token rows and the norm weight cooperatively (one
//     16-byte chunk per thread and token); each wave loads its gate row;
//  2  per token, fp64 sum of squares: per thread, fixed-order wave tree, then
//     the waves' sums in wave order; r = fp32(1 / sqrt(ss / H + eps));
//     t = bf16(x * r * w) into LDS; workgroups with by == 0 also write t and
//     its two fp8 pieces (the four threads of a 32-element block share its
//     maximum by lane exchange, the encoding of moe_pieces_kernel);
//  3  per token, the dot of t and the wave's gate row: every product of two
//     bf16 values is exact in fp32 and is added in fp64, per lane, then by a
//     fixed-order wave tree; logit = bf16(bf16(fp32(dot)) + bias), stored as
//     fp32.
// A product below 2^-126 in magnitude is rounded to an fp32 subnormal; no
// logit above 2^-100 can change by it.
// kMfma (TT = 16, large n): step 3 runs on the fp64 matrix cores instead.
// The workgroup covers experts [16 bpw by, 16 bpw (by + 1)) in blocks of 16;
// wave w takes block w % bpw over the K slice w / bpw of W / bpw equal
// slices.  v_mfma_f64_16x16x4 multiplies bf16 values widened to fp64 (exact
// products) and accumulates in fp64: lane l feeds token row l % 16 and expert
// column l % 16 at K position l / 16 of each step; the four lane groups walk
// interleaved 16-byte chunks of the slice (any K order serves, as long as
// both operands use the same).  The slices' partial sums are added in slice
// order through LDS, then rounded as above.
// Outputs of the top-k, softmax and grouping that the last workgroup of the
// logits launch runs (kSel): mlc-llm gating_softmax_topk + moe_cumsum /
// get_indices / get_indptr (model/mlp_optimized.py:118-148).
struct SelectArgs {
  int k;
  int32_t* idx;
  uint16_t* w;
  int32_t* indptr;
  int32_t* sorted_pairs;
  int32_t* token_indices;
  int32_t* expert_ids;
  int32_t* pair_pos;
  int32_t* zero;     // ints zeroed on the way (the decode launch's arrival counts)
  int zero_ints;
  int32_t* arrive;   // workgroups done: zero before the first launch, left zero
};

// Keys and tokens the fused selection holds in LDS (n * roundup(E, 32)).
constexpr int kFusedSelKeys = 4096;
constexpr int kFusedSelTok = 128;

__device__ void select_group_last(const float* logits, int n, int E, const SelectArgs& sel);

template <bool kPieces, int S, int W, int TT, bool kMfma, bool kSel = false>
__global__ __launch_bounds__(64 * W) void moe_router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
    const uint16_t* __restrict__ gate_w, const uint16_t* __restrict__ gate_b, int n, int H, int E,
    float eps, uint16_t* __restrict__ t_out, float* __restrict__ logits,
    uint8_t* __restrict__ pq, uint8_t* __restrict__ pqs, int epw, int32_t* __restrict__ zero_e,
    SelectArgs sel) {
  static_assert(!(kSel && kMfma), "the fused selection follows the VALU dots");
  constexpr int kChunks = 64 * S;                // 16-byte chunks of a row, at most
  constexpr int J = (kChunks + 64 * W - 1) / (64 * W);  // chunks per thread and token
  __shared__ u32x4 t_lds[TT][kChunks];
  __shared__ double ss_part[W][TT];
  __shared__ float rn_lds[TT];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tok0 = blockIdx.x * TT;
  const int ntok = min(TT, n - tok0);
  const int e0 = (int)blockIdx.y * epw * W + wave;  // the wave's first expert
  if (zero_e && blockIdx.x == 0 && blockIdx.y == 0 && tid <= E) zero_e[tid] = 0;
  const int H8 = H >> 3;
  const int NC = (H + 127) >> 7;

  u32x4 gv[S];
  uint16_t gbv = 0;  // the expert's bias, loaded with its gate row (not after the dots)
  auto load_gate = [&](int ee, u32x4* dst, uint16_t& b) {
    const u32x4* gr = (const u32x4*)(gate_w + (size_t)min(ee, E - 1) * H);
#pragma unroll
    for (int i = 0; i < S; ++i) dst[i] = gr[min(lane + 64 * i, H8 - 1)];
    b = gate_b[min(ee, E - 1)];
  };
  if constexpr (!kMfma) load_gate(e0, gv, gbv);
  // rows past n repeat the last token (computed, never stored)
  u32x4 xv[TT][J], wv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) wv[j] = ((const u32x4*)norm_w)[min(tid + 64 * W * j, H8 - 1)];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const u32x4* xr = (const u32x4*)(x + (size_t)min(tok0 + tt, n - 1) * H);
#pragma unroll
    for (int j = 0; j < J; ++j) xv[tt][j] = xr[min(tid + 64 * W * j, H8 - 1)];
  }

#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (tid + 64 * W * j < H8) {
        float f[8];
        unpack8(xv[tt][j], f);
#pragma unroll
        for (int q = 0; q < 8; ++q) ss = fma((double)f[q], (double)f[q], ss);
      }
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) ss_part[wave][tt] = ss;
  }
  __syncthreads();
  if (tid < TT) {
    double ss = ss_part[0][tid];
    for (int w = 1; w < W; ++w) ss += ss_part[w][tid];
    rn_lds[tid] = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
  }
  __syncthreads();

#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const float rn = rn_lds[tt];
    const int tok = tok0 + tt;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      // chunks in [H8, 16 NC) are the zero tail of the pieces' last 128
      const int c = tid + 64 * W * j;
      if (c >= (kPieces ? 16 * NC : H8)) continue;
      u32x4 o = {0u, 0u, 0u, 0u};
      if (c < H8) {
        float f[8], g[8];
        unpack8(xv[tt][j], f);
        unpack8(wv[j], g);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint16_t lo = f2bf(__fmul_rn(__fmul_rn(f[2 * d], rn), g[2 * d]));
          const uint16_t hi = f2bf(__fmul_rn(__fmul_rn(f[2 * d + 1], rn), g[2 * d + 1]));
          o[d] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        t_lds[tt][c] = o;
      }
      if (blockIdx.y == 0 && tt < ntok) {
        if (c < H8) ((u32x4*)(t_out + (size_t)tok * H))[c] = o;
        if constexpr (kPieces) {
          // the quad of a 32-element block is four consecutive threads of
          // one wave, all below H8 or all in the tail (H % 32 == 0)
          const int blk = c >> 2, quarter = c & 3;
          const int ch = blk >> 2, gg = blk & 3;
          const int Kp = NC * 128;
          float rr[8];
          unpack8(o, rr);
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(rr[q]));
            amax = fmaxf(amax, lane_xor1(amax));
            amax = fmaxf(amax, lane_xor2(amax));
            const uint32_t sc = e8m0_for_amax(amax);
            const float inv = __uint_as_float((254u - sc) << 23);
            const float scf = sc ? __uint_as_float(sc << 23) : __uint_as_float(0x00400000u);
            uint32_t lo, hi;
            e4m3_piece8(rr, inv, scf, lo, hi);
            const size_t prow = (size_t)tok * 2 + p;
            *(uint2*)(pq + prow * Kp + c * 8) = make_uint2(lo, hi);
            if (quarter == 0) {
              uint8_t* run = pqs + prow * 112 + gg * 28;
              run[ch] = (uint8_t)sc;
              if (ch == NC - 1)
                for (int z = NC; z < 28; ++z) run[z] = 0;
            }
          }
        }
      }
    }
  }
  __syncthreads();

  if constexpr (kMfma) {
    static_assert(TT == 16, "one MFMA row per token");
    typedef double d4 __attribute__((ext_vector_type(4)));
    const int bpw = epw;            // expert blocks per workgroup (divides W)
    const int KS = W / bpw;         // K slices per block
    const int ks = wave / bpw, wl = wave - ks * bpw;
    const int eb = (int)blockIdx.y * bpw + wl;
    const int r16 = lane & 15, g = lane >> 4;
    const u32x4* gr = (const u32x4*)(gate_w + (size_t)min(eb * 16 + r16, E - 1) * H);
    constexpr int NI = 16 * S;      // steps of four chunks over the padded row
    constexpr int U = 4;            // steps per batch; divides NI / KS for KS <= 8
    const int j0 = ks * (NI / KS), j1 = j0 + NI / KS;
    d4 acc = {0.0, 0.0, 0.0, 0.0};
    if (eb * 16 < E) {  // wave-uniform
      // chunks past H8 are zero in both operands
      auto fetch = [&](int j, u32x4* bb, u32x4* aa) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = 4 * (j + u) + g;
          const bool in = c < H8;
          const u32x4 bv = gr[min(c, H8 - 1)];
          const u32x4 av = t_lds[r16][min(c, H8 - 1)];
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            bb[u][d] = in ? bv[d] : 0u;
            aa[u][d] = in ? av[d] : 0u;
          }
        }
      };
      u32x4 bc[U], ac[U];
      fetch(j0, bc, ac);
      for (int j = j0; j < j1; j += U) {
        u32x4 bn[U], an[U];
        if (j + U < j1) fetch(j + U, bn, an);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const uint32_t aw = ac[u][q >> 1], bw = bc[u][q >> 1];
            const double a = (double)__uint_as_float((q & 1) ? (aw & 0xFFFF0000u) : (aw << 16));
            const double b = (double)__uint_as_float((q & 1) ? (bw & 0xFFFF0000u) : (bw << 16));
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc, 0, 0, 0);
          }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          bc[u] = bn[u];
          ac[u] = an[u];
        }
      }
    }
    // acc[i] of lane l: token row 4 i + l / 16, expert column l % 16
    auto finish = [&](double d, int tt, int ex) {
      if (tt < ntok && ex < E) {
        const float v = bf2f(f64_to_bf16_via_f32(d));
        logits[(size_t)(tok0 + tt) * E + ex] = bf2f(f2bf(__fadd_rn(v, bf2f(gate_b[ex]))));
      }
    };
    if (KS == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) finish(acc[i], 4 * i + g, eb * 16 + r16);
    } else {
      __syncthreads();  // t_lds is free: [KS][bpw][16][16] partial sums
      double* part = (double*)&t_lds[0][0];
#pragma unroll
      for (int i = 0; i < 4; ++i) part[((ks * bpw + wl) * 16 + 4 * i + g) * 16 + r16] = acc[i];
      __syncthreads();
      for (int u = tid; u < bpw * 256; u += 64 * W) {
        const int b = u >> 8, rc = u & 255;
        double sum = part[b * 256 + rc];
        for (int kk = 1; kk < KS; ++kk) sum += part[(kk * bpw + b) * 256 + rc];
        finish(sum, rc >> 4, ((int)blockIdx.y * bpw + b) * 16 + (rc & 15));
      }
    }
    return;
  }

  for (int ei = 0; ei < epw; ++ei) {
    const int e = e0 + ei * W;
    if (e >= E) break;  // wave-uniform
    u32x4 gn[S];
    uint16_t gbn = 0;
    if (ei + 1 < epw) load_gate(e + W, gn, gbn);
    double acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = 0.0;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int c = lane + 64 * i;
      if (c < H8) {
        float gf[8];
        unpack8(gv[i], gf);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          float tf[8];
          unpack8(t_lds[tt][c], tf);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[tt] += (double)__fmul_rn(tf[q], gf[q]);
        }
      }
    }
    const float bias = bf2f(gbv);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const double a = wave_sum_f64(acc[tt]);
      if (lane == 0 && tt < ntok) {
        const float d = bf2f(f64_to_bf16_via_f32(a));
        const float lg = bf2f(f2bf(__fadd_rn(d, bias)));
        float* dst = logits + (size_t)(tok0 + tt) * E + e;
        // kSel: device scope (sc1), read by the last workgroup on any XCD
        if constexpr (kSel) store_dev(dst, lg);
        else *dst = lg;
      }
    }
    if (ei + 1 < epw) {
#pragma unroll
      for (int i = 0; i < S; ++i) gv[i] = gn[i];
      gbv = gbn;
    }
  }
  if constexpr (kSel) {
    // Every wave waits for its own logits stores (complete sc1 stores are
    // visible at device scope), the workgroup meets, and one thread counts
    // it in; the workgroup whose count completes the launch's total runs the
    // selection over every token and resets the count for the next call.
    __shared__ int last;
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0) {
      const int total = (int)(gridDim.x * gridDim.y);
      const int prev =
          __hip_atomic_fetch_add(sel.arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == total - 1;
      if (last) store_dev(sel.arrive, 0);
    }
    __syncthreads();
    if (last) select_group_last(logits, n, E, sel);
  }
}


// Ranking keys staged in LDS for the selection: 16 K keys (64 KB) per pass,
// at most kSelTok tokens.
constexpr int kSelLds = 16384;
constexpr int kSelTok = 256;

// Top-k + softmax of the tokens [t0, t0 + nt), in passes of up to
// kSelLds / Ep tokens: the rows' ranking keys are staged in LDS (stride Ep,
// padded with -inf); one thread per (token, expert) counts the keys above
// its own and the k winners go to topi / topv at their rank; then one thread
// per (token, slot) takes its fp64 exponential, the token's k exponentials
// are summed in rank order (gathered by shuffle within the token's 8 lanes)
// and slot j of idx and w is written.  ti (when given) receives the indices
// at [t - t0][k]; expert counts go to hist (LDS).
// kKeys / kTok: capacity of keys and of topi / topv (8 per token); kDev:
// the logits are read with device-scope loads (written by other workgroups
// of the same launch).
template <int kKeys = kSelLds, int kTok = kSelTok, bool kDev = false>
__device__ __forceinline__ void select_range(const float* __restrict__ logits, int t0, int nt,
                                             int E, int k, uint32_t* keys, int* topi,
                                             float* topv, int32_t* __restrict__ idx_out,
                                             uint16_t* __restrict__ w_out, int* ti, int* hist) {
  const int lane = threadIdx.x & 63;
  const int Ep = (E + 31) & ~31;
  const int per = min(kKeys / Ep, kTok);
  for (int b0 = 0; b0 < nt; b0 += per) {
    const int nbt = min(per, nt - b0);
    const float* src = logits + (size_t)(t0 + b0) * E;
    __syncthreads();  // the previous pass's rows are no longer read
    for (int i = threadIdx.x; i < nbt * Ep; i += blockDim.x) {
      const int r = i / Ep, c = i - r * Ep;
      float v = -INFINITY;
      if (c < E) v = kDev ? load_dev(src + r * E + c) : src[r * E + c];
      keys[i] = rank_key(v, c);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nbt * Ep; i += blockDim.x) {
      const int r = i / Ep, c = i - r * Ep;
      const uint32_t key = keys[i];
      const u32x4* kr = (const u32x4*)(keys + r * Ep);
      int rank = 0;
      if (Ep <= 64) {
        // up to 16 chunks of the row read at once (past Ep: the row's own
        // first chunk again, not counted)
        u32x4 q[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) q[o] = kr[o < (Ep >> 2) ? o : 0];
#pragma unroll
        for (int o = 0; o < 16; ++o)
          if (o < (Ep >> 2))
            rank += (q[o][0] > key) + (q[o][1] > key) + (q[o][2] > key) + (q[o][3] > key);
      } else {
        for (int o = 0; o < (Ep >> 2); ++o) {
          const u32x4 q = kr[o];
          rank += (q[0] > key) + (q[1] > key) + (q[2] > key) + (q[3] > key);
        }
      }
      if (c < E && rank < k) {
        topi[r * 8 + rank] = c;
        topv[r * 8 + rank] = key_value(key);
      }
    }
    __syncthreads();
    // 8 lanes per token: the loop bound keeps a token's lanes together
    for (int i = threadIdx.x; i < nbt * 8; i += blockDim.x) {
      const int r = i >> 3, j = i & 7;
      const double ex = j < k ? exp((double)topv[r * 8 + j] - (double)topv[r * 8]) : 0.0;
      const int base = lane & ~7;
      double sum = __shfl(ex, base, kWave);
      for (int jj = 1; jj < k; ++jj) sum += __shfl(ex, base + jj, kWave);
      if (j < k) {
        const int t = t0 + b0 + r;
        const int e = topi[r * 8 + j];
        w_out[(size_t)t * k + j] = f64_to_bf16_via_f32(ex / sum);
        idx_out[(size_t)t * k + j] = e;
        if (ti) ti[(b0 + r) * k + j] = e;
        atomicAdd(&hist[e], 1);
      }
    }
  }
}

// Top-k + softmax of n <= 128 tokens and the grouping of their n*k pairs,
// one workgroup (mlc-llm gating_softmax_topk + moe_cumsum / get_indices /
// get_indptr, model/mlp_optimized.py:118-148).
__global__ __launch_bounds__(1024) void moe_select_permute_kernel(
    const float* __restrict__ logits, int n, int E, int k, int32_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out, int32_t* __restrict__ indptr,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ token_indices,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ pair_pos,
    int32_t* __restrict__ zero, int zero_ints) {
  // the decode launch's arrival counts start at zero (a kernel, not a memset:
  // the call may be captured in a graph)
  for (int i = threadIdx.x; i < zero_ints; i += blockDim.x) zero[i] = 0;
  __shared__ __align__(16) uint32_t keys[kSelLds];
  __shared__ int topi[kSelTok * 8];
  __shared__ float topv[kSelTok * 8];
  __shared__ int idx_lds[4096];
  __shared__ int cnt[256];
  __shared__ int base[256];
  __shared__ int wcnt[16 * 256];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) {
    cnt[e] = 0;
    base[e] = 0;
  }
  select_range(logits, 0, n, E, k, keys, topi, topv, idx_out, w_out, idx_lds, cnt);
  __syncthreads();
  expert_prefix(cnt, E, base, indptr);
  __syncthreads();
  place_pairs(idx_lds, 0, n * k, k, E, base, wcnt, sorted_pairs, token_indices, expert_ids,
              pair_pos);
}

// Top-k + softmax of n tokens whose logits are in LDS (lg [n][E], E <= 32),
// two tokens per wave, one per 32-lane half: lane e holds expert e's ranking
// key; k rounds of the half's maximum (registers only) give the keys in rank
// order, rank j's going to wk (LDS, [t][k]).  Then one thread per (token,
// rank j) takes its fp64 exponential against rank 0 (ex, LDS), and one per
// pair sums its token's k in rank order and writes slot j of idx and w -- the
// arithmetic of select_range.  The indices also go to ti (LDS, [t][k]) and the
// expert counts to hist (LDS).  The exponentials and quotients are spread
// over every lane of the workgroup, not k of each half-wave.
__device__ __forceinline__ void select_halves(const float* lg, int n, int E, int k,
                                              int32_t* __restrict__ idx_out,
                                              uint16_t* __restrict__ w_out, int* ti, int* hist,
                                              uint32_t* wk, double* ex) {
  rank_halves(lg, n, E, k, wk, (int)(blockDim.x >> 6));
  lds_barrier();
  const int np = n * k;
  for (int p = threadIdx.x; p < np; p += blockDim.x) ex[p] = pair_exp(wk, p, k);
  lds_barrier();
  for (int p = threadIdx.x; p < np; p += blockDim.x) {
    const int ex_id = key_expert(wk[p]);
    w_out[p] = pair_weight(ex, p, k);
    idx_out[p] = ex_id;
    ti[p] = ex_id;
    atomicAdd(&hist[ex_id], 1);
  }
}

// One token (E <= 32, k <= 8) by one wave: route_one_token (moe_select.h).
// The logits were written by other workgroups of this launch (device-scope
// loads).
__device__ __forceinline__ void select_one_token(const float* logits, int E,
                                                 const SelectArgs& sel) {
  const int lane = threadIdx.x & 63;
  const float v = lane < E ? load_dev(logits + lane) : 0.0f;
  for (int i = lane; i < sel.zero_ints; i += 64) sel.zero[i] = 0;
  route_one_token(v, E, sel.k, sel.idx, sel.w, sel.indptr, sel.sorted_pairs, sel.token_indices,
                  sel.expert_ids, sel.pair_pos);
}

// The selection and grouping of moe_select_permute_kernel, run by the last
// workgroup of the logits launch (n * roundup(E, 32) <= kFusedSelKeys, any
// block size up to 1024 threads): the logits are read with device-scope loads.
__device__ void select_group_last(const float* logits, int n, int E, const SelectArgs& sel) {
  if (n == 1 && E <= 32 && sel.k <= 8) {  // one token: one wave, no barrier
    if (threadIdx.x < 64) select_one_token(logits, E, sel);
    return;
  }
  __shared__ __align__(16) uint32_t keys[kFusedSelKeys];
  __shared__ __align__(16) float lg[kFusedSelKeys];
  __shared__ int topi[kFusedSelTok * 8];
  __shared__ float topv[kFusedSelTok * 8];
  __shared__ int idx_lds[kFusedSelTok * 8];
  __shared__ int cnt[256];
  __shared__ int base[256];
  __shared__ int wcnt[16 * 256];
  const int tid = threadIdx.x;
  // The n x E logits into LDS with device-scope loads, all issued before any
  // is used: 16 bytes a thread when E % 4 == 0 (n E <= kFusedSelKeys <= 8
  // blockDim.x: at most 2 loads a thread), else one float each (at most 8).
  const int total = n * E;
  if ((E & 3) == 0) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)logits, (short)0, total * 4, kBufferWord3);
    u32x4 v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + j * (int)blockDim.x;
      if (4 * q < total) v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, q * 16, 0, kCpolSc1);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + j * (int)blockDim.x;
      if (4 * q < total) *(u32x4*)(lg + 4 * q) = v[j];
    }
  } else {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = tid + j * (int)blockDim.x;
      if (i < total) v[j] = load_dev(logits + i);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = tid + j * (int)blockDim.x;
      if (i < total) lg[i] = v[j];
    }
  }
  for (int i = tid; i < sel.zero_ints; i += blockDim.x) sel.zero[i] = 0;
  for (int e = tid; e < E; e += blockDim.x) {
    cnt[e] = 0;
    base[e] = 0;
  }
  // The barriers below wait for LDS only: nothing here reads back the
  // global stores (the zeroed counters, idx, w, indptr), which the launch's
  // end completes.
  lds_barrier();  // lg and the counts are complete
  if (E <= 32)  // (keys and topi are select_range's; here the ranks' scratch)
    select_halves(lg, n, E, sel.k, sel.idx, sel.w, idx_lds, cnt, (uint32_t*)topi,
                  (double*)keys);
  else
    select_range<kFusedSelKeys, kFusedSelTok, false>(lg, 0, n, E, sel.k, keys, topi, topv,
                                                     sel.idx, sel.w, idx_lds, cnt);
  lds_barrier();
  expert_prefix(cnt, E, base, sel.indptr);
  lds_barrier();
  place_pairs(idx_lds, 0, n * sel.k, sel.k, E, base, wcnt, sel.sorted_pairs, sel.token_indices,
              sel.expert_ids, sel.pair_pos);
}

// Tokens per chunk of the large-n grouping.  Ranking costs E^2 key
// compares per token (16 K at E = 128), so small chunks: 16 workgroups at
// 256 tokens rather than 4.
constexpr int kSelChunk = 16;

// Large n, first pass: top-k + softmax of the kSelChunk tokens of chunk
// blockIdx.x and the chunk's expert histogram, counts[chunk][E].
__global__ __launch_bounds__(1024) void moe_select_count_kernel(
    const float* __restrict__ logits, int n, int E, int k, int32_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out, int32_t* __restrict__ counts) {
  __shared__ __align__(16) uint32_t keys[kSelLds];
  __shared__ int topi[kSelChunk * 8];
  __shared__ float topv[kSelChunk * 8];
  __shared__ int h[256];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) h[e] = 0;
  const int t0 = blockIdx.x * kSelChunk;
  select_range(logits, t0, min(kSelChunk, n - t0), E, k, keys, topi, topv, idx_out, w_out,
               nullptr, h);
  __syncthreads();
  for (int e = tid; e < E; e += 1024) counts[(size_t)blockIdx.x * E + e] = h[e];
}

// Large n, second pass: workgroup c places the pairs of chunk c (kSelChunk
// tokens' pairs).  Its base for expert e is the prefix over experts of the totals plus
// the counts of expert e in the chunks before c; chunk 0 writes indptr.
__global__ __launch_bounds__(1024) void moe_place_kernel(
    const int32_t* __restrict__ idx, const int32_t* __restrict__ counts, int nchunks, int nk,
    int k, int E, int32_t* __restrict__ indptr, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ token_indices, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ pair_pos) {
  __shared__ int tot[256];
  __shared__ int base[256];
  __shared__ int wcnt[16 * 256];  // first holds the partial sums below
  const int tid = threadIdx.x, c = blockIdx.x;
  // thread (part, e) sums chunks j = part, part + parts, ... of expert e
  // (all of them, and those before c); the parts are then added in order
  const int parts = 1024 / E;
  {
    const int e = tid % E, part = tid / E;
    int s = 0, before = 0;
    if (part < parts) {
      for (int j = part; j < nchunks; j += parts) {
        const int v = counts[(size_t)j * E + e];
        s += v;
        before += j < c ? v : 0;
      }
      wcnt[part * E + e] = s;
      wcnt[2048 + part * E + e] = before;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 1024) {
    int s = 0, before = 0;
    for (int part = 0; part < parts; ++part) {
      s += wcnt[part * E + e];
      before += wcnt[2048 + part * E + e];
    }
    tot[e] = s;
    base[e] = before;
  }
  __syncthreads();
  expert_prefix(tot, E, base, c == 0 ? indptr : nullptr);
  __syncthreads();
  const int p0 = c * kSelChunk * k;
  place_pairs(idx, p0, min(nk, p0 + kSelChunk * k), k, E, base, wcnt, sorted_pairs,
              token_indices, expert_ids, pair_pos);
}

// Stable counting sort of the n*k (token, slot) pairs by expert, one
// workgroup.  Totals come from LDS atomics (order-free); placement follows
// place_pairs.
__global__ __launch_bounds__(1024) void moe_permute_kernel(
    const int32_t* __restrict__ idx, int nk, int k, int E, int32_t* __restrict__ indptr,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ token_indices,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ pair_pos) {
  __shared__ int cnt[256];
  __shared__ int base[256];
  __shared__ int wcnt[16 * 256];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) {
    cnt[e] = 0;
    base[e] = 0;
  }
  __syncthreads();
  for (int p = tid; p < nk; p += 1024) {
    const int v = idx[p];
    if (v >= 0 && v < E) atomicAdd(&cnt[v], 1);
  }
  __syncthreads();
  expert_prefix(cnt, E, base, indptr);
  __syncthreads();
  place_pairs(idx, 0, nk, k, E, base, wcnt, sorted_pairs, token_indices, expert_ids, pair_pos);
}

}  // namespace moe

// t_pieces (optional, H % 32 == 0): the two fp8 pieces of t, packed as
// moe_launch_pieces writes them.  Up to 256 tokens run one per workgroup of
// four waves; beyond, two tokens share a workgroup, so each gate row read
// from L2 serves two tokens.
extern "C" int moe_launch_router_pieces(const void* x, const void* norm_w, const void* gate_w,
                                        const void* gate_b, int n, int H, int E, int k, float eps,
                                        void* t_out, void* idx_out, void* w_out, void* pq,
                                        void* pqs, hipStream_t stream) {
  if (n == 0) return moe::kOk;
  if (H > 4096 || H % 8 || E > 256 || k > 8 || (pq && H % 32)) return moe::kErrUnsupported;
  const uint16_t *px = (const uint16_t*)x, *pn = (const uint16_t*)norm_w,
                 *pg = (const uint16_t*)gate_w, *pb = (const uint16_t*)gate_b;
  uint16_t* pt = (uint16_t*)t_out;
  int32_t* pi = (int32_t*)idx_out;
  uint16_t* pw = (uint16_t*)w_out;
  uint8_t *q = (uint8_t*)pq, *qs = (uint8_t*)pqs;
#define MOE_RT(PC, S, W, TT, KE)                                                             \
  hipLaunchKernelGGL((moe::moe_router_kernel<PC, S, W, TT, KE>), dim3((n + TT - 1) / TT),   \
                     dim3(64 * W), 0, stream, px, pn, pg, pb, n, H, E, k, eps, pt, pi, pw, q, qs)
#define MOE_RT_S(PC, W, TT, KE)                 \
  if (H <= 64 * 6 * 8) MOE_RT(PC, 6, W, TT, KE); \
  else MOE_RT(PC, 8, W, TT, KE)
  if (n <= 256) {
    if (pq) { MOE_RT_S(true, 4, 1, 4); } else { MOE_RT_S(false, 4, 1, 4); }
  } else {
    if (pq) { MOE_RT_S(true, 4, 2, 4); } else { MOE_RT_S(false, 4, 2, 4); }
  }
#undef MOE_RT_S
#undef MOE_RT
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

extern "C" int moe_launch_router(const void* x, const void* norm_w, const void* gate_w,
                                 const void* gate_b, int n, int H, int E, int k, float eps,
                                 void* t_out, void* idx_out, void* w_out, hipStream_t stream) {
  return moe_launch_router_pieces(x, norm_w, gate_w, gate_b, n, H, E, k, eps, t_out, idx_out,
                                  w_out, nullptr, nullptr, stream);
}

// Logits of the n tokens into logits[n][E] (fp32 holding bf16 values), t,
// and (pq != null, H % 32 == 0) the two fp8 pieces of t.  One expert per
// wave (n <= 1024) or all E per workgroup; TT tokens per workgroup share each
// gate row read.  zero_e (if not null): E + 1 ints set to zero by workgroup
// (0, 0) (the decode launch's completion counts and its status word).
extern "C" int moe_launch_router_logits(const void* x, const void* norm_w, const void* gate_w,
                                        const void* gate_b, int n, int H, int E, float eps,
                                        void* t_out, float* logits, void* pq, void* pqs,
                                        void* zero_e, hipStream_t stream) {
  if (n == 0) return moe::kOk;
  if (H > 4096 || H % 8 || E > 256 || (pq && H % 32)) return moe::kErrUnsupported;
  const uint16_t *px = (const uint16_t*)x, *pn = (const uint16_t*)norm_w,
                 *pg = (const uint16_t*)gate_w, *pb = (const uint16_t*)gate_b;
  uint16_t* pt = (uint16_t*)t_out;
  uint8_t *q = (uint8_t*)pq, *qs = (uint8_t*)pqs;
  constexpr int W = 8;
  // experts per wave: one up to 1024 tokens (more workgroups per token
  // tile), all of them above, where 8 tokens per workgroup share each gate
  // row read (the tile's norm and t then computed once)
  // Above 1024 tokens: 16 tokens per workgroup on the fp64 matrix cores,
  // epw = expert blocks of 16 per workgroup, the largest power of two up to
  // min(blocks, W) that still gives 256 workgroups (one per CU: the t tile
  // takes 96-128 KB of LDS)
  static const int mfma_min = [] {  // MOE_ROUTER_MFMA_MIN overrides (tuning runs)
    const char* v = getenv("MOE_ROUTER_MFMA_MIN");
    return v ? atoi(v) : 1024;
  }();
  const bool mfma = n > mfma_min;
  int epw = 1;
  if (mfma) {
    const int nblk = (E + 15) / 16, gx = (n + 15) / 16;
    while (epw * 2 <= std::min(nblk, W)) epw *= 2;
    while (epw > 1 && gx * ((nblk + epw - 1) / epw) < 256) epw /= 2;
  }
  const int ey = mfma ? ((E + 15) / 16 + epw - 1) / epw : (E + W - 1) / W;
#define MOE_LG(PC, S, TT, MF)                                                                     \
  hipLaunchKernelGGL((moe::moe_router_logits_kernel<PC, S, W, TT, MF>),                           \
                     dim3((n + TT - 1) / TT, ey), dim3(64 * W), 0, stream, px, pn, pg, pb, n, H, \
                     E, eps, pt, logits, q, qs, epw, (int32_t*)zero_e, moe::SelectArgs{})
#define MOE_LG_TT(PC, S)                        \
  if (mfma) MOE_LG(PC, S, 16, true);            \
  else if (n <= 128) MOE_LG(PC, S, 1, false);   \
  else MOE_LG(PC, S, 4, false)
  if (H <= 64 * 6 * 8) {
    if (pq) { MOE_LG_TT(true, 6); } else { MOE_LG_TT(false, 6); }
  } else {
    if (pq) { MOE_LG_TT(true, 8); } else { MOE_LG_TT(false, 8); }
  }
#undef MOE_LG_TT
#undef MOE_LG
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

// The logits launch of moe_launch_router_logits (one token per workgroup,
// one expert per wave) followed, in its last workgroup to finish, by the
// top-k, softmax and grouping of moe_launch_select_group: one launch instead
// of two.  n * roundup(E, 32) <= 4096 keys (n <= 128 at E = 32); otherwise
// kErrUnsupported and nothing is launched.  `arrive` (one int) must be zero
// before the first launch; every launch leaves it zero.
extern "C" int moe_launch_router_select(const void* x, const void* norm_w, const void* gate_w,
                                        const void* gate_b, int n, int H, int E, int k, float eps,
                                        void* t_out, float* logits, void* pq, void* pqs,
                                        void* zero_e, void* idx_out, void* w_out, void* indptr,
                                        void* sorted_pairs, void* token_indices, void* expert_ids,
                                        void* pair_pos, void* zero, int zero_ints, void* arrive,
                                        hipStream_t stream) {
  if (n == 0) return moe::kOk;
  if (H > 4096 || H % 8 || E > 256 || k < 1 || k > 8 || (pq && H % 32) || !arrive)
    return moe::kErrUnsupported;
  if (n > moe::kFusedSelTok || n * ((E + 31) & ~31) > moe::kFusedSelKeys) return moe::kErrUnsupported;
  constexpr int W = 8;
  static_assert(moe::kFusedSelKeys <= 8 * 64 * W, "the staging's loads per thread");
  const moe::SelectArgs sel{k,
                            (int32_t*)idx_out,
                            (uint16_t*)w_out,
                            (int32_t*)indptr,
                            (int32_t*)sorted_pairs,
                            (int32_t*)token_indices,
                            (int32_t*)expert_ids,
                            (int32_t*)pair_pos,
                            (int32_t*)zero,
                            zero_ints,
                            (int32_t*)arrive};
  const uint16_t *px = (const uint16_t*)x, *pn = (const uint16_t*)norm_w,
                 *pg = (const uint16_t*)gate_w, *pb = (const uint16_t*)gate_b;
  uint16_t* pt = (uint16_t*)t_out;
  uint8_t *q = (uint8_t*)pq, *qs = (uint8_t*)pqs;
  const dim3 grid(n, (E + W - 1) / W);
#define MOE_LS(PC, S)                                                                           \
  hipLaunchKernelGGL((moe::moe_router_logits_kernel<PC, S, W, 1, false, true>), grid,          \
                     dim3(64 * W), 0, stream, px, pn, pg, pb, n, H, E, eps, pt, logits, q, qs, 1, \
                     (int32_t*)zero_e, sel)
  if (H <= 64 * 6 * 8) {
    if (pq) { MOE_LS(true, 6); } else { MOE_LS(false, 6); }
  } else {
    if (pq) { MOE_LS(true, 8); } else { MOE_LS(false, 8); }
  }
#undef MOE_LS
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

// Chunks of tokens whose expert counts the large-n grouping keeps.
extern "C" int moe_select_chunks(int n) { return (n + moe::kSelChunk - 1) / moe::kSelChunk; }

// Top-k + softmax of the logits, then the grouping of the pairs: one
// workgroup for n <= 128, otherwise a select/count pass over chunks of
// kSelChunk tokens (counts[chunks][E]) and a placement pass.
// zero_ints (n <= 128 only): ints of `counts` to zero on the way (the decode
// launch's arrival counts).
extern "C" int moe_launch_select_group(const float* logits, int n, int E, int k, void* idx_out,
                                       void* w_out, void* counts, void* indptr,
                                       void* sorted_pairs, void* token_indices,
                                       void* expert_ids, void* pair_pos, int zero_ints,
                                       hipStream_t stream) {
  if (E > 256 || k > 8 || k < 1) return moe::kErrUnsupported;
  int32_t* pi = (int32_t*)idx_out;
  uint16_t* pw = (uint16_t*)w_out;
  int32_t *ip = (int32_t*)indptr, *sp = (int32_t*)sorted_pairs, *ti = (int32_t*)token_indices,
          *ei = (int32_t*)expert_ids, *pp = (int32_t*)pair_pos;
  if (n <= 128) {
    hipLaunchKernelGGL(moe::moe_select_permute_kernel, dim3(1), dim3(1024), 0, stream, logits, n,
                       E, k, pi, pw, ip, sp, ti, ei, pp, (int32_t*)counts, zero_ints);
  } else {
    const int nch = moe_select_chunks(n);
    int32_t* cnt = (int32_t*)counts;
    hipLaunchKernelGGL(moe::moe_select_count_kernel, dim3(nch), dim3(1024), 0, stream, logits,
                       n, E, k, pi, pw, cnt);
    hipLaunchKernelGGL(moe::moe_place_kernel, dim3(nch), dim3(1024), 0, stream, pi, cnt, nch,
                       n * k, k, E, ip, sp, ti, ei, pp);
  }
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

extern "C" int moe_launch_permute(const void* idx, int nk, int k, int E, void* indptr,
                                  void* sorted_pairs, void* token_indices, void* expert_ids,
                                  void* pair_pos, hipStream_t stream) {
  hipLaunchKernelGGL(moe::moe_permute_kernel, dim3(1), dim3(1024), 0, stream, (const int32_t*)idx,
                     nk, k, E, (int32_t*)indptr, (int32_t*)sorted_pairs, (int32_t*)token_indices,
                     (int32_t*)expert_ids, (int32_t*)pair_pos);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
