// Fused RMSNorm + router GEMV + top-k + softmax, and the expert-grouping pass.
//
// Router: model/mlp.py:375-382 (norm -> gate -> topk -> softmax); the decode
// variant's gating_softmax_topk call is model/mlp_optimized.py:187.
// Grouping: mlc-llm moe_cumsum / get_indices / get_indptr / moe_expand_indptr
// as called at model/mlp_optimized.py:119-148.
#include <algorithm>
#include <climits>

#include "moe_common.h"

namespace moe {

// Unpack the eight bf16 of a 16-byte chunk to fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = bf2f((uint16_t)(v[d] & 0xFFFFu));
    f[2 * d + 1] = bf2f((uint16_t)(v[d] >> 16));
  }
}

// One workgroup of 1024 threads (16 waves) routes TB <= 16 tokens.
//  phase 1  one wave per token: fp64 sum of squares, r = fp32(1/sqrt(ss/H+eps)),
//           t = bf16(x*r*w) to HBM and to LDS;
//  phase 2  1024/E threads per expert, each a strided set of 16-byte chunks of
//           the expert's gate row, fp64 partial dots for all TB tokens; the
//           partials are summed in a fixed order, rounded fp64->fp32->bf16, the
//           bias added in fp32 and rounded to bf16 again;
//  phase 3  one wave per token: k rounds of a wave arg-max under the order
//           (logit descending, expert ascending), then an fp64 softmax.
// Loads are issued in unconditional batches (indices clamped in range) so that
// each thread has one batch of requests in flight instead of a chain.
constexpr int kRouterThreads = 1024;
constexpr int kRouterWaves = kRouterThreads / 64;

template <int TB>
__global__ __launch_bounds__(kRouterThreads) void moe_router_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
    const uint16_t* __restrict__ gate_w, const uint16_t* __restrict__ gate_b, int n, int H, int E,
    int k, float eps, uint16_t* __restrict__ t_out, int32_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* t_lds = (uint16_t*)smem;                                      // [TB][H]
  double* part = (double*)(smem + (size_t)TB * H * 2);                    // [1024][TB]
  float* logit = (float*)((unsigned char*)part + kRouterThreads * TB * 8);  // [TB][E]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tok0 = blockIdx.x * TB;
  const int H8 = H >> 3;

  constexpr int kMaxChunks = 8;  // H <= 4096: at most 8 16-byte chunks per lane
  for (int tb = wave; tb < TB; tb += kRouterWaves) {
    const int tok = tok0 + tb;
    u32x4* trow_lds = (u32x4*)(t_lds + (size_t)tb * H);
    if (tok < n) {
      const u32x4* xr = (const u32x4*)(x + (size_t)tok * H);
      const u32x4* wr = (const u32x4*)norm_w;
      u32x4 xv[kMaxChunks], wv[kMaxChunks];
#pragma unroll
      for (int i = 0; i < kMaxChunks; ++i) {
        const int c = min(lane + kWave * i, H8 - 1);
        xv[i] = xr[c];
        wv[i] = wr[c];
      }
      double ss = 0.0;
#pragma unroll
      for (int i = 0; i < kMaxChunks; ++i) {
        if (lane + kWave * i < H8) {
          float f[8];
          unpack8(xv[i], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
        }
      }
      ss = wave_sum(ss);
      const float r = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
      u32x4* trow = (u32x4*)(t_out + (size_t)tok * H);
#pragma unroll
      for (int i = 0; i < kMaxChunks; ++i) {
        const int c = lane + kWave * i;
        if (c < H8) {
          float f[8], g[8];
          unpack8(xv[i], f);
          unpack8(wv[i], g);
          u32x4 o;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint16_t lo = f2bf(__fmul_rn(__fmul_rn(f[2 * d], r), g[2 * d]));
            const uint16_t hi = f2bf(__fmul_rn(__fmul_rn(f[2 * d + 1], r), g[2 * d + 1]));
            o[d] = (uint32_t)lo | ((uint32_t)hi << 16);
          }
          trow[c] = o;
          trow_lds[c] = o;
        }
      }
    } else {
      for (int c = lane; c < H8; c += kWave) trow_lds[c] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __syncthreads();

  const int ks = kRouterThreads / E;  // threads per expert
  {
    const int e = tid / ks, s = tid - (tid / ks) * ks;
    double acc[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[tb] = 0.0;
    if (e < E) {
      constexpr int kBatch = 12;
      const u32x4* wr = (const u32x4*)(gate_w + (size_t)e * H);
      for (int c0 = s; c0 < H8; c0 += kBatch * ks) {
        u32x4 wv[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) wv[u] = wr[min(c0 + u * ks, H8 - 1)];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int c = c0 + u * ks;
          if (c < H8) {
            float wf[8];
            unpack8(wv[u], wf);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              float tf[8];
              unpack8(((const u32x4*)(t_lds + (size_t)tb * H))[c], tf);
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[tb] = fma((double)tf[i], (double)wf[i], acc[tb]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) part[tid * TB + tb] = acc[tb];
  }
  __syncthreads();
  for (int pi = tid; pi < E * TB; pi += kRouterThreads) {
    const int e = pi / TB, tb = pi - (pi / TB) * TB;
    double sum = 0.0;
    for (int s = 0; s < ks; ++s) sum += part[(e * ks + s) * TB + tb];
    const float dot = bf2f(f2bf((float)sum));
    logit[tb * E + e] = bf2f(f2bf(__fadd_rn(dot, bf2f(gate_b[e]))));
  }
  __syncthreads();

  for (int tb = wave; tb < TB; tb += kRouterWaves) {
    const int tok = tok0 + tb;
    if (tok >= n) continue;
    float v[4];
    bool taken[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? logit[tb * E + e] : 0.0f;
      taken[j] = e >= E;
    }
    double sel_v[8];
    int sel_i[8];
    for (int j = 0; j < k; ++j) {
      float bv = -INFINITY;
      int bi = INT_MAX;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int e = lane + 64 * jj;
        if (!taken[jj] && (v[jj] > bv || (v[jj] == bv && e < bi))) {
          bv = v[jj];
          bi = e;
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (bi < E && (bi & 63) == lane) taken[bi >> 6] = true;
      sel_v[j] = (double)bv;
      sel_i[j] = bi < E ? bi : 0;
    }
    if (lane == 0) {
      double ex[8], sum = 0.0;
      for (int j = 0; j < k; ++j) {
        ex[j] = exp(sel_v[j] - sel_v[0]);
        sum = j == 0 ? ex[0] : sum + ex[j];
      }
      for (int j = 0; j < k; ++j) {
        idx_out[(size_t)tok * k + j] = sel_i[j];
        w_out[(size_t)tok * k + j] = f2bf((float)(ex[j] / sum));
      }
    }
  }
}

// Decode router: one token per workgroup of four waves.  Wave w owns experts
// e = w, w + 4, ... and needs no other wave until the top-k:
//  1  every lane issues its loads at once: chunks c = lane + 64 i (i < S) of
//     x and the norm weight, and the first kDecExp gate rows it owns;
//  2  fp64 sum of squares per lane, fixed-order wave tree (each wave computes
//     the norm of the whole token itself); r = fp32(1 / sqrt(ss / H + eps));
//     t = bf16(x * r * w), kept packed;
//  3  wave 0 writes t; the waves share the t pieces by chunk slot (i % 4 ==
//     w): the four lanes of a 32-element block share its maximum by lane
//     exchange (same encoding as moe_pieces_kernel);
//  4  per owned expert, fp64 dot of t and the gate row: per lane, then a
//     fixed-order wave tree (the next batch's rows load meanwhile);
//     logit = bf16(bf16(dot) + bias) into LDS;
//  5  wave 0: lane e ranks logit e by (value descending, expert ascending)
//     against all others; the k winners' fp64 exponentials are summed in rank
//     order and normalised.
constexpr int kDecWaves = 4;
constexpr int kDecExp = 4;  // gate rows per lane per load batch

template <bool kPieces, int S>
__global__ __launch_bounds__(64 * kDecWaves) void moe_router_decode_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
    const uint16_t* __restrict__ gate_w, const uint16_t* __restrict__ gate_b, int H, int E, int k,
    float eps, uint16_t* __restrict__ t_out, int32_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out, uint8_t* __restrict__ pq, uint8_t* __restrict__ pqs) {
  __shared__ float logit[256];
  __shared__ double topv[8];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int W = kDecWaves;
  const int tok = blockIdx.x;
  const int H8 = H >> 3;
  const int NC = (H + 127) >> 7;
  const u32x4* xr = (const u32x4*)(x + (size_t)tok * H);
  const u32x4* nr = (const u32x4*)norm_w;

  u32x4 xv[S], wv[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int c = min(lane + 64 * i, H8 - 1);
    xv[i] = xr[c];
    wv[i] = nr[c];
  }
  const int nown = (E - wave + W - 1) / W;  // experts owned by this wave
  if (threadIdx.x >= (unsigned)E && threadIdx.x < (unsigned)((E + 31) & ~31))
    logit[threadIdx.x] = -INFINITY;
  u32x4 gv[kDecExp][S];
  auto load_gate = [&](int eb) {
#pragma unroll
    for (int b = 0; b < kDecExp; ++b) {
      // a wave owning no expert (E < 4) still issues the batch: row 0
      const int e = max(0, min(wave + W * min(eb + b, nown - 1), E - 1));
      const u32x4* gr = (const u32x4*)(gate_w + (size_t)e * H);
#pragma unroll
      for (int i = 0; i < S; ++i) gv[b][i] = gr[min(lane + 64 * i, H8 - 1)];
    }
  };
  load_gate(0);  // in flight during the norm

  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if (lane + 64 * i < H8) {
      float f[8];
      unpack8(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
    }
  }
  ss = wave_sum_f64(ss);
  const float rn = (float)(1.0 / sqrt(ss / (double)H + (double)eps));

  u32x4 tp[S];  // t, packed bf16 (zero past H)
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int c = lane + 64 * i;
    float f[8], g[8];
    unpack8(xv[i], f);
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
    for (int d = 0; d < 4; ++d) tp[i][d] = in ? o[d] : 0u;
    if (wave == 0 && in) ((u32x4*)(t_out + (size_t)tok * H))[c] = o;
    if constexpr (kPieces) {
      // a quad (32-element block) lies wholly inside or outside [0, 16 * NC)
      // because H % 32 == 0
      if (i % W == wave && c < 16 * NC) {
        const int blk = c >> 2, quarter = c & 3;
        const int ch = blk >> 2, gg = blk & 3;
        const int Kp = NC * 128;
        float rr[8];
        unpack8(tp[i], rr);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          float amax = 0.0f;
#pragma unroll
          for (int q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(rr[q]));
          amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
          amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
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

  for (int eb = 0; eb < nown; eb += kDecExp) {
    double acc[kDecExp];
#pragma unroll
    for (int b = 0; b < kDecExp; ++b) {
      acc[b] = 0.0;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        float tf[8], gf[8];
        unpack8(tp[i], tf);
        unpack8(gv[b][i], gf);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[b] = fma((double)tf[q], (double)gf[q], acc[b]);
      }
    }
    if (eb + kDecExp < nown) load_gate(eb + kDecExp);  // next rows load during the trees
#pragma unroll
    for (int b = 0; b < kDecExp; ++b) acc[b] = wave_sum_f64(acc[b]);
    if (lane < kDecExp && eb + lane < nown) {
      double a = acc[0];
#pragma unroll
      for (int b = 1; b < kDecExp; ++b) a = lane == b ? acc[b] : a;
      const int e = wave + W * (eb + lane);
      const float d = bf2f(f2bf((float)a));
      logit[e] = bf2f(f2bf(__fadd_rn(d, bf2f(gate_b[e]))));
    }
  }
  __syncthreads();

  if (wave == 0) {
    // rank of each logit: how many others come first (logits past E are
    // -inf and never do)
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const float v = e < E ? logit[e] : 0.0f;
      int rank = 0;
      for (int o0 = 0; o0 < E; o0 += 32) {
        float ov[32];
#pragma unroll
        for (int o = 0; o < 32; ++o) ov[o] = logit[o0 + o];
#pragma unroll
        for (int o = 0; o < 32; ++o)
          rank += (ov[o] > v || (ov[o] == v && o0 + o < e)) ? 1 : 0;
      }
      if (e < E && rank < k) {
        idx_out[(size_t)tok * k + rank] = e;
        topv[rank] = (double)v;
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    double ex = 0.0;
    if (lane < k) ex = exp(topv[lane] - topv[0]);
    // summed in rank order, as a single lane would
    auto lane_f64 = [&](int j) {
      const uint64_t u = __builtin_bit_cast(uint64_t, ex);
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, j);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
      return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    };
    double sum = lane_f64(0);
    for (int j = 1; j < k; ++j) sum += lane_f64(j);
    if (lane < k) w_out[(size_t)tok * k + lane] = f2bf((float)(ex / sum));
  }
}

// Stable counting sort of the n*k (token, slot) pairs by expert, one
// workgroup.  Totals come from LDS atomics (order-free); placement is
// deterministic: within a round of 1024 pairs a pair's rank among same-expert
// pairs comes from ballots, so pairs keep flattened (token, slot) order inside
// each expert, exactly as np.argsort(kind="stable").  Pairs whose expert id is
// out of range are not placed (pair_pos = -1).
__global__ __launch_bounds__(1024) void moe_permute_kernel(
    const int32_t* __restrict__ idx, int nk, int k, int E, int32_t* __restrict__ indptr,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ token_indices,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ pair_pos) {
  __shared__ int cnt[256];
  __shared__ int base[256];
  __shared__ int wcnt[16 * 256];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < nk; p += 1024) {
    const int v = idx[p];
    if (v >= 0 && v < E) atomicAdd(&cnt[v], 1);
  }
  __syncthreads();
  if (wave == 0) {  // exclusive prefix of the counts, 64 experts per step
    int carry = 0;
    for (int b = 0; b < E; b += 64) {
      const int e = b + lane;
      const int c = e < E ? cnt[e] : 0;
      int v = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
      }
      if (e < E) {
        base[e] = carry + v - c;
        indptr[e] = carry + v - c;
      }
      carry += __shfl(v, 63, 64);
    }
    if (lane == 0) indptr[E] = carry;
  }
  __syncthreads();

  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int round0 = 0; round0 < nk; round0 += 1024) {
    const int p = round0 + tid;
    const bool inb = p < nk;
    const int v = inb ? idx[p] : -1;
    const bool ok = inb && v >= 0 && v < E;
    for (int i = tid; i < 16 * E; i += 1024) wcnt[(i / E) * 256 + (i % E)] = 0;
    __syncthreads();
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = ((v >> b) & 1) != 0;
      const uint64_t bb = __ballot(ok && bit);
      same &= bit ? bb : ~bb;
    }
    const int rank = __popcll(same & lt);
    if (ok && rank == 0) wcnt[wave * 256 + v] = __popcll(same);
    __syncthreads();
    if (ok) {
      int pos = base[v] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w * 256 + v];
      sorted_pairs[pos] = p;
      token_indices[pos] = p / k;
      expert_ids[pos] = v;
      pair_pos[p] = pos;
    } else if (inb) {
      pair_pos[p] = -1;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 1024) {
      int s = 0;
      for (int w = 0; w < 16; ++w) s += wcnt[w * 256 + e];
      base[e] += s;
    }
    __syncthreads();
  }
}

}  // namespace moe

// t_pieces (optional, H % 32 == 0): the two fp8 pieces of t, packed as
// moe_launch_pieces writes them.  Returns kErrUnsupported when the fused form
// does not apply (n > kDecodeMax or H > 4096 with pieces requested).
extern "C" int moe_launch_router_pieces(const void* x, const void* norm_w, const void* gate_w,
                                        const void* gate_b, int n, int H, int E, int k, float eps,
                                        void* t_out, void* idx_out, void* w_out, void* pq,
                                        void* pqs, hipStream_t stream) {
  if (n == 0) return moe::kOk;
  if (n > 512 || H > 4096 || (pq && H % 32)) return moe::kErrUnsupported;
  const uint16_t *px = (const uint16_t*)x, *pn = (const uint16_t*)norm_w,
                 *pg = (const uint16_t*)gate_w, *pb = (const uint16_t*)gate_b;
  const dim3 block(64 * moe::kDecWaves);
  uint16_t* pt = (uint16_t*)t_out;
  int32_t* pi = (int32_t*)idx_out;
  uint16_t* pw = (uint16_t*)w_out;
  uint8_t *q = (uint8_t*)pq, *qs = (uint8_t*)pqs;
#define MOE_DEC(PC, S)                                                                          \
  hipLaunchKernelGGL((moe::moe_router_decode_kernel<PC, S>), dim3(n), block, 0, stream, px, pn, \
                     pg, pb, H, E, k, eps, pt, pi, pw, q, qs)
  if (H <= 64 * 6 * 8) {
    if (pq) MOE_DEC(true, 6); else MOE_DEC(false, 6);
  } else {
    if (pq) MOE_DEC(true, 8); else MOE_DEC(false, 8);
  }
#undef MOE_DEC
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

extern "C" int moe_launch_router(const void* x, const void* norm_w, const void* gate_w,
                                 const void* gate_b, int n, int H, int E, int k, float eps,
                                 void* t_out, void* idx_out, void* w_out, hipStream_t stream) {
  if (n == 0) return moe::kOk;
  if (n <= 512)
    return moe_launch_router_pieces(x, norm_w, gate_w, gate_b, n, H, E, k, eps, t_out, idx_out,
                                    w_out, nullptr, nullptr, stream);
  const uint16_t *px = (const uint16_t*)x, *pn = (const uint16_t*)norm_w,
                 *pg = (const uint16_t*)gate_w, *pb = (const uint16_t*)gate_b;
  uint16_t *pt = (uint16_t*)t_out, *pw = (uint16_t*)w_out;
  int32_t* pi = (int32_t*)idx_out;
  // One token per workgroup while that fills the chip; four once the gate
  // matrix re-reads (one per workgroup) start to cost more than latency.
  constexpr int NT = moe::kRouterThreads;
  if (n <= 512) {
    const size_t lds = (size_t)1 * H * 2 + NT * 1 * 8 + (size_t)1 * E * 4;
    hipLaunchKernelGGL(moe::moe_router_kernel<1>, dim3(n), dim3(NT), lds, stream, px, pn, pg, pb,
                       n, H, E, k, eps, pt, pi, pw);
  } else {
    const size_t lds = (size_t)4 * H * 2 + NT * 4 * 8 + (size_t)4 * E * 4;
    hipLaunchKernelGGL(moe::moe_router_kernel<4>, dim3((n + 3) / 4), dim3(NT), lds, stream, px, pn,
                       pg, pb, n, H, E, k, eps, pt, pi, pw);
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
