// Selection and grouping helpers shared by the router's launches and the
// decode launch (which routes in its workgroups from two tokens' logits up):
// the top-k ranking of logit keys held in LDS, the expert prefix and the
// stable counting sort of (token, slot) pairs by expert.
#pragma once
#include "moe_common.h"

namespace moe {

// Maximum of v over this lane's 32-lane half of the wave, in registers: DPP
// quad permutes, half-row and row mirrors (the row's maximum in every lane),
// then v_permlane16_swap for the two rows of the half.  All lanes active.
__device__ __forceinline__ uint32_t half_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return max((uint32_t)b[0], (uint32_t)b[1]);
}

__device__ __forceinline__ double readlane_f64(double x, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Top-k ranking of n tokens whose logits are in LDS (lg [n][E], E <= 32),
// two tokens per wave, one per 32-lane half: lane e holds expert e's ranking
// key; k rounds of the half's maximum (registers only) give the keys in rank
// order, rank j's going to wk (LDS, [t][k]); on_rank(t, j, key) runs in the
// lane that writes it.  All lanes of every wave call it (at most 1024
// threads); the caller's barrier publishes wk.
struct NoRankHook {
  __device__ void operator()(int, int, uint32_t) const {}
};
// nw = the workgroup's waves (blockDim.x / 64, passed in: a read of blockDim
// is a vector load that waits for every load in flight before it).
template <class F = NoRankHook>
__device__ __forceinline__ void rank_halves(const float* lg, int n, int E, int k, uint32_t* wk,
                                            int nw, F on_rank = F{}) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, e = lane & 31;
  for (int t0 = 2 * wave; t0 < n; t0 += 2 * nw) {
    const int t = t0 + half;
    const bool live = t < n;
    // keys below every real key (rank_key(-inf, e) >= 0x007F0000) pad the half
    uint32_t key = (live && e < E) ? rank_key(lg[t * E + e], e) : 0u;
    for (int j = 0; j < k; ++j) {
      const uint32_t m = half_max_u32(key);
      if (live && e == j) {
        wk[t * k + j] = m;
        on_rank(t, j, m);
      }
      if (key == m) key = 0u;  // keys are distinct (the expert is in the low bits)
    }
  }
}

// The expert of a ranking key (0xFFFF - expert in its low 16 bits).
__device__ __forceinline__ int key_expert(uint32_t key) { return 0xFFFF - (int)(key & 0xFFFFu); }

// The softmax over a token's k selected logits, in fp64, as two passes split
// by the caller's barrier: pair_exp gives pair p's exponential against its
// token's rank 0 (wk: the ranked keys, [t][k]), pair_weight sums the token's
// k exponentials in rank order and returns p's weight, fp64 -> fp32 -> bf16.
__device__ __forceinline__ double pair_exp(const uint32_t* wk, int p, int k) {
  return exp((double)key_value(wk[p]) - (double)key_value(wk[p / k * k]));
}
__device__ __forceinline__ uint16_t pair_weight(const double* ex, int p, int k) {
  const int t0 = p / k * k;
  double sum = ex[t0];
  for (int jj = 1; jj < k; ++jj) sum += ex[t0 + jj];
  return f64_to_bf16_via_f32(ex[p] / sum);
}

// One token's top-k and softmax by one wave (E <= 32, k <= 8), registers
// only: lane e < E holds expert e's logit v; the same ranking keys, k rounds
// of the half-wave maximum and fp64 softmax against rank 0, summed in rank
// order, as the workgroup forms.  Lanes j < k get rank j's expert (id) and
// gate weight (w, bf16); every lane of the wave must call it.
__device__ __forceinline__ void one_token_topk(float v, int E, int k, int& id, uint16_t& w) {
  const int lane = threadIdx.x & 63;
  uint32_t key = lane < E ? rank_key(v, lane) : 0u;
  uint32_t win = 0u;
  for (int j = 0; j < k; ++j) {
    const uint32_t m = half_max_u32(key);
    if (lane == j) win = m;
    if (key == m) key = 0u;
  }
  const uint32_t top = (uint32_t)__builtin_amdgcn_readlane((int)win, 0);
  const double ex = lane < k ? exp((double)key_value(win) - (double)key_value(top)) : 0.0;
  double sum = readlane_f64(ex, 0);
  for (int jj = 1; jj < k; ++jj) sum += readlane_f64(ex, jj);
  id = key_expert(win);
  w = lane < k ? f64_to_bf16_via_f32(ex / sum) : (uint16_t)0;
}

// One token's routing outputs by one wave: one_token_topk, then the stable
// counting sort of its k pairs by expert from lane reads (a pair's position:
// the pairs of a lower expert, and those of its expert with a lower slot) and
// indptr (lane e: the pairs of an expert below e) -- the same outputs as the
// workgroup forms, bit for bit, with no LDS round trip or barrier.
__device__ __forceinline__ void route_one_token(float v, int E, int k, int32_t* idx, uint16_t* w,
                                                int32_t* indptr, int32_t* sorted_pairs,
                                                int32_t* token_indices, int32_t* expert_ids,
                                                int32_t* pair_pos) {
  const int lane = threadIdx.x & 63;
  int id;
  uint16_t wt;
  one_token_topk(v, E, k, id, wt);
  int below_e = 0, pos = 0;  // lane e: pairs of experts below e; lane j < k: pair j's position
  for (int q = 0; q < k; ++q) {
    const int xq = __builtin_amdgcn_readlane(id, q);
    below_e += xq < lane ? 1 : 0;
    pos += (xq < id || (xq == id && q < lane)) ? 1 : 0;
  }
  if (lane <= E) indptr[lane] = below_e;
  if (lane < k) {
    w[lane] = wt;
    idx[lane] = id;
    sorted_pairs[pos] = lane;
    token_indices[pos] = 0;
    expert_ids[pos] = id;
    pair_pos[lane] = pos;
  }
}

// Placement of pairs [p0, p1) of a stable counting sort by expert, given
// base[e] (LDS) = the sorted position of the chunk's first pair of expert e.
// Within a round of 1024 pairs a pair's rank among same-expert pairs comes
// from ballots, so pairs keep flattened (token, slot) order inside each
// expert, exactly as np.argsort(kind="stable").  Pairs whose expert id is out
// of range are not placed (pair_pos = -1).  All threads of the workgroup (at
// most 1024) call it; a round is blockDim.x pairs.
__device__ __forceinline__ void place_pairs(const int32_t* idx, int p0, int p1, int k, int E,
                                            int* base, int* wcnt,
                                            int32_t* __restrict__ sorted_pairs,
                                            int32_t* __restrict__ token_indices,
                                            int32_t* __restrict__ expert_ids,
                                            int32_t* __restrict__ pair_pos) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nthr = blockDim.x;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int round0 = p0; round0 < p1; round0 += nthr) {
    const int p = round0 + tid;
    const bool inb = p < p1;
    const int v = inb ? idx[p] : -1;
    const bool ok = inb && v >= 0 && v < E;
    for (int i = tid; i < 16 * E; i += nthr) wcnt[(i / E) * 256 + (i % E)] = 0;
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
    // per expert: the waves' counts become their exclusive prefix (in wave
    // order) on top of base, and base moves past the round
    const int nwv = (nthr + 63) >> 6;
    for (int e = tid; e < E; e += nthr) {
      int run = base[e];
      for (int w = 0; w < nwv; ++w) {
        const int c = wcnt[w * 256 + e];
        wcnt[w * 256 + e] = run;
        run += c;
      }
      base[e] = run;
    }
    __syncthreads();
    if (ok) {
      const int pos = wcnt[wave * 256 + v] + rank;
      sorted_pairs[pos] = p;
      token_indices[pos] = p / k;
      expert_ids[pos] = v;
      pair_pos[p] = pos;
    } else if (inb) {
      pair_pos[p] = -1;
    }
    __syncthreads();
  }
}

// Exclusive prefix over experts of tot[e] (LDS), by wave 0: base[e] +=
// prefix, and indptr (when given) = the prefix with indptr[E] = the total.
__device__ __forceinline__ void expert_prefix(const int* tot, int E, int* base,
                                              int32_t* __restrict__ indptr) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x >= 64) return;
  int carry = 0;
  for (int b = 0; b < E; b += 64) {
    const int e = b + lane;
    const int c = e < E ? tot[e] : 0;
    int v = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    if (e < E) {
      base[e] += carry + v - c;
      if (indptr) indptr[e] = carry + v - c;
    }
    carry += __shfl(v, 63, 64);
  }
  if (indptr && lane == 0) indptr[E] = carry;
}

}  // namespace moe
