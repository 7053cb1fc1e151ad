// Expert matmuls on gfx950's block-scaled matrix instruction
// v_mfma_scale_f32_16x16x128_f8f6f4: the MXFP4 weights enter the MFMA as
// they lie in the checkpoint (e2m1 nibbles + one E8M0 byte per 32), so no
// dequantisation runs on the vector ALUs at all.
//
// Reference operators: moe_einsum_fused (model/mlp.py:238-326) for the plain
// epilogue and mxfp4_moe_mlp1_* / mxfp4_moe_mlp2_* (model/mlp_optimized.py:
// 214-660) for the grouped-pair forms, with the fp32 semantics of
// model/mlp.py:387-395: out = bias + sum_k x[k] * W[c, k].
//
// Activations as fp8 pieces.  The instruction's other operand is fp8 e4m3
// with its own E8M0 scale per 32 elements.  An activation row x is written
// as a sum of P pieces x = sum_p q_p * 2^(s_p - 127) + residual, each piece
// one e4m3 code per element and one scale per 32-element block, chosen
// greedily (the piece quantises what the earlier pieces left).  Two pieces
// carry the 8-bit significand of a bf16 value (mlp1's normalised tokens);
// four carry the fp32 SwiGLU output to about 16 bits.  The pieces of one
// token occupy P of the 16 MFMA rows, so each output lane holds all pieces
// of a token and sums them in registers.
//
// Operand layout of the 16x16x128 instruction (A = fp8 activations, B = fp4
// weights, D = fp32), per 128-wide K chunk, lane l = 16 * g + r:
//   A  row r, bytes 0..15  -> k = 16 g + 0..15, bytes 16..31 -> k = 64 + 16 g + 0..15
//   B  column r (a weight row), nibble i (low nibble first) -> k = 32 g + i,
//      i.e. one whole MXFP4 block: block 4 * chunk + g of that row
//   scale_a / scale_b of lane (r, g) = the E8M0 of K block g of row / column r
//   D  column r (weight row), elements i = 0..3 -> rows 4 g + i
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "moe_common.h"
#include "moe_select.h"

namespace moe {

constexpr int kMxMaxChunks = 24;                           // K <= 3072
constexpr int kMxSclRun = 28;                              // scale bytes per (row, lane group)
constexpr int kMxSclRow = 4 * kMxSclRun;                   // 112 scale bytes per piece row
constexpr int kMxMaxGroups = 3;
constexpr int kMxRowMap = 32;                              // >= kMxMaxGroups * 16 / 2 tokens
static_assert(kMxMaxGroups * 8 <= kMxRowMap, "row map");
constexpr int kLdsBytes = 160 * 1024;                      // per CU
constexpr int kNumCUs = 256;                               // MI355X
constexpr int kNumXcds = 8;                                // 8 XCDs of 32 CUs, one L2 each

// LDS bytes per staged activation row and per 16-row A operand group for a
// kernel that runs NCT chunks (the 16-byte pad spreads the 16 rows of one
// lane group over distinct banks).
__host__ __device__ constexpr int mx_row_stride(int nct) { return nct * 128 + 16; }
__host__ __device__ constexpr int mx_group_bytes(int nct) {
  return 16 * mx_row_stride(nct) + 16 * kMxSclRow;
}

template <int S, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (S < E) {
    f(std::integral_constant<int, S>{});
    static_for<S + 1, E>(f);
  }
}

// ---------------------------------------------------------------------------
// Pieces.  Packed layout for `rows` rows of length K, NC = ceil(K / 128):
//   q  [rows][P][NC * 128]   e4m3 codes, zero beyond K
//   qs [rows][P][4][28]      qs[.., g, c] = E8M0 of block 4c + g (0 past NC)
// Four adjacent threads share one (row, 32-element block), 8 elements each;
// the block maximum is combined over the four with two lane exchanges.
template <int P, bool kF32>
__global__ __launch_bounds__(256) void moe_pieces_kernel(const void* __restrict__ x, int rows,
                                                         int K, int NC, uint8_t* __restrict__ q,
                                                         uint8_t* __restrict__ qs) {
  const int nblk = 4 * NC;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nthreads = (int64_t)rows * nblk * 4;
  // Whole quads lie past the end (nthreads and 256 are multiples of 4); they
  // compute on block 0 so every lane takes part in the exchanges, and store
  // nothing.
  const bool valid = id < nthreads;
  const int64_t idc = valid ? id : (id & 3);
  const int quarter = (int)(idc & 3);
  const int64_t rb = idc >> 2;
  const int row = (int)(rb / nblk), blk = (int)(rb - (int64_t)row * nblk);
  const int c = blk >> 2, g = blk & 3;
  const int Kp = NC * 128;
  const int k0 = blk * 32 + quarter * 8;
  float r[8];
  if (blk * 32 < K) {
    if constexpr (kF32) {
      const f32x4* src = (const f32x4*)((const float*)x + (size_t)row * K + k0);
      const f32x4 v0 = src[0], v1 = src[1];
      r[0] = v0[0]; r[1] = v0[1]; r[2] = v0[2]; r[3] = v0[3];
      r[4] = v1[0]; r[5] = v1[1]; r[6] = v1[2]; r[7] = v1[3];
    } else {
      const u32x4 v = *(const u32x4*)((const uint16_t*)x + (size_t)row * K + k0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r[2 * j] = __uint_as_float(v[j] << 16);
        r[2 * j + 1] = __uint_as_float(v[j] & 0xFFFF0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = 0.0f;
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(r[i]));
    amax = fmaxf(amax, lane_xor1(amax));
    amax = fmaxf(amax, lane_xor2(amax));
    const uint32_t s = e8m0_for_amax(amax);
    const float inv = __uint_as_float((254u - s) << 23);                           // 2^(127 - s)
    const float sc = s ? __uint_as_float(s << 23) : __uint_as_float(0x00400000u);  // 2^(s - 127)
    uint32_t lo, hi;
    e4m3_piece8(r, inv, sc, lo, hi);
    const size_t prow = (size_t)row * P + p;
    if (!valid) continue;
    *(uint2*)(q + prow * Kp + k0) = make_uint2(lo, hi);
    if (quarter == 0) {
      uint8_t* run = qs + prow * kMxSclRow + g * kMxSclRun;
      run[c] = (uint8_t)s;
      if (c == NC - 1)
        for (int z = NC; z < kMxSclRun; ++z) run[z] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped expert GEMV.  Work is counted in units: one unit = one 16-row
// weight tile of one expert for one batch of that expert's tokens (a batch is
// at most `groups_cap` * 16/P tokens, the pieces that fit in LDS).  Every
// workgroup scans the per-expert unit counts from indptr and takes an equal
// contiguous share of all units, so experts with many tokens (several
// batches) are spread over the chip like the rest.  A share splits into
// segments of one (expert, batch); for each segment the workgroup stages that
// batch's pieces in LDS and its waves take the segment's tiles round-robin:
// the tile's scale bytes and NCT weight loads (MFMA-native: lane (r, g) reads
// block 4c + g of row r, 16 B, for chunk c) are issued together, scales
// first, so MFMA c waits only for the loads up to chunk c; every token group
// of the batch then runs NCT MFMAs over them.  Each wave's first tile is
// issued before the first staging, so its loads overlap it.

// LDS areas of one pass, as byte offsets from the dynamic LDS base (the A
// operand groups start at 0).
struct MxLds {
  int sstage;    // per-wave scale staging, 16 G bytes per wave
  int pre;       // unit prefix, E + 1 ints
  int ipl;       // indptr, E + 1 ints
  int rowmap;    // one batch's sorted_pairs, kMxRowMap ints
  int tile_ctr;  // the segment's tile counter
  int act;       // kEpi 3: the share's SwiGLU outputs, fp32 [tokens][columns]
};

// A segment of a workgroup's share: expert, first token of its batch, first
// tile and tile count (e < 0: none).
struct MxSeg {
  int e, b0, t0, len;
};

// Exclusive prefix of the unit counts, ceil(cnt_e / tpb) * ntiles, into pre,
// and indptr into ipl unless it is null.  Run by one wave.
__device__ __forceinline__ void mx_unit_prefix(const int* __restrict__ indptr, int E, int tpb,
                                               int ntiles, int* pre, int* ipl) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  if (lane == 0) pre[0] = 0;
  for (int b = 0; b < E; b += 64) {
    const int i = b + lane;
    int v = 0;
    if (i < E) {
      const int a0 = indptr[i], a1 = indptr[i + 1];
      v = (a1 - a0 + tpb - 1) / tpb * ntiles;
      if (ipl) {
        ipl[i] = a0;
        if (i == E - 1) ipl[E] = a1;
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, kWave);
      if (lane >= o) v += t;
    }
    if (i < E) pre[i + 1] = carry + v;
    carry += __shfl(v, 63, kWave);
  }
}

// The workgroup's share [ubeg, uend) of the units counted in pre (E + 1
// prefix, LDS).  Workgroups go to the XCDs round-robin (workgroup b on XCD
// b % xcds); numbering them XCD-major hands each XCD one contiguous run of
// unit ranges, so the workgroups that stage an expert's activations share an
// L2.  Units lie batch after batch (ntiles each).  With no more batches than
// workgroups, every batch gets floor or ceil of grid / batches workgroups and
// each of those an equal share of its tiles, starting and ending on
// multiples of `align` tiles: one segment (one staging) per workgroup.  A
// share that straddled two batches would stage twice and finish last.  With
// more batches than workgroups, the units are split evenly and a share may
// span several segments.  balance: also split evenly when the batch split
// would load its busiest workgroups more than 1.25 times the average (q
// workgroups for most batches gives ntiles / q tiles each against
// ntiles * batches / grid on average: with q = 1, 140 batches on 256
// workgroups put a whole batch on 116 of them at 1.7 times the average).
__device__ __forceinline__ void mx_share(const int* pre, int E, int ntiles, int align, int xcds,
                                         int& ubeg, int& uend, bool balance = false) {
  const int total = pre[E];  // < 2^31 (the launchers check)
  const int vb = xcds > 1 ? (int)(blockIdx.x % xcds) * (int)(gridDim.x / xcds) +
                                (int)(blockIdx.x / xcds)
                          : (int)blockIdx.x;
  const int nbatches = (int)(total / ntiles);
  if (nbatches > 0 && nbatches <= (int)gridDim.x &&
      !(balance && 5 * ((int)gridDim.x / nbatches) * nbatches < 4 * (int)gridDim.x)) {
    const int q = (int)gridDim.x / nbatches, rmd = (int)gridDim.x % nbatches;
    int b, i, w;
    if (vb < rmd * (q + 1)) {
      b = vb / (q + 1);
      i = vb - b * (q + 1);
      w = q + 1;
    } else {
      b = rmd + (vb - rmd * (q + 1)) / q;
      i = vb - rmd * (q + 1) - (b - rmd) * q;
      w = q;
    }
    const int na = ntiles / align;
    ubeg = b * ntiles + align * (na * i / w);
    uend = b * ntiles + align * (na * (i + 1) / w);
  } else {
    // floor(total * vb / grid) in 32-bit steps: total = a grid + r, r < grid
    const int g = (int)gridDim.x, a = (int)total / g, r = (int)total - a * g;
    ubeg = a * vb + r * vb / g;
    uend = a * (vb + 1) + r * (vb + 1) / g;
  }
}

// The largest e with pre[e] <= u: the expert of unit u.
__device__ __forceinline__ int mx_expert_of(const int* pre, int E, int u) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= u) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The decode launch's shares with the workgroups weighted by cost.  Batches
// lie expert after expert (tpb tokens each, an expert's last one the rest,
// ntiles units each); a batch of nb tokens costs wa + ceil(nb / tpg) per
// tile: a tile's MFMAs, A-operand reads and epilogue grow with its operand
// groups (at decode 64, phase 2 took 0.96, 1.11 and 1.25-1.35 us per tile
// and workgroup with 1, 2 and 3 groups; wa = 5 gives 6 : 7 : 8).  With NB
// batches (NB <= grid) and W their total cost, batch b's workgroups start at
// b + floor((grid - NB) * W_b / W), W_b the cost of the batches before it,
// so each gets at least one and the rest in proportion to its cost.
// Workgroup vb (numbered XCD-major as in mx_share) takes its equal share of
// its batch's tiles, starting and ending on multiples of `align`.  indptr
// may be the LDS copy.  Run by one wave; writes [ubeg, uend) to out[0],
// out[1].
__device__ __forceinline__ void mx_weighted_share(const int* __restrict__ indptr, int E, int tpb,
                                                  int tpg, int wa, int ntiles, int align,
                                                  int xcds, int* out) {
  const int lane = threadIdx.x & 63;
  const int grid = (int)gridDim.x;
  const int vb = xcds > 1 ? (int)(blockIdx.x % xcds) * (grid / xcds) + (int)(blockIdx.x / xcds)
                          : (int)blockIdx.x;
  const int wfull = wa + (tpb + tpg - 1) / tpg;  // a full batch's cost
  auto expert = [&](int e, int& nbat, int& wsum) {
    nbat = 0;
    wsum = 0;
    if (e < E) {
      const int cnt = indptr[e + 1] - indptr[e];
      nbat = (cnt + tpb - 1) / tpb;
      if (nbat > 0) wsum = (nbat - 1) * wfull + wa + (cnt - (nbat - 1) * tpb + tpg - 1) / tpg;
    }
  };
  if (lane == 0) {
    out[0] = 0;
    out[1] = 0;
  }
  int NB = 0, W = 0;
  for (int b = 0; b < E; b += 64) {
    int nbat, wsum;
    expert(b + lane, nbat, wsum);
    NB += wave_sum(nbat);
    W += wave_sum(wsum);
  }
  if (W == 0) return;
  const int spare = grid - NB;
  auto start_of = [&](int bi, int wp) { return bi + (int)((int64_t)spare * wp / W); };
  int cb = 0, cw = 0;
  for (int b = 0; b < E; b += 64) {
    int nbat, wsum;
    expert(b + lane, nbat, wsum);
    int sb = nbat, sw = wsum;  // inclusive scans over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int tb = __shfl_up(sb, o, kWave), tw = __shfl_up(sw, o, kWave);
      if (lane >= o) {
        sb += tb;
        sw += tw;
      }
    }
    const int bb = cb + sb - nbat, wb = cw + sw - wsum;  // this expert's first batch, cost before it
    for (int j = 0; j < nbat; ++j) {
      const int s0 = start_of(bb + j, wb + j * wfull);
      const int s1 = j + 1 < nbat ? start_of(bb + j + 1, wb + (j + 1) * wfull)
                                  : start_of(bb + nbat, wb + wsum);
      if (s0 <= vb && vb < s1) {
        const int w = s1 - s0, i = vb - s0, na = ntiles / align, bi = bb + j;
        out[0] = bi * ntiles + align * (na * i / w);
        out[1] = bi * ntiles + align * (na * (i + 1) / w);
      }
    }
    cb += __shfl(sb, 63, kWave);
    cw += __shfl(sw, 63, kWave);
  }
}

// One grouped GEMV pass over the units counted in L.pre (indptr in L.ipl).
// align: with one segment per workgroup, shares of a batch start and end at
// multiples of `align` tiles.  kWait: wait(e, b0, nb) runs before each
// segment's staging, called by every thread and ending in a workgroup
// barrier; the first segment's first tile loads are issued before it.
// first: the share's first segment.  balance: mx_share's (the decode launch,
// whose shares must be one segment each, leaves it off).  share (LDS, may be
// null): [ubeg, uend) computed by the caller instead of mx_share's.
// rowmap_ready: the caller put the first segment's sorted_pairs entries in
// L.rowmap (the decode launch's own routing); they are not loaded.
template <int P, int kEpi, int NCT, bool kWait, class WaitFn>
__device__ __forceinline__ void mx_pass(
    uint8_t* lds, const MxLds& L, const uint8_t* __restrict__ q, const uint8_t* __restrict__ qs,
    int Kp, const int* __restrict__ sorted_pairs, int k_top, int arow_mode, int orow_mode,
    const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, int N, int G, int E, int groups_cap, float alpha,
    float limit, float* __restrict__ out, int out_ld, int xcds, int align, WaitFn&& wait,
    MxSeg& first, int nthr, bool balance = false, const int* share = nullptr,
    bool rowmap_ready = false) {
  constexpr int TPG = 16 / P;  // tokens per 16-row operand group
  constexpr int kMxRowStride = mx_row_stride(NCT);
  constexpr int kMxGroupBytes = mx_group_bytes(NCT);
  const int lane = threadIdx.x & 63;
  // wave index in a scalar register: branches on it are uniform
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // nthr = blockDim.x, read once by the caller: blockDim comes from the
  // dispatch packet by a vector load, so each read waits for every load in
  // flight before it (the tile loads, in a later segment's staging)
  const int nwaves = nthr >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int ntiles = N >> 4;
  const int tpb = groups_cap * TPG;
  uint8_t* const sstage = lds + L.sstage + wave * (16 * G);
  int* const pre = (int*)(lds + L.pre);
  int* const ipl = (int*)(lds + L.ipl);
  int* const rowmap = (int*)(lds + L.rowmap);
  __attribute__((address_space(3))) int* const tile_ctr =
      (__attribute__((address_space(3))) int*)(int*)(lds + L.tile_ctr);
  first.e = -1;

  int ubeg, uend;
  if (share) {
    ubeg = share[0];
    uend = share[1];
  } else {
    mx_share(pre, E, ntiles, align, xcds, ubeg, uend, balance);
  }
  if (ubeg >= uend) return;
  auto expert_of = [&](int u) { return mx_expert_of(pre, E, u); };

  // Two-stage pipeline per wave: a tile's weights come in two halves of
  // H0 and H1 chunks held in wa / wb.  While one half's MFMAs run, the other
  // half's loads (or the next tile's first half) are in flight.
  constexpr int H0 = (NCT + 1) / 2, H1 = NCT - H0;
  u32x4 wa[H0], wb[H1];
  u32x4 sc0, sc1;          // the tile's scale bytes, staged in LDS at compute time
  float bn = 0.0f, bn_next = 0.0f;
  // Block index of chunk c for this lane: 4c + g.  Past K the lane re-reads
  // block G-1 (finite data; its A operand bytes are zero).  With NCT == 23
  // (89 <= G <= 92) only the last chunk can pass K, so the others address
  // from one base with immediate offsets.  The opaque copy of g keeps the
  // compiler from hoisting 2*NCT per-chunk offsets out of the tile loop.
  auto blk_of = [&](int c, int gl) {
    return (NCT == 23 && c < 22) ? 4 * c + gl : min(4 * c + gl, G - 1);
  };
  // First half: the tile's 16 x G scale bytes (contiguous, 16-byte aligned,
  // G <= 96 units: two 16-byte loads per lane), its bias and chunks 0..H0-1.
  auto issue_h0 = [&](int e, int tile) {
    int gl = g;
    asm volatile("" : "+v"(gl));
    const size_t row0 = (size_t)e * N + (tile << 4);
    const uint8_t* st = scales + row0 * G;
    sc0 = *(const u32x4*)(st + min(lane, G - 1) * 16);
    sc1 = *(const u32x4*)(st + min(lane + 64, G - 1) * 16);
    bn_next = bf2f(bias[row0 + r]);
    const uint8_t* wp = blocks + (row0 + r) * G * 16;
    static_for<0, H0>([&](auto cv) {
      constexpr int c = decltype(cv)::value;
      wa[c] = *(const u32x4*)(wp + blk_of(c, gl) * 16);
    });
  };
  auto issue_h1 = [&](int e, int tile) {
    int gl = g;
    asm volatile("" : "+v"(gl));
    const uint8_t* wp = blocks + ((size_t)e * N + (tile << 4) + r) * G * 16;
    static_for<0, H1>([&](auto cv) {
      constexpr int c = decltype(cv)::value;
      wb[c] = *(const u32x4*)(wp + blk_of(H0 + c, gl) * 16);
    });
  };
  // kWait: chunks [c0, c1) of a tile pulled into the caches while the pass
  // waits, by direct-to-LDS loads into the third operand group (free until
  // the staging, whose loads are issued later and so land later).
  auto warm = [&](int e, int tile, auto c0v, auto c1v) {
    int gl = g;
    asm volatile("" : "+v"(gl));
    const uint8_t* wp = blocks + ((size_t)e * N + (tile << 4) + r) * G * 16;
    static_for<decltype(c0v)::value, decltype(c1v)::value>([&](auto cv) {
      constexpr int c = decltype(cv)::value;
      __builtin_amdgcn_global_load_lds((const void*)(wp + blk_of(c, gl) * 16),
                                       (lds_ptr_t)(lds + 2 * kMxGroupBytes + c * 1024), 16, 0, 0);
    });
  };
  // The scale bytes pass through LDS to reach the lane that needs each one.
  // Lanes past the G units store unit G - 1 again (the bytes they loaded):
  // with the stores under lane conditions, the compiler lost track of the
  // loads still in flight across the branches and waited for all of them
  // (vmcnt(0), the second half's loads included) before the tile's first
  // MFMA.
  auto stage_scales = [&]() {
    *(u32x4*)(sstage + min(lane, G - 1) * 16) = sc0;
    *(u32x4*)(sstage + min(lane + 64, G - 1) * 16) = sc1;
  };
  const uint32_t sstage_off = L.sstage + wave * (16 * G) + r * G;
  auto scale_b = [&](uint32_t ss, int c) -> uint32_t { return lds[ss + blk_of(c, g)]; };

  auto seg_at = [&](int u) {
    MxSeg sgm;
    sgm.e = expert_of(u);
    const int off = u - pre[sgm.e];
    sgm.b0 = off / ntiles * tpb;
    sgm.t0 = off % ntiles;
    sgm.len = min(uend - u, ntiles - sgm.t0);
    return sgm;
  };

  const bool need_sp = arow_mode != 2 || orow_mode == 0;
  // Direct-to-LDS staging of packed pieces (NCT == 23): a group's bytes tile
  // exactly into 1 KB windows, one 64-lane x 16-byte global_load_lds each.
  // A 16-byte slot is 16 code bytes of a piece row, the row's pad (never
  // read) or 16 of its scale bytes.  Rows past the batch are not loaded:
  // their LDS bytes keep whatever they held (an MFMA output row depends on
  // its own operand row only, and rows past the batch are neither stored nor
  // combined with other rows; zero-filling them instead measured slower at
  // 64 tokens).  No registers hold the data, so a batch's whole staging is
  // in flight at once.
  constexpr bool kDirect = kEpi != 2 && NCT == 23;
  static_assert(mx_group_bytes(23) % 1024 == 0, "group windows");
  // kWait: the pieces were written by other workgroups of this launch with
  // device-scope stores; device-scope (sc1) loads read them coherently (a
  // 128-byte line may hold bytes of several writers and of other batches).
  auto fill_direct = [&](int start, int b0, int nb) {
    constexpr int kWin = kMxGroupBytes / 1024;
    const int nwin = ((nb + TPG - 1) / TPG) * kWin;
    for (int wi = wave; wi < nwin; wi += nwaves) {
      const int gi = wi / kWin;
      const int o = (wi - gi * kWin) * 1024 + lane * 16;
      const bool in_rows = o < 16 * kMxRowStride;
      const int m = in_rows ? o / kMxRowStride : (o - 16 * kMxRowStride) / kMxSclRow;
      const int within =
          in_rows ? o - m * kMxRowStride : o - 16 * kMxRowStride - m * kMxSclRow;
      const int tt = gi * TPG + m / P;
      if (tt < nb) {
        const int row = arow_mode == 0   ? rowmap[tt] / k_top
                        : arow_mode == 1 ? rowmap[tt]
                                         : start + b0 + tt;
        const size_t prow = (size_t)row * P + (m % P);
        const uint8_t* src = in_rows ? q + prow * Kp + (within < Kp ? within : 0)
                                     : qs + prow * kMxSclRow + within;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(lds + wi * 1024), 16, 0,
                                         kWait ? kCpolSc1 : 0);
      }
    }
  };

  MxSeg sg = seg_at(ubeg);
  first = sg;
  // kEpi 3 (one segment per share): the SwiGLU outputs of the share's
  // columns, [token of the batch][column - act_c0]
  float* const act_t = (float*)(lds + L.act);
  const int act_c0 = sg.t0 * 8, act_ld = (uend - ubeg) * 8;
  if constexpr (kDirect && kWait) {
    // the first tile's loads go out before the wait, the staging after it
    const int start = ipl[sg.e], nb = min(tpb, ipl[sg.e + 1] - start - sg.b0);
    if (!rowmap_ready && arow_mode != 2 && (int)threadIdx.x < nb)
      rowmap[threadIdx.x] = sorted_pairs[start + sg.b0 + (int)threadIdx.x];
    const bool rm_lane =
        !rowmap_ready && arow_mode == 2 && orow_mode == 0 && (int)threadIdx.x < nb;
    int rm = 0;
    if (rm_lane) rm = sorted_pairs[start + sg.b0 + (int)threadIdx.x];
    if (threadIdx.x == 0) *tile_ctr = 0;
    // the wait's first poll goes out ahead of the tile loads: loads return in
    // issue order, so a poll issued after them would wait for all of them
    wait.pre(sg.e);
    __builtin_amdgcn_sched_barrier(0);
    issue_h0(sg.e, sg.t0 + (wave < sg.len ? wave : 0));
    if (wave < sg.len)
      warm(sg.e, sg.t0 + wave, std::integral_constant<int, H0>{}, std::integral_constant<int, NCT>{});
    __builtin_amdgcn_sched_barrier(0);
    wait(sg.e, sg.b0, nb);  // its barrier also publishes the row map
    fill_direct(start, sg.b0, nb);
    wait_vmcnt<0>();
    if (rm_lane) rowmap[threadIdx.x] = rm;
    lds_barrier();
  } else if constexpr (kDirect) {
    // The first batch is staged before any tile is requested: loads complete
    // in issue order, so the first MFMAs then wait for their own tile only
    // rather than for a whole chip-wide round of tile loads.
    const int start = ipl[sg.e], nb = min(tpb, ipl[sg.e + 1] - start - sg.b0);
    if (!rowmap_ready && arow_mode != 2) {
      if ((int)threadIdx.x < nb) rowmap[threadIdx.x] = sorted_pairs[start + sg.b0 + (int)threadIdx.x];
      __syncthreads();  // (nothing else in flight)
    }
    fill_direct(start, sg.b0, nb);
    const bool rm_lane =
        !rowmap_ready && arow_mode == 2 && orow_mode == 0 && (int)threadIdx.x < nb;
    int rm = 0;
    if (rm_lane) rm = sorted_pairs[start + sg.b0 + (int)threadIdx.x];
    if (threadIdx.x == 0) *tile_ctr = 0;
    __builtin_amdgcn_sched_barrier(0);
    issue_h0(sg.e, sg.t0 + (wave < sg.len ? wave : 0));
    __builtin_amdgcn_sched_barrier(0);
    // everything before the first half's 15 loads (2 scale, 1 bias, 12
    // chunks) has landed: the staging and the row map entry
    wait_vmcnt<15>();
    if (rm_lane) rowmap[threadIdx.x] = rm;
    lds_barrier();
  } else {
    // in flight during the first staging (a wave without a tile in the first
    // segment loads the segment's first tile; it is replaced before use)
    issue_h0(sg.e, sg.t0 + (wave < sg.len ? wave : 0));
  }

  if (NCT * 128 > Kp) {  // zero the K tail of every staged row once
    const int tail16 = (NCT * 128 - Kp) >> 4;
    for (int u = threadIdx.x; u < groups_cap * 16 * tail16; u += nthr) {
      const int row = u / tail16, c = u - row * tail16;
      *(u32x4*)(lds + (row >> 4) * kMxGroupBytes + (row & 15) * kMxRowStride + Kp + c * 16) =
          u32x4{0u, 0u, 0u, 0u};
    }
  }

  for (int u = ubeg; u < uend;) {
    const int e = sg.e, b0 = sg.b0, t0 = sg.t0, len = sg.len;
    const int start = ipl[e];
    const int nb = min(tpb, ipl[e + 1] - start - b0);
    // The batch's sorted_pairs entries go to LDS (rowmap[tt] for token tt of
    // the batch), so no global load sits in the staging's address chain or in
    // the epilogue: loads complete in issue order, and waiting on one issued
    // behind the tiles in flight would wait for all of them.  The barriers
    // here wait for LDS traffic only (lds_barrier), for the same reason.
    // (direct staging stages the first segment above)
    if (!kDirect || u != ubeg) {
      if (u != ubeg) lds_barrier();  // the previous segment's operands are no longer read
      if constexpr (kWait) wait(e, b0, nb);
      if (threadIdx.x == 0) *tile_ctr = 0;  // read after the staging's barrier
      if (need_sp) {
        if ((int)threadIdx.x < nb) rowmap[threadIdx.x] = sorted_pairs[start + b0 + (int)threadIdx.x];
        lds_barrier();
      }
      // Later segments stage through registers, not by direct-to-LDS loads:
      // the compiler cannot tell which LDS bytes such a load writes, so with
      // one inside this loop it waits for every load in flight (vmcnt(0))
      // before each operand group's first MFMA, draining the two-stage tile
      // pipeline; without one the chunk waits are exact (the GEMV passes at
      // 120B decode 256: block 408-414 us against 416-420).  The decode
      // launch's mlp1 pass (kEpi 3, one segment per workgroup, so this
      // branch never runs there) keeps the direct staging and with it the
      // drained waits: at decode 64 the launch measured 94.0 us that way,
      // 94.9 with exact waits and 96.2 with an explicit vmcnt(0) at the same
      // places (the code shapes differ).
      if constexpr (kDirect && kEpi == 3) {
        fill_direct(start, b0, nb);
        wait_vmcnt<0>();
      } else if constexpr (kEpi == 2) {
        // Stage the batch from fp32 rows (q holds float rows of length 32 G),
        // encoding the P pieces on the way, exactly as moe_pieces_kernel does:
        // four threads per 32-element block (8 elements each), the block
        // maximum by lane exchange.  Blocks past K are zero.  Whole quads past
        // the end compute on the batch's first block and store nothing.
        const float* xf = (const float*)q;
        const int K = G * 32;
        const int nblk = NCT * 4;
        const int tasks = nb * nblk * 4;
        for (int t0q = 0; t0q < tasks; t0q += nthr) {
          const int id = t0q + threadIdx.x;
          const bool valid = id < tasks;
          const int idc = valid ? id : (id & 3);
          const int quarter = idc & 3, rb = idc >> 2;
          const int tt = rb / nblk, blk = rb - tt * nblk;
          const int j = start + b0 + tt;
          const int k0 = blk * 32 + quarter * 8;
          float rr[8];
          if (blk * 32 < K) {
            const f32x4* src = (const f32x4*)(xf + (size_t)j * K + k0);
            const f32x4 v0 = src[0], v1 = src[1];
            rr[0] = v0[0]; rr[1] = v0[1]; rr[2] = v0[2]; rr[3] = v0[3];
            rr[4] = v1[0]; rr[5] = v1[1]; rr[6] = v1[2]; rr[7] = v1[3];
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) rr[i] = 0.0f;
          }
          const int gi = tt / TPG, c = blk >> 2, gg = blk & 3;
#pragma unroll
          for (int p = 0; p < P; ++p) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(rr[i]));
            amax = fmaxf(amax, lane_xor1(amax));
            amax = fmaxf(amax, lane_xor2(amax));
            const uint32_t sc = e8m0_for_amax(amax);
            const float inv = __uint_as_float((254u - sc) << 23);
            const float scf = sc ? __uint_as_float(sc << 23) : __uint_as_float(0x00400000u);
            uint32_t lo, hi;
            e4m3_piece8(rr, inv, scf, lo, hi);
            if (valid) {
              const int m = (tt - gi * TPG) * P + p;
              *(uint2*)(lds + gi * kMxGroupBytes + m * kMxRowStride + k0) = make_uint2(lo, hi);
              if (quarter == 0)
                lds[gi * kMxGroupBytes + 16 * kMxRowStride + m * kMxSclRow + gg * kMxSclRun + c] =
                    (uint8_t)sc;
            }
          }
        }
      } else {
        // Stage the batch: 16-byte units, kFill loads in flight per thread.
        // Units past the end repeat the last one (same data to the same place).
        constexpr int kFill = NCT == 23 ? 8 : 4;
        const int row16 = Kp >> 4;
        const int units = row16 + kMxSclRow / 16;
        const int total_units = nb * P * units;
        for (int u0 = threadIdx.x; u0 < total_units; u0 += kFill * nthr) {
          u32x4 v[kFill];
          uint32_t dst[kFill];
#pragma unroll
          for (int i = 0; i < kFill; ++i) {
            const int uu = min(u0 + i * nthr, total_units - 1);
            const int rp = uu / units, c = uu - rp * units;
            const int tt = rp / P, p = rp - tt * P;
            const int j = start + b0 + tt;
            const int row = arow_mode == 0 ? rowmap[tt] / k_top : arow_mode == 1 ? rowmap[tt] : j;
            const int gi = tt / TPG, m = (tt - gi * TPG) * P + p;
            const size_t prow = (size_t)row * P + p;
            const uint8_t* src = c < row16 ? q + prow * Kp + c * 16
                                           : qs + prow * kMxSclRow + (c - row16) * 16;
            if constexpr (kWait) {
              // other workgroups of this launch wrote the pieces (device scope)
              const uint64_t lo = load_dev((const uint64_t*)src);
              const uint64_t hi = load_dev((const uint64_t*)src + 1);
              v[i] = u32x4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
            } else {
              v[i] = *(const u32x4*)src;
            }
            dst[i] = c < row16 ? gi * kMxGroupBytes + m * kMxRowStride + c * 16
                               : gi * kMxGroupBytes + 16 * kMxRowStride + m * kMxSclRow +
                                     (c - row16) * 16;
          }
#pragma unroll
          for (int i = 0; i < kFill; ++i) *(u32x4*)(lds + dst[i]) = v[i];
        }
      }
      lds_barrier();  // (the staging's loads have been waited for)
    }
    const int ngroups = (nb + TPG - 1) / TPG;
    const int u_next = u + len;
    MxSeg nx = {-1, 0, 0, 0};
    if (u_next < uend) nx = seg_at(u_next);

    // MFMAs of chunks [C0, C0 + NH) of one operand group, from register half w.
    auto run_half = [&](auto c0v, auto nhv, const u32x4* w, int gi, f32x4& acc) {
      constexpr int C0 = decltype(c0v)::value, NH = decltype(nhv)::value;
      const uint32_t ar = gi * kMxGroupBytes + r * kMxRowStride + 16 * g;
      const uint8_t* as = lds + gi * kMxGroupBytes + 16 * kMxRowStride + r * kMxSclRow +
                          g * kMxSclRun;
      // A operands stream from LDS one chunk ahead of the MFMA chain.  Each
      // chunk's offset passes through an opaque asm, so its reads cannot be
      // hoisted ahead of the chain (which would hold all chunks in registers);
      // the scheduling barrier after each MFMA keeps at most two chunks live.
      auto load_a = [&](int c) {
        uint32_t o = ar + 128 * c;
        asm volatile("" : "+v"(o));
        const u32x4 a0 = *(const u32x4*)(lds + o);
        const u32x4 a1 = *(const u32x4*)(lds + o + 64);
        return i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                     (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      };
      // An opaque copy of this lane's staged scale row offset keeps the
      // compiler from hoisting the per-chunk reads out of the group loop.
      uint32_t ss = sstage_off;
      asm volatile("" : "+v"(ss));
      uint32_t sa = *(const uint32_t*)(as + (C0 & ~3));
      uint32_t sb = scale_b(ss, C0);
      i32x8 acur = load_a(C0);
      static_for<0, NH>([&](auto jv) {
        constexpr int j = decltype(jv)::value;
        constexpr int c = C0 + j;
        i32x8 anext;
        uint32_t sa_next = 0, sb_next = 0;
        if constexpr (j + 1 < NH) {
          anext = load_a(c + 1);
          sb_next = scale_b(ss, c + 1);
          if constexpr ((c & 3) == 3) sa_next = *(const uint32_t*)(as + c + 1);
        }
        const i32x8 B = {(int)w[j][0], (int)w[j][1], (int)w[j][2], (int)w[j][3], 0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(acur, B, acc, 0, 4, c & 3, (int)sa,
                                                               0, (int)sb);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (j + 1 < NH) {
          acur = anext;
          sb = sb_next;
          if constexpr ((c & 3) == 3) sa = sa_next;
        }
      });
    };

    // Wave w computes tile w of the segment first (its first half was
    // prefetched); further tiles are handed out from an LDS counter when a
    // wave issues its next first half, so waves whose loads are served
    // faster take more tiles and the workgroup's waves finish together.
    for (int tl = wave; tl < len;) {
      int tl_next = len;
      const int tile = t0 + tl;
      const int r0 = tile << 4;
      issue_h1(e, tile);
      stage_scales();
      bn = bn_next;
      // One operand group: both halves and the epilogue.  The last group
      // issues the next tile's first half between its halves; it is peeled
      // out of the loop so the current first half is dead by then.
      auto do_group = [&](int gi, auto lastv) {
        constexpr bool last = decltype(lastv)::value;
          f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
          run_half(std::integral_constant<int, 0>{}, std::integral_constant<int, H0>{}, wa, gi, acc);
          // keeps the first-half MFMAs ahead of the (uniform) prefetch branch
          asm volatile("" : "+v"(acc));
          if constexpr (last) {
            // next first half: this segment's next tile, else this wave's first
            // tile of the next segment, else (nothing left) expert 0's tile 0,
            // the same for every such wave, so these loads hit in the caches.
            // Issued unconditionally: a branch here would make the waits of
            // the second half below count the new loads too.
            int grab = 0;
            if (lane == 0)
              grab = __hip_atomic_fetch_add(tile_ctr, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP);
            tl_next = __builtin_amdgcn_readfirstlane(grab) + nwaves;
            int ne = 0, nt = 0;
            if (tl_next < len) {
              ne = e;
              nt = t0 + tl_next;
            } else if (nx.e >= 0 && wave < nx.len) {
              ne = nx.e;
              nt = nx.t0 + wave;
            }
            issue_h0(ne, nt);
          }
          run_half(std::integral_constant<int, H0>{}, std::integral_constant<int, H1>{}, wb, gi, acc);
          // The MFMAs combine operands of all 64 lanes, so they must run with the
          // full wave active.  Their results are only stored under per-lane
          // conditions below; without this barrier the compiler may sink the
          // chains into those divergent branches.
          asm volatile("" : "+v"(acc));
          // lane (r, g): weight row r0 + r; operand rows 4g + i hold token
          // (4g + i) / P, piece (4g + i) % P of this group
          if constexpr (P == 4) {
            const int tt = gi * TPG + g;
            const float y = (((acc[3] + acc[2]) + acc[1]) + acc[0]) + bn;
            if (tt < nb) {
              const int j = start + b0 + tt;
              const int orow = orow_mode == 0 ? rowmap[tt] : j;
              out[(size_t)orow * out_ld + r0 + r] = y;
            }
          } else if constexpr (P == 3) {
            // Rows 3t + p hold piece p of token t (t < 5; row 15 unused), lane
            // group g rows 4g .. 4g + 3: group 0 holds token 0 and piece 0 of
            // token 1, group 1 the rest of token 1 and pieces 0, 1 of token 2,
            // group 2 piece 2 of token 2 and token 3, group 3 token 4.  The
            // straddling shares come from the next lane group (lane + 16).
            // Sums run from the smallest piece up, as for P = 4.
            const float send = g == 1 ? acc[1] + acc[0] : acc[0];
            const float recv = __shfl_down(send, 16, kWave);
            float y0, y1 = 0.0f;
            int l0 = g + 1;  // local token of y0 (y1: token 1 of group 0)
            if (g == 0) {
              y0 = ((acc[2] + acc[1]) + acc[0]) + bn;
              y1 = (recv + acc[3]) + bn;
              l0 = 0;
            } else if (g == 1) {
              y0 = ((recv + acc[3]) + acc[2]) + bn;
            } else if (g == 2) {
              y0 = ((acc[3] + acc[2]) + acc[1]) + bn;
            } else {
              y0 = ((acc[2] + acc[1]) + acc[0]) + bn;
            }
  #pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int tt = gi * TPG + (h == 0 ? l0 : 1);
              if ((h == 0 || g == 0) && tt < nb) {
                const int j = start + b0 + tt;
                const int orow = orow_mode == 0 ? rowmap[tt] : j;
                float* dst = out + (size_t)orow * out_ld + r0 + r;
                // the decode launch's mlp2: device scope (sc1), read by the
                // gated combine of other workgroups
                if constexpr (kWait)
                  __hip_atomic_store(dst, h == 0 ? y0 : y1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
                else
                  *dst = h == 0 ? y0 : y1;
              }
            }
          } else {
            const float y0 = (acc[1] + acc[0]) + bn;
            const float y1 = (acc[3] + acc[2]) + bn;
            const int tt0 = gi * TPG + 2 * g;
            if constexpr (kEpi == 1 || kEpi == 3) {
              const float l0 = lane_xor1(y0);  // odd rows hold the linear half
              const float l1 = lane_xor1(y1);
              if ((r & 1) == 0) {
                const float yy[2] = {y0, y1}, ll[2] = {l0, l1};
  #pragma unroll
                for (int h = 0; h < 2; ++h) {
                  if (tt0 + h < nb) {
                    const int j = start + b0 + tt0 + h;
                    const int orow = orow_mode == 0 ? rowmap[tt0 + h] : j;
                    const float xg = fminf(yy[h], limit);
                    const float xl = fminf(fmaxf(ll[h], -limit), limit);
                    const float z = __fmul_rn(alpha, xg);
                    const float sig = 1.0f / (1.0f + expf(-z));
                    const float v = __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
                    if constexpr (kEpi == 1)
                      out[(size_t)orow * out_ld + ((r0 + r) >> 1)] = v;
                    else
                      act_t[(tt0 + h) * act_ld + ((r0 + r) >> 1) - act_c0] = v;
                  }
                }
              }
            } else {
              const float yy[2] = {y0, y1};
  #pragma unroll
              for (int h = 0; h < 2; ++h) {
                if (tt0 + h < nb) {
                  const int j = start + b0 + tt0 + h;
                  const int orow = orow_mode == 0 ? rowmap[tt0 + h] : j;
                  out[(size_t)orow * out_ld + r0 + r] = yy[h];
                }
              }
            }
          }
      };
      // Unrolled (ngroups <= kMxMaxGroups): a runtime loop holding stores and
      // no loads gets a full vmcnt(0) in its preheader from the compiler,
      // which would wait for the second half's loads before the first half.
      static_for<0, kMxMaxGroups - 1>([&](auto gv) {
        if (decltype(gv)::value < ngroups - 1) do_group(decltype(gv)::value, std::false_type{});
      });
      do_group(ngroups - 1, std::true_type{});
      tl = tl_next;
    }
    // a wave without tiles in this segment starts its next-segment tile now
    if (wave >= len && nx.e >= 0) issue_h0(nx.e, nx.t0 + (wave < nx.len ? wave : 0));
    u = u_next;
    sg = nx;
  }
}

// arow_mode: piece row of sorted position j: 0 = sorted_pairs[j] / k_top
// (token), 1 = sorted_pairs[j] (pair), 2 = j.  orow_mode: output row: 0 =
// sorted_pairs[j], 1 = j.  kEpi: 0 = store y (N columns), 1 = interleaved
// SwiGLU (N/2 columns), 2 = store y with the activations given as fp32 rows
// (arow_mode 2), encoded into P pieces while they are staged; 3 = (P = 2,
// one segment per share) the SwiGLU outputs kept in LDS (MxLds::act).
template <int P, int kEpi, int NCT>
__global__ __launch_bounds__(NCT == 23 ? 768 : 512) void moe_mx_gemv_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ qs, int Kp,
    const int* __restrict__ indptr, const int* __restrict__ sorted_pairs, int k_top,
    int arow_mode, int orow_mode, const uint8_t* __restrict__ blocks,
    const uint8_t* __restrict__ scales, const uint16_t* __restrict__ bias, int N, int G, int E,
    int groups_cap, float alpha, float limit, float* __restrict__ out, int out_ld, int xcds) {
  extern __shared__ __align__(16) uint8_t lds[];
  // LDS: [groups_cap A operand groups][per-wave scale staging][E+1 unit
  // prefix][E+1 indptr][sorted_pairs of one batch, kMxRowMap ints][tile counter]
  MxLds L;
  L.sstage = groups_cap * mx_group_bytes(NCT);
  L.pre = L.sstage + (int)(blockDim.x >> 6) * (16 * G);
  L.ipl = L.pre + 4 * (E + 1);
  L.rowmap = L.ipl + 4 * (E + 1);
  L.tile_ctr = L.rowmap + 4 * kMxRowMap;
  L.act = 0;
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0)
    mx_unit_prefix(indptr, E, groups_cap * (16 / P), N >> 4, (int*)(lds + L.pre),
                   (int*)(lds + L.ipl));
  __syncthreads();
  MxSeg first;
  mx_pass<P, kEpi, NCT, false>(lds, L, q, qs, Kp, sorted_pairs, k_top, arow_mode, orow_mode,
                               blocks, scales, bias, N, G, E, groups_cap, alpha, limit, out,
                               out_ld, xcds, 1, [](int, int, int) {}, first, (int)blockDim.x,
                               true);
}

// ---------------------------------------------------------------------------
// Decode chain in one launch: mlp1 with the interleaved SwiGLU, the encoding
// of act into three fp8 pieces, and mlp2 (model/mlp.py:387-395 with the
// expert grouping of mxfp4_moe_mlp1/2_decode, model/mlp_optimized.py:
// 214-660).  Phase 1 is the mlp1 pass (two pieces of t, 16 tokens per batch)
// with one segment per workgroup whose share starts and ends on 32-column
// blocks of act; its SwiGLU outputs stay in LDS, and the workgroup encodes
// its blocks of act itself (as moe_pieces_kernel<3, true> would from the fp32
// rows) and adds its tile count to done[e].  Phase 2 is the mlp2 pass over
// those pieces; each workgroup issues its first tile's weight loads, then
// waits until done[e] counts all of expert e's mlp1 tiles before staging, so
// mlp2's start overlaps mlp1's tail.
//
// Coherence across the XCDs' L2s without writing back or invalidating them:
// the act pieces are stored and (by the staging DMA) loaded with device
// scope (sc1), the code sequence of agent-scope atomic stores and loads, and
// the counts are agent-scope atomics.  Every wave waits for its own stores
// to complete (vmcnt(0): on gfx9 the count covers stores, and a completed
// sc1 store is visible at device scope) before the workgroup barrier after
// which one thread adds the count; a waiting workgroup issues its staging
// only after its count load returned the target.  The barrier alone would
// not order them: a workgroup-scope fence waits for LDS traffic only.
//
// Requirements (checked by the launcher): H == I with 23 chunks of 128, one
// workgroup per CU and every workgroup resident at once (the grid is the CU
// count and nothing else runs on the device: a workgroup waiting in phase 2
// relies on the phase-1 work of the others), at most 64 mlp1 batches, and
// done[0..E) and *status zero at launch.  The wait is bounded (spin_max
// polls): a workgroup that gives up adds 1 to *status and goes on, so the
// launch always ends; its y rows are then wrong and the status says so.
constexpr int kDecodeGroups1 = 2;  // mlp1 batch: 2 groups of 8 tokens
constexpr int kDecodeSpinMax = 1 << 20;  // about a second of polling

// The gated combine of one token's 4 columns c0 .. c0 + 3 (model/mlp.py:
// 346-362 and the residual of :402), as moe_gating_kernel computes it: fp32
// sum over slots r = 0..k-1 in order of y[token, r] * w[token, r], multiply and
// add rounded separately, bf16, then bf16(x + moe).  y rows are read with
// device scope (sc1: other workgroups wrote them with sc1 stores), 16 bytes a
// lane, so four lanes read one 64-byte row segment; every load of up to 4
// slots is issued before the first use.  A nonzero status (a wait gave up)
// makes the columns NaN.
__device__ __forceinline__ void combine4(__amdgpu_buffer_rsrc_t yr, const uint16_t* w,
                                         const uint16_t* x, uint16_t* out, const int* status,
                                         int tok, int k, int H, int c0) {
#pragma clang fp contract(off)
  const int st = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint2 xv = *(const uint2*)(x + (size_t)tok * H + c0);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int r0 = 0; r0 < k; r0 += 4) {
    u32x4 v[4];
    float wr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (r0 + q < k) {
        const int pr = tok * k + r0 + q;
        wr[q] = bf2f(w[pr]);
        v[q] = __builtin_amdgcn_raw_buffer_load_b128(yr, (pr * H + c0) * 4, 0, kCpolSc1);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (r0 + q < k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] + __uint_as_float(v[q][i]) * wr[q];
      }
    }
  }
  uint32_t o[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t xw = j == 0 ? xv.x : xv.y;
    const float x0 = __uint_as_float(xw << 16), x1 = __uint_as_float(xw & 0xFFFF0000u);
    const uint32_t a = f2bf(__fadd_rn(x0, bf2f(f2bf(acc[2 * j]))));
    const uint32_t b = f2bf(__fadd_rn(x1, bf2f(f2bf(acc[2 * j + 1]))));
    o[j] = st != 0 ? 0x7FC07FC0u : a | (b << 16);
  }
  *(uint2*)(out + (size_t)tok * H + c0) = make_uint2(o[0], o[1]);
}
// The decode launch's own routing (logits null: indptr and sorted_pairs are
// given).  With logits ([n][E] floats holding bf16 values, E <= 32, n E <=
// kDecodeRouteKeys) every workgroup ranks them in LDS with the router's
// ranking code, counts each expert's pairs, takes indptr from the counts and
// finds its two batches' pairs in the grouping's stable order (token, then
// slot, within an expert) by ballots over the pairs' experts, without a full
// sort.  The routing outputs are written on the way, spread out: token t's
// gate weights (the router's fp64 softmax) and experts by workgroup t, each
// batch's grouping entries (sorted_pairs, token_indices, expert_ids,
// pair_pos) by the workgroup whose mlp2 share starts at the batch's first
// tile, indptr by workgroup 0; the gating launch after this one reads w.  The
// router is then one logits launch: its last-arriver selection (a
// device-scope count, then one workgroup ranking and grouping every token)
// took about 9 of its 14 us at 64 tokens, and the routing here costs the
// decode launch about 4.
struct DecodeRoute {
  const float* logits;
  int n;
  int32_t* idx;
  uint16_t* w;
  int32_t* indptr;
  int32_t* sorted_pairs;
  int32_t* token_indices;
  int32_t* expert_ids;
  int32_t* pair_pos;
};
constexpr int kDecodeRouteKeys = 4096;

__global__ __launch_bounds__(768) void moe_mx_decode_kernel(
    const uint8_t* __restrict__ tq, const uint8_t* __restrict__ tqs,
    const int* __restrict__ indptr, const int* __restrict__ sorted_pairs, int k_top,
    const uint8_t* __restrict__ blocks1, const uint8_t* __restrict__ scales1,
    const uint16_t* __restrict__ bias1, const uint8_t* __restrict__ blocks2,
    const uint8_t* __restrict__ scales2, const uint16_t* __restrict__ bias2, int H, int E,
    int gcap2, float alpha, float limit, uint8_t* aq, uint8_t* aqs, float* __restrict__ y,
    int* done, int* status, int spin_max, int prepoll, int xcds, const uint16_t* __restrict__ gw,
    const uint16_t* __restrict__ resid, uint16_t* __restrict__ out, int* arrive, DecodeRoute rt) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int kGroupBytes = mx_group_bytes(23);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nthr = blockDim.x;  // read once (a vector load from the dispatch packet)
  const int nwaves = nthr >> 6;
  const int G = H >> 5, Kp = 23 * 128;
  const int ntiles1 = (2 * H) >> 4, ntiles2 = H >> 4;
  const int tpb1 = kDecodeGroups1 * 8;
  // LDS: [kMxMaxGroups operand groups: phase 2's batch; phase 1's two groups
  // and, in the third, its SwiGLU outputs][scale staging][phase-1 prefix]
  // [indptr][row map][tile counter][phase-2 prefix]
  MxLds L1;
  L1.sstage = kMxMaxGroups * kGroupBytes;
  L1.pre = L1.sstage + nwaves * (16 * G);
  L1.ipl = L1.pre + 4 * (E + 1);
  L1.rowmap = L1.ipl + 4 * (E + 1);
  L1.tile_ctr = L1.rowmap + 4 * kMxRowMap;
  L1.act = kDecodeGroups1 * kGroupBytes;
  MxLds L2 = L1;
  L2.pre = L1.tile_ctr + 16;
  L2.rowmap = L1.rowmap + 64;  // phase 1's batch: 16 entries at most, phase 2's: 15
  const int* const ipl = (const int*)(lds + L1.ipl);
  constexpr int tpb2 = kMxMaxGroups * 5;  // (gcap2 == kMxMaxGroups)
  // the 16 bytes at tile_ctr: [0] the pass's tile counter, [1..2] phase 2's
  // share, [3] the combine's job count
  int* const share2 = (int*)(lds + L1.tile_ctr + 4);
  if (threadIdx.x == 0) *(int*)(lds + L1.tile_ctr + 12) = 0;
  const bool route = rt.logits != nullptr;
  if (route) {
    // Scratch in the operand groups (free until phase 1's staging).
    const int n = rt.n, np = n * k_top, tid = threadIdx.x;
    const int lane = tid & 63;
    float* lg = (float*)lds;                  // [n][E]
    uint32_t* wk = (uint32_t*)(lds + 16384);  // the ranked keys, [t][k]
    int* pidx = (int*)(lds + 18432);          // each pair's expert
    int* cnt = (int*)(lds + 20480);           // [E]
    int* ipl2 = (int*)(lds + 21504);          // wave 1's copy of indptr, [E + 1]
    int* const ipl_w = (int*)(lds + L1.ipl);
    for (int i = tid; i < (n * E) >> 2; i += nthr)
      ((f32x4*)lg)[i] = ((const f32x4*)rt.logits)[i];
    for (int e = tid; e < E; e += nthr) cnt[e] = 0;
    __syncthreads();
    rank_halves(lg, n, E, k_top, wk, nwaves, [&](int t, int j, uint32_t key) {
      const int e = key_expert(key);
      pidx[t * k_top + j] = e;
      atomicAdd(&cnt[e], 1);
    });
    __syncthreads();
    // indptr (the exclusive prefix of the counts), by the wave that needs it
    auto wave_indptr = [&](int* dst) {
      int carry = 0;
      for (int b = 0; b < E; b += 64) {
        const int e = b + lane;
        const int c = e < E ? cnt[e] : 0;
        int v = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int u = __shfl_up(v, o, kWave);
          if (lane >= o) v += u;
        }
        if (e < E) dst[e] = carry + v - c;
        carry += __shfl(v, 63, kWave);
      }
      if (lane == 0) dst[E] = carry;
    };
    // The pairs of batch (e, b0, nb) in the grouping's stable order (token,
    // then slot, within an expert) by one wave: ballots over the pairs'
    // experts rank each pair among its expert's; rank b0 + tt goes to
    // rowmap[tt], and with `out` the batch's grouping entries (sorted
    // position ipl[e] + rank) are written.
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    auto batch_pairs = [&](const int* ip, int e, int b0, int nb, int* rowmap, bool out) {
      int seen = 0;
      for (int c0 = 0; c0 < np; c0 += 64) {
        const int p = c0 + lane;
        const bool m = p < np && pidx[p] == e;
        const uint64_t bal = __ballot(m);
        const int r = seen + __popcll(bal & lt) - b0;
        if (m && r >= 0 && r < nb) {
          rowmap[r] = p;
          if (out) {
            const int pos = ip[e] + b0 + r;
            rt.sorted_pairs[pos] = p;
            rt.token_indices[pos] = p / k_top;
            rt.expert_ids[pos] = e;
            rt.pair_pos[p] = pos;
          }
        }
        seen += __popcll(bal);
      }
    };
    if (wave == 0) {
      // phase 1's batch (mx_share's batch split, as mx_pass computes it)
      int* pre1 = (int*)(lds + L1.pre);
      wave_indptr(ipl_w);
      mx_unit_prefix(ipl, E, tpb1, ntiles1, pre1, nullptr);
      int ub, ue;
      mx_share(pre1, E, ntiles1, 4, xcds, ub, ue);
      if (ub < ue) {
        const int e1 = mx_expert_of(pre1, E, ub);
        const int b0 = (ub - pre1[e1]) / ntiles1 * tpb1;
        batch_pairs(ipl, e1, b0, min(tpb1, ipl[e1 + 1] - ipl[e1] - b0), (int*)(lds + L1.rowmap),
                    false);
      }
    } else if (wave == 1) {
      // phase 2's batch (the weighted share); the workgroup whose share starts
      // at the batch's first tile (one per batch) writes its grouping entries
      int* pre2 = (int*)(lds + L2.pre);
      wave_indptr(ipl2);
      mx_unit_prefix(ipl2, E, tpb2, ntiles2, pre2, nullptr);
      mx_weighted_share(ipl2, E, tpb2, 5, 5, ntiles2, 1, xcds, share2);
      const int ub = share2[0], ue = share2[1];
      if (ub < ue) {
        const int e2 = mx_expert_of(pre2, E, ub);
        const int b0 = (ub - pre2[e2]) / ntiles2 * tpb2;
        batch_pairs(ipl2, e2, b0, min(tpb2, ipl2[e2 + 1] - ipl2[e2] - b0),
                    (int*)(lds + L2.rowmap), (ub - pre2[e2]) % ntiles2 == 0);
      }
    } else if (wave == 2 && (int)blockIdx.x < n) {
      // token blockIdx.x's gate weights and experts: the router's softmax
      // (fp64, summed in rank order)
      const int t = blockIdx.x;
      const double ex = lane < k_top ? pair_exp(wk, t * k_top + lane, k_top) : 0.0;
      double sum = readlane_f64(ex, 0);
      for (int jj = 1; jj < k_top; ++jj) sum += readlane_f64(ex, jj);
      if (lane < k_top) {
        rt.w[t * k_top + lane] = f64_to_bf16_via_f32(ex / sum);
        rt.idx[t * k_top + lane] = pidx[t * k_top + lane];
      }
    } else if (wave == 3 && blockIdx.x == 0) {
      int* ipl3 = ipl2 + (E + 1);  // wave 3's copy
      wave_indptr(ipl3);
      for (int e = lane; e <= E; e += 64) rt.indptr[e] = ipl3[e];
    }
    __syncthreads();
  } else {
    if (wave == 0)
      mx_unit_prefix(indptr, E, tpb1, ntiles1, (int*)(lds + L1.pre), (int*)(lds + L1.ipl));
    else if (wave == 1)
      mx_unit_prefix(indptr, E, tpb2, ntiles2, (int*)(lds + L2.pre), nullptr);
    __syncthreads();
  }

  MxSeg s1;
  auto no_wait = [](int, int, int) {};
  mx_pass<2, 3, 23, false, decltype(no_wait)&>(
      lds, L1, tq, tqs, Kp, sorted_pairs, k_top, 0, 1, blocks1, scales1, bias1, 2 * H, G, E,
      kDecodeGroups1, alpha, limit, nullptr, 0, xcds, 4, no_wait, s1, nthr, false, nullptr, route);
  lds_barrier();  // every wave's SwiGLU outputs are in LDS
  // Phase 2's share, weighted by the batches' operand groups, from the LDS
  // copy of indptr (at the launch's start its global loads held every wave
  // about 2 us at the first barrier); the publish barrier below makes it
  // visible.
  if (wave == 1 && !route) mx_weighted_share(ipl, E, tpb2, 5, 5, ntiles2, 1, xcds, share2);
  if (s1.e >= 0) {
    // Encode the share's act blocks: four threads per (token, 32-column
    // block), 8 columns each; the share that ends at column H also writes the
    // zero blocks up to 128 * 23 and clears the unused scale slots.
    const int start = ipl[s1.e];
    const int nb = min(tpb1, ipl[s1.e + 1] - start - s1.b0);
    const int act_ld = s1.len * 8, nblk = act_ld >> 5, blk0 = s1.t0 >> 2;
    const int nbt = nblk + (s1.t0 + s1.len == ntiles1 ? 4 * 23 - G : 0);
    const int tasks = nb * nbt * 4;
    const float* act = (const float*)(lds + L1.act);
    for (int t0q = 0; t0q < tasks; t0q += nthr) {
      const int id = t0q + threadIdx.x;
      const bool valid = id < tasks;
      const int idc = valid ? id : (id & 3);
      const int quarter = idc & 3, rb = idc >> 2;
      const int tt = rb / nbt, bl = rb - tt * nbt;
      const int blk = blk0 + bl, c = blk >> 2, gg = blk & 3;
      const int k0 = blk * 32 + quarter * 8;
      float rr[8];
      if (bl < nblk) {
        const f32x4* src = (const f32x4*)(act + tt * act_ld + bl * 32 + quarter * 8);
        const f32x4 v0 = src[0], v1 = src[1];
        rr[0] = v0[0]; rr[1] = v0[1]; rr[2] = v0[2]; rr[3] = v0[3];
        rr[4] = v1[0]; rr[5] = v1[1]; rr[6] = v1[2]; rr[7] = v1[3];
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) rr[i] = 0.0f;
      }
      const size_t j = (size_t)(start + s1.b0 + tt);
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(rr[i]));
        amax = fmaxf(amax, lane_xor1(amax));
        amax = fmaxf(amax, lane_xor2(amax));
        const uint32_t sc = e8m0_for_amax(amax);
        const float inv = __uint_as_float((254u - sc) << 23);
        const float scf = sc ? __uint_as_float(sc << 23) : __uint_as_float(0x00400000u);
        uint32_t lo, hi;
        e4m3_piece8(rr, inv, scf, lo, hi);
        if (!valid) continue;
        const size_t prow = j * 3 + p;
        store_dev((uint64_t*)(aq + prow * Kp + k0), ((uint64_t)hi << 32) | lo);
        if (quarter == 0) {
          uint8_t* run = aqs + prow * kMxSclRow + gg * kMxSclRun;
          store_dev(run + c, (uint8_t)sc);
          if (c == 22)
            for (int z = 23; z < kMxSclRun; ++z) store_dev(run + z, (uint8_t)0);
        }
      }
    }
    // Publish: each wave waits until its device-scope stores have completed
    // (visible to every XCD), then the barrier, then the count.
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(done + s1.e, s1.len, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    lds_barrier();  // (no share in phase 1) phase 2's share is in LDS
  }

  // Phase 2: wait for all of expert e's mlp1 tiles, then stage its pieces.
  // One thread polls done[e], at most spin_max times, sleeping between
  // polls; spin_max == 0 gives up without polling.  With prepoll the first
  // poll is issued before the segment's tile loads (pre) and read here.
  struct WaitMlp1 {
    const int* ipl;
    int* done;
    int* status;
    int spin_max, ntiles1, tpb1, prepoll;
    int first;
    __device__ __forceinline__ int target(int e) const {
      return ntiles1 * ((ipl[e + 1] - ipl[e] + tpb1 - 1) / tpb1);
    }
    __device__ __forceinline__ void pre(int e) {
      if (threadIdx.x == 0 && spin_max > 0 && prepoll)
        first = __hip_atomic_load(done + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __device__ __forceinline__ void operator()(int e, int, int) {
      if (threadIdx.x == 0) {
        const int tg = target(e);
        const bool pre_polled = prepoll && spin_max > 0;
        bool seen = pre_polled && first >= tg;
        for (int it = pre_polled ? 1 : 0; !seen && it < spin_max; ++it) {
          seen = __hip_atomic_load(done + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= tg;
          if (!seen) __builtin_amdgcn_s_sleep(2);
        }
        // gave up: the staged pieces may be incomplete; report it
        if (!seen) __hip_atomic_fetch_add(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      lds_barrier();  // the staging's sc1 loads are issued after the count was seen
    }
  };
  WaitMlp1 wait_mlp1{ipl, done, status, spin_max, ntiles1, tpb1, prepoll, 0};
  MxSeg s2;
  mx_pass<3, 0, 23, true, decltype(wait_mlp1)&>(
      lds, L2, aq, aqs, Kp, sorted_pairs, k_top, 2, 0, blocks2, scales2, bias2, H, G, E,
      kMxMaxGroups, 0.0f, 0.0f, y, H, xcds, 1, wait_mlp1, s2, nthr, false, share2, route);

  // The gated combine (with the residual), done by whichever workgroup writes
  // a token's last y tile: every workgroup holds one mlp2 segment (a batch's
  // tiles t0 .. t0 + len - 1), so after its stores complete it counts each
  // (token, 16-column tile) it produced; the count that reaches k_top makes
  // that tile a combine job of this workgroup, and four lanes take each job.
  // No workgroup waits here.
  if (out != nullptr && s2.e >= 0) {
    wait_vmcnt<0>();  // this wave's y stores are complete (visible to every XCD)
    __syncthreads();  // and every wave's; the pass no longer reads the LDS
    const int start = ipl[s2.e];
    const int nb = min(tpb2, ipl[s2.e + 1] - start - s2.b0);
    const int* rowmap = (const int*)(lds + L2.rowmap);  // the batch's sorted_pairs entries
    int* jobs = (int*)lds;                               // at most 15 x 180 ints
    int* njobs = (int*)(lds + L2.tile_ctr + 12);         // zero since the start
    for (int id = threadIdx.x; id < nb * s2.len; id += nthr) {
      const int tt = id / s2.len, tile = s2.t0 + id - tt * s2.len;
      const int job = rowmap[tt] / k_top * ntiles2 + tile;
      const int prev = __hip_atomic_fetch_add(arrive + job, 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      if (prev == k_top - 1) jobs[atomicAdd(njobs, 1)] = job;
    }
    __syncthreads();
    const int nj = *njobs;
    const __amdgpu_buffer_rsrc_t yr =
        __builtin_amdgcn_make_buffer_rsrc(y, (short)0, ipl[E] * H * 4, kBufferWord3);
    for (int q = threadIdx.x; q < nj * 4; q += nthr) {
      const int job = jobs[q >> 2];
      const int tok = job / ntiles2;
      combine4(yr, gw, resid, out, status, tok, k_top, H, (job - tok * ntiles2) * 16 + (q & 3) * 4);
    }
  }
}

// ---------------------------------------------------------------------------
// One token: mlp1, then mlp2 with the gated combine, as two launches in which
// every wave holds one 16-row weight tile and issues all of its loads at
// once.  With one token a persistent pass gives each wave under one tile, so
// its unit prefix (a global load ahead of the first weight address), its
// two-stage pipeline and the gating launch after mlp2 are latency only.
// Here the first weight address needs only the token's k expert indices, and
// each mlp2 workgroup owns 16 output columns for all k experts (one wave per
// slot), so the k rows are combined in LDS.  The arithmetic is that of
// moe_mx_gemv_kernel (the same operand layout, the same MFMA chain over the
// 23 chunks, the same epilogues and act encoding) and of moe_gating_kernel,
// so the outputs equal those launches' bit for bit.

constexpr int kT1Nct = 23;  // K chunks (K = 32 G with 89 <= G <= 92)
constexpr int kT1Kp = kT1Nct * 128;

// One wave's 16-row weight tile: 23 chunks, its scale bytes and the bias of
// this lane's row.
struct T1Tile {
  u32x4 w[kT1Nct];
  u32x4 sc0, sc1;
  float bn;
};

// Block index of chunk c for lane group g: 4 c + g; only the last chunk can
// pass K (then block G - 1 is re-read; its A bytes are zero).
__device__ __forceinline__ int t1_blk(int c, int g, int G) {
  return c < kT1Nct - 1 ? 4 * c + g : min(4 * c + g, G - 1);
}

__device__ __forceinline__ void t1_issue(T1Tile& t, const uint8_t* __restrict__ blocks,
                                         const uint8_t* __restrict__ scales,
                                         const uint16_t* __restrict__ bias, size_t row0, int G) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const uint8_t* st = scales + row0 * G;  // 16 rows x G bytes, contiguous
  t.sc0 = *(const u32x4*)(st + min(lane, G - 1) * 16);
  t.sc1 = *(const u32x4*)(st + min(lane + 64, G - 1) * 16);
  t.bn = bf2f(bias[row0 + r]);
  const uint8_t* wp = blocks + (row0 + r) * G * 16;
  static_for<0, kT1Nct>([&](auto cv) {
    constexpr int c = decltype(cv)::value;
    t.w[c] = *(const u32x4*)(wp + t1_blk(c, g, G) * 16);
  });
}

// The tile's scale bytes to this wave's LDS staging (16 G bytes), from which
// lane (r, g) reads row r's byte of each block it multiplies.  Lanes past
// the G units store unit G - 1 again (the bytes they loaded): no branch, so
// the compiler cannot sink a scale load into one, behind the chunk loads.
__device__ __forceinline__ void t1_stage_scales(const T1Tile& t, uint8_t* sstage, int G) {
  const int lane = threadIdx.x & 63;
  *(u32x4*)(sstage + min(lane, G - 1) * 16) = t.sc0;
  *(u32x4*)(sstage + min(lane + 64, G - 1) * 16) = t.sc1;
}

// The MFMA chain of one tile over chunks 0..22 in order against A rows in
// LDS: `arows` piece rows at `a_base` (row stride mx_row_stride(23)), their
// scale rows right after them (kMxSclRow each).  MFMA rows at or past arows
// read row 0: their outputs are not used.  ss: this wave's staged weight
// scale bytes.
__device__ __forceinline__ f32x4 t1_chain(const uint8_t* lds, uint32_t a_base, int arows,
                                          uint32_t ss, const T1Tile& t, int G) {
  constexpr int kRS = mx_row_stride(kT1Nct);
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int ra = r < arows ? r : 0;
  const uint32_t ar = a_base + ra * kRS + 16 * g;
  const uint32_t as = a_base + arows * kRS + ra * kMxSclRow + g * kMxSclRun;
  const uint32_t sr = ss + r * G;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  static_for<0, kT1Nct>([&](auto cv) {
    constexpr int c = decltype(cv)::value;
    const u32x4 a0 = *(const u32x4*)(lds + ar + 128 * c);
    const u32x4 a1 = *(const u32x4*)(lds + ar + 128 * c + 64);
    const i32x8 A = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                     (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    const uint32_t sa = *(const uint32_t*)(lds + as + (c & ~3));
    const uint32_t sb = lds[sr + t1_blk(c, g, G)];
    const i32x8 B = {(int)t.w[c][0], (int)t.w[c][1], (int)t.w[c][2], (int)t.w[c][3], 0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 0, 4, c & 3, (int)sa, 0,
                                                           (int)sb);
  });
  return acc;
}

// The one-token launches route the token themselves from its E <= 32
// logits (each wave: the router's one-token top-k and softmax, registers
// only), so the router is its logits launch alone.  The first mlp1
// workgroup writes the routing outputs.
struct Token1Route {
  int32_t* idx;
  uint16_t* w;
  int32_t* indptr;
  int32_t* sorted_pairs;
  int32_t* token_indices;
  int32_t* expert_ids;
  int32_t* pair_pos;
};

// mlp1 of one token with the interleaved SwiGLU epilogue: workgroup
// (q, slot) holds 4 waves, wave v the weight tile 4 q + v (16 rows: 8 gate
// and 8 linear, interleaved) of the expert of rank `slot`; act row `slot`
// ([k][I], fp32) gets its 8 columns.  t's two pieces (rows 0 and 1 of tq,
// scale rows of tqs) are staged in LDS.
__global__ __launch_bounds__(256) void moe_mx_token1_mlp1_kernel(
    const uint8_t* __restrict__ tq, const uint8_t* __restrict__ tqs,
    const float* __restrict__ logits, int E, Token1Route rt, const uint8_t* __restrict__ blocks,
    const uint8_t* __restrict__ scales, const uint16_t* __restrict__ bias, int N, int G,
    float alpha, float limit, uint8_t* __restrict__ aq, uint8_t* __restrict__ aqs) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int kRS = mx_row_stride(kT1Nct);
  constexpr int kUnits = kT1Kp / 16, kSclUnits = kMxSclRow / 16;
  constexpr int kStage = 2 * (kUnits + kSclUnits);  // 16-byte units of the two piece rows
  static_assert(kStage <= 2 * 256, "two units a thread");
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = blockIdx.y, k = gridDim.y;
  const int tile = blockIdx.x * 4 + wave;
  // the logits and the staging's loads first (they complete first), then the
  // tile's, once the token's experts are known
  const float v = lane < E ? logits[lane] : 0.0f;
  u32x4 sv[2];
  uint32_t sd[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = min((int)threadIdx.x + 256 * i, kStage - 1);
    const int p = u < 2 * kUnits ? u / kUnits : (u - 2 * kUnits) / kSclUnits;
    const int c = u < 2 * kUnits ? u - p * kUnits : u - 2 * kUnits - p * kSclUnits;
    sv[i] = u < 2 * kUnits ? *(const u32x4*)(tq + p * kT1Kp + c * 16)
                           : *(const u32x4*)(tqs + p * kMxSclRow + c * 16);
    sd[i] = u < 2 * kUnits ? p * kRS + c * 16 : 2 * kRS + p * kMxSclRow + c * 16;
  }
  __builtin_amdgcn_sched_barrier(0);
  int id;
  uint16_t wt;
  one_token_topk(v, E, k, id, wt);
  const int e = __builtin_amdgcn_readlane(id, slot);
  T1Tile t;
  t1_issue(t, blocks, scales, bias, (size_t)e * N + (tile << 4), G);
  __builtin_amdgcn_sched_barrier(0);
  if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0)
    route_one_token(v, E, k, rt.idx, rt.w, rt.indptr, rt.sorted_pairs, rt.token_indices,
                    rt.expert_ids, rt.pair_pos);
#pragma unroll
  for (int i = 0; i < 2; ++i) *(u32x4*)(lds + sd[i]) = sv[i];  // (repeats store the same bytes)
  const uint32_t ss = 2 * kRS + 2 * kMxSclRow + wave * (16 * G);
  t1_stage_scales(t, lds + ss, G);
  lds_barrier();
  f32x4 acc = t1_chain(lds, 0, 2, ss, t, G);
  // the chain combines all 64 lanes: keep it out of the store branch below
  asm volatile("" : "+v"(acc));
  // lane group 0 holds the token (rows 0 and 1: its two pieces)
  const float y0 = (acc[1] + acc[0]) + t.bn;
  const float l0 = lane_xor1(y0);  // odd rows hold the linear half
  // The workgroup's four tiles are act columns 32 bx .. 32 bx + 31 of this
  // slot: one 32-element block, which it encodes into mlp2's three fp8
  // pieces itself, exactly as moe_pieces_kernel<3, true> does (thread q of
  // the first quad takes wave q's eight values; the block maximum by lane
  // exchange).  Piece rows: slot 3 + p, Kp bytes of codes each, 112 scale
  // bytes (run (block & 3), slot block >> 2).
  float* const actb = (float*)(lds + ss - wave * (16 * G) + 4 * (16 * G));  // 32 floats
  if (g == 0 && (r & 1) == 0) {
    const float xg = fminf(y0, limit);
    const float xl = fminf(fmaxf(l0, -limit), limit);
    const float z = __fmul_rn(alpha, xg);
    const float sig = 1.0f / (1.0f + expf(-z));
    actb[wave * 8 + (r >> 1)] = __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
  }
  lds_barrier();
  const int blk = blockIdx.x, c = blk >> 2, gg = blk & 3;
  if (wave == 0 && lane < 4) {
    float rr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) rr[i] = actb[lane * 8 + i];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(rr[i]));
      amax = fmaxf(amax, lane_xor1(amax));
      amax = fmaxf(amax, lane_xor2(amax));
      const uint32_t sc = e8m0_for_amax(amax);
      const float inv = __uint_as_float((254u - sc) << 23);
      const float scf = sc ? __uint_as_float(sc << 23) : __uint_as_float(0x00400000u);
      uint32_t lo, hi;
      e4m3_piece8(rr, inv, scf, lo, hi);
      const int prow = slot * 3 + p;
      *(uint2*)(aq + (size_t)prow * kT1Kp + blk * 32 + lane * 8) = make_uint2(lo, hi);
      if (lane == 0) aqs[prow * kMxSclRow + gg * kMxSclRun + c] = (uint8_t)sc;
    }
  } else if (wave == 1 && blk == (int)gridDim.x - 1) {
    // the last block's workgroup also writes the zero blocks up to 128 x 23
    // (codes 0, the scale of a zero block), as the pieces kernel encodes them
    const int nz = 4 * kT1Nct - (blk + 1);  // zero blocks of each piece row
    const uint32_t sc0 = e8m0_for_amax(0.0f);
    for (int u = lane; u < 3 * nz * 2; u += 64) {
      const int prow = slot * 3 + u / (2 * nz), h = u % (2 * nz);
      *(u32x4*)(aq + (size_t)prow * kT1Kp + (blk + 1) * 32 + h * 16) = u32x4{0u, 0u, 0u, 0u};
    }
    if (lane < 3 * nz) {
      const int prow = slot * 3 + lane / nz, zb = blk + 1 + lane % nz;
      aqs[prow * kMxSclRow + (zb & 3) * kMxSclRun + (zb >> 2)] = (uint8_t)sc0;
    }
  }
}

// mlp2 of one token with the gated combine: workgroup c holds KT waves and
// owns output columns 16 c .. 16 c + 15; wave s multiplies the weight tile of
// the expert of rank s against the KT act rows, encoded into three pieces
// while staged (rows 3 s + p, the P = 3 batch layout with the slots as its
// tokens), and keeps its own slot's rows; the KT results meet in LDS and
// out = bf16(x + bf16(sum_s y_s w_s)) is summed in slot order (w: the
// router's bf16 gate weights).
template <int KT>
__global__ __launch_bounds__(64 * KT) void moe_mx_token1_mlp2_kernel(
    const uint8_t* __restrict__ aq, const uint8_t* __restrict__ aqs,
    const float* __restrict__ logits, int E,
    const uint16_t* __restrict__ x,
    const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, int N, int G, uint16_t* __restrict__ out) {
  static_assert(KT >= 1 && KT <= 5, "one 16-row operand group: 5 tokens of 3 pieces");
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int kRS = mx_row_stride(kT1Nct);
  constexpr int kRows = 3 * KT;
  constexpr int kThreads = 64 * KT;
  // the KT slots' act pieces (rows 3 s + p, written by the one-token mlp1
  // launch): 16-byte units of the code rows, then of the scale rows
  constexpr int kRowUnits = kT1Kp / 16, kSclUnits = kMxSclRow / 16;
  constexpr int kUnits = kRows * (kRowUnits + kSclUnits);
  constexpr int kRounds = (kUnits + kThreads - 1) / kThreads;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t sbase = kRows * kRS + kRows * kMxSclRow;  // weight scale staging
  float* const ys = (float*)(lds + sbase + KT * 16 * G);   // [KT][16]
  uint16_t* const wsl = (uint16_t*)(ys + KT * 16);          // [KT] gate weights
  // the logits, the residual column of the combine (read at the end it would
  // cost a memory round trip of its own) and this thread's units of the act
  // pieces first (they complete first), then the tile's loads, once the
  // token's experts are known; units past the end repeat the last one (the
  // same bytes to the same place)
  const float v = lane < E ? logits[lane] : 0.0f;
  const uint16_t xres = x[(blockIdx.x << 4) + (threadIdx.x & 15)];
  u32x4 pv[kRounds];
  uint32_t pd[kRounds];
#pragma unroll
  for (int i = 0; i < kRounds; ++i) {
    const int u = min(i * kThreads + (int)threadIdx.x, kUnits - 1);
    const bool code = u < kRows * kRowUnits;
    const int m = code ? u / kRowUnits : (u - kRows * kRowUnits) / kSclUnits;
    const int cu = code ? u - m * kRowUnits : u - kRows * kRowUnits - m * kSclUnits;
    const uint8_t* src = code ? aq + (size_t)m * kT1Kp + cu * 16 : aqs + m * kMxSclRow + cu * 16;
    pv[i] = *(const u32x4*)src;  // (one load from a selected address: no branch)
    pd[i] = code ? m * kRS + cu * 16 : kRows * kRS + m * kMxSclRow + cu * 16;
  }
  __builtin_amdgcn_sched_barrier(0);
  int id;
  uint16_t wt;
  one_token_topk(v, E, KT, id, wt);
  const int e = __builtin_amdgcn_readlane(id, wave);
  T1Tile t;
  t1_issue(t, blocks, scales, bias, (size_t)e * N + ((size_t)blockIdx.x << 4), G);
  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0 && lane < KT) wsl[lane] = wt;
#pragma unroll
  for (int i = 0; i < kRounds; ++i) *(u32x4*)(lds + pd[i]) = pv[i];
  const uint32_t ss = sbase + wave * (16 * G);
  t1_stage_scales(t, lds + ss, G);
  lds_barrier();
  f32x4 acc = t1_chain(lds, 0, kRows, ss, t, G);
  asm volatile("" : "+v"(acc));
  // Rows 3 s + p hold piece p of slot s; lane group g holds rows 4 g .. 4 g + 3
  // (the P = 3 epilogue of moe_mx_gemv_kernel: slot 1 straddles groups 0 and
  // 1, slot 2 groups 1 and 2; sums run from the smallest piece up).
  const float send = g == 1 ? acc[1] + acc[0] : acc[0];
  const float recv = __shfl_down(send, 16, kWave);
  float y;
  int gs;
  if (wave == 0) {
    y = ((acc[2] + acc[1]) + acc[0]) + t.bn;
    gs = 0;
  } else if (wave == 1) {
    y = (recv + acc[3]) + t.bn;
    gs = 0;
  } else if (wave == 2) {
    y = ((recv + acc[3]) + acc[2]) + t.bn;
    gs = 1;
  } else if (wave == 3) {
    y = ((acc[3] + acc[2]) + acc[1]) + t.bn;
    gs = 2;
  } else {
    y = ((acc[2] + acc[1]) + acc[0]) + t.bn;
    gs = 3;
  }
  if (g == gs) ys[wave * 16 + r] = y;
  lds_barrier();
  if (threadIdx.x < 16) {
    // multiply and add round separately, as moe_gating_kernel does
#pragma clang fp contract(off)
    const int col = (blockIdx.x << 4) + (int)threadIdx.x;
    float a = 0.0f;
#pragma unroll
    for (int s = 0; s < KT; ++s) a = a + ys[s * 16 + threadIdx.x] * bf2f(wsl[s]);
    out[col] = f2bf(__fadd_rn(bf2f(xres), bf2f(f2bf(a))));
  }
}

template <int P, int kEpi>
int launch_mx(int NC, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const uint8_t* q,
              const uint8_t* qs, int Kp, const int* indptr, const int* sp, int k_top, int arow,
              int orow, const uint8_t* blocks, const uint8_t* scales, const uint16_t* bias, int N,
              int G, int E, int gcap, float alpha, float limit, float* out, int out_ld, int xcds) {
  static const bool lds_ok = [] {  // allow more than 64 KB of dynamic LDS, once per kernel
    const int bytes = kLdsBytes;
    return hipFuncSetAttribute((const void*)moe_mx_gemv_kernel<P, kEpi, 23>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess &&
           hipFuncSetAttribute((const void*)moe_mx_gemv_kernel<P, kEpi, kMxMaxChunks>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
  }();
  if (!lds_ok) return kErrLaunch;
  if (NC == 23)
    hipLaunchKernelGGL((moe_mx_gemv_kernel<P, kEpi, 23>), grid, block, lds, stream, q, qs, Kp,
                       indptr, sp, k_top, arow, orow, blocks, scales, bias, N, G, E, gcap, alpha,
                       limit, out, out_ld, xcds);
  else
    hipLaunchKernelGGL((moe_mx_gemv_kernel<P, kEpi, kMxMaxChunks>), grid, block, lds, stream, q,
                       qs, Kp, indptr, sp, k_top, arow, orow, blocks, scales, bias, N, G, E, gcap,
                       alpha, limit, out, out_ld, xcds);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace moe

extern "C" {

// Packed pieces of `rows` rows of length K: q bytes then (256-aligned) qs bytes.
size_t moe_pieces_q_bytes(int64_t rows, int64_t K, int pieces) {
  const int64_t nc = (K + 127) / 128;
  return (size_t)(((rows * pieces * nc * 128) + 255) / 256 * 256);
}

size_t moe_pieces_total_bytes(int64_t rows, int64_t K, int pieces) {
  return moe_pieces_q_bytes(rows, K, pieces) +
         (size_t)((rows * pieces * moe::kMxSclRow + 255) / 256 * 256);
}

int moe_launch_pieces(const void* x, int x_is_f32, int rows, int K, int pieces, void* packed,
                      hipStream_t stream) {
  if (rows == 0) return moe::kOk;
  const int NC = (K + 127) / 128;
  uint8_t* q = (uint8_t*)packed;
  uint8_t* qs = q + moe_pieces_q_bytes(rows, K, pieces);
  const int64_t threads = (int64_t)rows * 4 * NC * 4;
  const dim3 grid((uint32_t)((threads + 255) / 256));
#define MOE_PIECES(P, F)                                                                       \
  hipLaunchKernelGGL((moe::moe_pieces_kernel<P, F>), grid, dim3(256), 0, stream, x, rows, K, NC, \
                     q, qs)
  if (pieces == 2 && !x_is_f32) MOE_PIECES(2, false);
  else if (pieces == 2) MOE_PIECES(2, true);
  else if (pieces == 3 && x_is_f32) MOE_PIECES(3, true);
  else if (pieces == 4 && !x_is_f32) MOE_PIECES(4, false);
  else if (pieces == 4) MOE_PIECES(4, true);
  else return moe::kErrUnsupported;
#undef MOE_PIECES
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

// packed: pieces of the activation rows (moe_launch_pieces), or with
// swiglu == 2 fp32 activation rows of length K (arow_mode 2, pieces == 4),
// encoded while staged; max_tokens bounds the tokens of one expert (sizes the
// LDS batch); rows_active bounds the pairs (and so the experts that hold any).
// swiglu: 0 plain, 1 interleaved SwiGLU epilogue, 2 plain with fp32 rows.
int moe_launch_mx_gemv(const void* packed, int rows, int pieces, const void* indptr,
                       const void* sorted_pairs, int k_top, int arow_mode, int orow_mode,
                       const void* blocks, const void* scales, const void* bias, int E, int N,
                       int K, int max_tokens, int rows_active, int swiglu, float alpha,
                       float limit, void* out, int out_ld, hipStream_t stream) {
  if (max_tokens <= 0) return moe::kOk;
  const int NC = (K + 127) / 128, Kp = NC * 128, G = K / 32;
  const uint8_t* q = (const uint8_t*)packed;
  const uint8_t* qs = q + moe_pieces_q_bytes(rows, K, pieces);
  // Waves per workgroup and workgroups per CU of the persistent grid;
  // MOE_MX_WAVES / MOE_MX_WG_PER_CU override (tuning runs).
  static const int waves_env = [] {
    const char* v = getenv("MOE_MX_WAVES");
    const int w = v ? atoi(v) : 0;
    return w < 1 ? 0 : w > 12 ? 12 : w;
  }();
  const int tpg = 16 / pieces;
  const int gbytes = moe::mx_group_bytes(NC == 23 ? 23 : moe::kMxMaxChunks);
  // scale staging, unit prefix, indptr, one batch's sorted_pairs, tile counter
  auto fixed_of = [&](int w) {
    return w * 16 * G + 2 * (E + 1) * 4 + (moe::kMxRowMap + 4) * 4;
  };
  const int want = min(moe::kMxMaxGroups, (max_tokens + tpg - 1) / tpg);
  // 11 waves, fewer (down to 8) where each wave's scale staging would leave
  // LDS for fewer token groups than the batch needs (E = 128 at 11 waves:
  // two groups, 16-token batches; at 10: three): a group more per staging
  // serves more tokens per weight read than a wave more in flight.  The
  // generic (24-chunk) kernel is built for at most 8 waves.
  int waves = waves_env;
  if (waves == 0) {
    waves = 11;
    while (waves > 8 && (moe::kLdsBytes - fixed_of(waves)) / gbytes < want) --waves;
  }
  if (NC != 23) waves = min(waves, 8);
  static const int wg_per_cu = [] {
    const char* v = getenv("MOE_MX_WG_PER_CU");
    const int t = v ? atoi(v) : 1;
    return t < 1 ? 1 : t;
  }();
  const int fixed = fixed_of(waves);
  const int gfit = (moe::kLdsBytes - fixed) / gbytes;
  const int gcap = min(want, gfit);
  if (gcap < 1) return moe::kErrUnsupported;
  const size_t lds = (size_t)gcap * gbytes + fixed;
  // Upper bound of the work units (16-row tiles x token batches) over the
  // experts that can hold pairs; the grid never exceeds it.
  const int ntiles = N / 16;
  const int64_t tpb = (int64_t)gcap * tpg;
  const int64_t units_max =
      (int64_t)ntiles * ((int64_t)max(1, min(E, rows_active)) + (int64_t)rows_active / tpb);
  if (units_max >= ((int64_t)1 << 31)) return moe::kErrUnsupported;  // int unit indices
  const int64_t target = (int64_t)moe::kNumCUs * wg_per_cu;
  const int nwg = (int)(units_max < target ? (units_max < 1 ? 1 : units_max) : target);
  const dim3 grid(nwg);
  const dim3 block(64 * waves);
  static const bool xcd_env = [] {
    const char* v = getenv("MOE_MX_XCD");
    return !(v && atoi(v) == 0);
  }();
  const int xcds = (xcd_env && nwg % moe::kNumXcds == 0) ? moe::kNumXcds : 1;
  const int* ip = (const int*)indptr;
  const int* sp = (const int*)sorted_pairs;
  const uint8_t* b = (const uint8_t*)blocks;
  const uint8_t* s = (const uint8_t*)scales;
  const uint16_t* bi = (const uint16_t*)bias;
  float* o = (float*)out;
  if (pieces == 2 && swiglu)
    return moe::launch_mx<2, 1>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  if (pieces == 2)
    return moe::launch_mx<2, 0>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  if (pieces == 3 && !swiglu)
    return moe::launch_mx<3, 0>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  if (pieces == 3 && swiglu == 2)  // fp32 activation rows, encoded while staged
    return moe::launch_mx<3, 2>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  if (pieces == 4 && swiglu == 2)  // fp32 activation rows, encoded while staged
    return moe::launch_mx<4, 2>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  if (pieces == 4 && !swiglu)
    return moe::launch_mx<4, 0>(NC, grid, block, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode,
                                orow_mode, b, s, bi, N, G, E, gcap, alpha, limit, o,
                                out_ld, xcds);
  return moe::kErrUnsupported;
}

// Waves per workgroup of the decode launch (MOE_DECODE_WAVES overrides, 8-12:
// tuning runs).
static int decode_waves() {
  static const int w = [] {
    const char* v = getenv("MOE_DECODE_WAVES");
    const int x = v ? atoi(v) : 11;
    return x < 8 ? 8 : x > 12 ? 12 : x;
  }();
  return w;
}

// The decode launch's first poll goes out before the phase-2 tile loads only
// for batches of at most this many (token, expert) pairs.  There the mlp1
// tiles are few and usually finished when phase 2 starts, and the early poll
// spares the wait behind the tile loads (about 1.5 us of the 40 us launch at
// one token, measured); with more pairs the extra round trip per segment
// costs more than it saves (about 4 us of 110 us at 64 tokens).
constexpr int kDecodePrepollMaxPairs = 16;

static size_t decode_lds_bytes(int E, int H) {
  using namespace moe;
  return (size_t)kMxMaxGroups * mx_group_bytes(23) + decode_waves() * 16 * (H / 32) +
         3 * (E + 1) * 4 + (kMxRowMap + 4) * 4;
}

// Polls of the decode launch's bounded wait (moe_set_decode_spin_limit).
static std::atomic<int> g_decode_spin_max{moe::kDecodeSpinMax};

// Whether the current device can hold the decode launch (256 or more CUs;
// one workgroup of 64 * decode_waves() threads with the whole LDS fits on a
// CU, registers included), found once per device so that launches made
// under graph capture query nothing: kOk, kErrUnsupported or kErrLaunch.
static int decode_device_fit() {
  using namespace moe;
  constexpr int kMaxDevices = 64;
  static std::atomic<int> fit[kMaxDevices];  // 0: not known yet, else status + 1
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return kErrLaunch;
  if (dev < 0 || dev >= kMaxDevices) return kErrUnsupported;
  const int known = fit[dev].load(std::memory_order_acquire);
  if (known) return known - 1;
  int rc = kOk, cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    rc = kErrLaunch;
  else if (cus < kNumCUs)
    rc = kErrUnsupported;  // every workgroup must be resident
  else if (hipFuncSetAttribute((const void*)moe_mx_decode_kernel,
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               kLdsBytes) != hipSuccess ||
           hipOccupancyMaxActiveBlocksPerMultiprocessor(
               &per_cu, (const void*)moe_mx_decode_kernel, 64 * decode_waves(), kLdsBytes) !=
               hipSuccess)
    rc = kErrLaunch;
  else if (per_cu < 1)
    rc = kErrUnsupported;
  fit[dev].store(rc + 1, std::memory_order_release);
  return rc;
}

// kOk when moe_launch_mx_decode can run this shape on the current device,
// else kErrUnsupported (the caller then runs mlp1, the encoding and mlp2 as
// separate launches).
int moe_mx_decode_check(int E, int H, int I, int nk) {
  using namespace moe;
  if (H != I || (H + 127) / 128 != 23 || H % 32) return kErrUnsupported;
  if (decode_lds_bytes(E, H) > (size_t)kLdsBytes) return kErrUnsupported;
  const int fit = decode_device_fit();
  if (fit != kOk) return fit;
  const int grid = kNumCUs;
  constexpr int gcap2 = kMxMaxGroups;
  // Batches are bounded by (experts holding pairs) + nk / tokens per batch.
  // Phase 1 needs one segment per workgroup whose share (at most
  // 4 ceil(quads / floor(grid / batches)) tiles) fits the LDS act tile of 96.
  const int64_t nb1 = (int64_t)min(E, nk) + nk / (kDecodeGroups1 * 8);
  const int64_t nb2 = (int64_t)min(E, nk) + nk / (gcap2 * 5);
  if (nb1 > grid || nb2 > grid) return kErrUnsupported;
  const int quads = (2 * H / 16) / 4;
  const int wmin = grid / (int)nb1;
  if (4 * ((quads + wmin - 1) / wmin) > 96) return kErrUnsupported;
  return kOk;
}

// The decode chain in one launch (moe_mx_decode_kernel): t pieces (2, rows
// n) -> act pieces (3, rows nk, written) -> y (fp32 [nk][H], rows by pair).
// done: E ints and status: one int, all zero at launch; status counts the
// workgroups whose bounded wait gave up (their y rows are wrong).
// With out (and w, x, arrive: n * H / 16 ints, zero at launch) the launch also
// writes out = bf16(x + bf16(sum_r y[t, r] w[t, r])) (the gated combine).
// With logits (n x E, E <= 32, n E <= 4096 and a multiple of 4, 16-byte
// aligned, nk <= 512; not with out) the
// launch routes itself and writes idx, the gate weights route_w, indptr,
// sorted_pairs and the other grouping arrays (route: token_indices,
// expert_ids, pair_pos).
int moe_launch_mx_decode(const void* t_packed, int n, const void* indptr,
                         const void* sorted_pairs, int k_top, const void* blocks1,
                         const void* scales1, const void* bias1, const void* blocks2,
                         const void* scales2, const void* bias2, int E, int H, int I, int nk,
                         float alpha, float limit, void* act_packed, void* y, void* done,
                         void* status, const void* w, const void* x, void* out, void* arrive,
                         const void* logits, void* idx, void* route_w, void* const* route,
                         hipStream_t stream) {
  using namespace moe;
  if (nk <= 0) return kOk;
  if (!done || !status) return kErrUnsupported;
  if (out && (!w || !x || !arrive || (H & 15))) return kErrUnsupported;
  DecodeRoute rt{};
  if (logits) {
    if (out || !idx || !route_w || !route || E > 32 || (int64_t)n * E > kDecodeRouteKeys ||
        (n * E) % 4 || nk > 512 || nk != n * k_top || ((uintptr_t)logits & 15u))
      return kErrUnsupported;
    rt = DecodeRoute{(const float*)logits, n, (int32_t*)idx, (uint16_t*)route_w,
                     (int32_t*)indptr, (int32_t*)sorted_pairs, (int32_t*)route[0],
                     (int32_t*)route[1], (int32_t*)route[2]};
  }
  const int rc = moe_mx_decode_check(E, H, I, nk);
  if (rc != kOk) return rc;
  const int grid = kNumCUs;
  const int waves = decode_waves();
  constexpr int gcap2 = kMxMaxGroups;
  const size_t lds = decode_lds_bytes(E, H);
  const uint8_t* tq = (const uint8_t*)t_packed;
  uint8_t* aq = (uint8_t*)act_packed;
  hipLaunchKernelGGL(moe_mx_decode_kernel, dim3(grid), dim3(64 * waves), lds, stream, tq,
                     tq + moe_pieces_q_bytes(n, H, 2), (const int*)indptr,
                     (const int*)sorted_pairs, k_top, (const uint8_t*)blocks1,
                     (const uint8_t*)scales1, (const uint16_t*)bias1, (const uint8_t*)blocks2,
                     (const uint8_t*)scales2, (const uint16_t*)bias2, H, E, gcap2, alpha, limit,
                     aq, aq + moe_pieces_q_bytes(nk, I, 3), (float*)y, (int*)done,
                     (int*)status, g_decode_spin_max.load(std::memory_order_relaxed),
                     nk <= kDecodePrepollMaxPairs ? 1 : 0, grid % kNumXcds == 0 ? kNumXcds : 1,
                     (const uint16_t*)w, (const uint16_t*)x, (uint16_t*)out, (int*)arrive, rt);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Bound of the decode launch's wait, in polls (about 1 us each); a negative
// value restores the default.  Returns the previous bound.
int moe_decode_spin_limit_exchange(int polls) {
  return g_decode_spin_max.exchange(polls < 0 ? moe::kDecodeSpinMax : polls);
}

// kOk when the one-token launches (moe_mx_token1_*_kernel) take this shape:
// E <= 32 experts, k = 4 slots, H and I of 23 chunks of 128 (H, I multiples
// of 32).
int moe_mx_token1_check(int E, int k, int H, int I) {
  using namespace moe;
  if (k != 4 || E < k || E > 32) return kErrUnsupported;
  if (H % 32 || I % 32 || (H + 127) / 128 != kT1Nct || (I + 127) / 128 != kT1Nct)
    return kErrUnsupported;
  return kOk;
}

// One token's mlp1 with SwiGLU: t pieces (2, one row) and its E logits ->
// act rows by slot ([k][I], fp32); route: idx, w, indptr, sorted_pairs,
// token_indices, expert_ids, pair_pos, written by the first workgroup.
int moe_launch_mx_token1_mlp1(const void* t_packed, const void* logits, int E,
                              void* const* route, const void* blocks, const void* scales,
                              const void* bias, int k, int H, int I, float alpha, float limit,
                              void* act_packed, hipStream_t stream) {
  using namespace moe;
  if (moe_mx_token1_check(E, k, H, I) != kOk) return kErrUnsupported;
  const Token1Route rt{(int32_t*)route[0], (uint16_t*)route[1], (int32_t*)route[2],
                       (int32_t*)route[3], (int32_t*)route[4], (int32_t*)route[5],
                       (int32_t*)route[6]};
  const uint8_t* tq = (const uint8_t*)t_packed;
  const int G = H / 32;
  // LDS: t's two piece rows and their scales, the waves' scale staging, the
  // workgroup's 32 act values
  const size_t lds = 2 * mx_row_stride(kT1Nct) + 2 * kMxSclRow + 4 * 16 * G + 32 * 4;
  uint8_t* aq = (uint8_t*)act_packed;
  hipLaunchKernelGGL(moe_mx_token1_mlp1_kernel, dim3(2 * I / 64, k), dim3(256), lds, stream, tq,
                     tq + moe_pieces_q_bytes(1, H, 2), (const float*)logits, E, rt,
                     (const uint8_t*)blocks,
                     (const uint8_t*)scales, (const uint16_t*)bias, 2 * I, G, alpha, limit, aq,
                     aq + moe_pieces_q_bytes(k, I, 3));
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// One token's mlp2 with the gated combine and the residual: act rows by slot
// ([k][I], fp32), the token's E logits and x -> out = bf16(x + bf16(sum_s
// y_s w_s)) ([H], bf16).
int moe_launch_mx_token1_mlp2(const void* act_packed, const void* logits, int E, const void* x,
                              const void* blocks, const void* scales, const void* bias, int k,
                              int H, int I, void* out, hipStream_t stream) {
  using namespace moe;
  if (moe_mx_token1_check(E, k, H, I) != kOk) return kErrUnsupported;
  constexpr int KT = 4;
  const int G = I / 32;
  const size_t lds =
      3 * KT * (mx_row_stride(kT1Nct) + kMxSclRow) + KT * 16 * G + KT * 16 * 4 + KT * 2;
  const uint8_t* aq = (const uint8_t*)act_packed;
  hipLaunchKernelGGL(moe_mx_token1_mlp2_kernel<KT>, dim3(H / 16), dim3(64 * KT), lds, stream, aq,
                     aq + moe_pieces_q_bytes(k, I, 3), (const float*)logits, E,
                     (const uint16_t*)x, (const uint8_t*)blocks, (const uint8_t*)scales,
                     (const uint16_t*)bias, H, G, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
