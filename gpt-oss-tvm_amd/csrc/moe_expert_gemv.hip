// Grouped expert matmul for small per-expert token counts (decode).
//
// Computes, for every expert e and every (token, slot) pair routed to it,
//   out[pair][c] = bias[e][c] + sum_i x[row(pair)][i] * W_e[c][i]
// where W_e is MXFP4 in the checkpoint layout blocks [E, N, K/32, 16] +
// scales [E, N, K/32] (model/mlp.py:100-144).  This is the arithmetic of the
// reference's moe_einsum_fused (model/mlp.py:267-326) and of the decode
// kernels mxfp4_moe_mlp{1,2}_decode (model/mlp_optimized.py:462-660).
//
// Mapping (activation-stationary): a workgroup per (expert, kRowsWG weight
// rows, 16-token tile), one wave per K-slice of kS = 10 MX blocks (320 K),
// ceil(G / kS) waves.
//   * each wave loads its 16 tokens x 320 K activation fragment into
//     registers once (lane (n, q) holds elements 8q..8q+7 of each block of
//     token n) and keeps it for all the workgroup's rows;
//   * weights stream in 32-row tiles: 32 rows x 10 blocks x 16 B per wave,
//     five 16-byte loads per lane over contiguous 160-byte row segments, two
//     tiles ahead (plain loads: a non-temporal hint measured 25-35% slower); each wave moves its blocks through a
//     private LDS tile (row stride 176 B, conflict-free reads) into the MFMA
//     operand layout, lane (m, q) taking dword q of each block of row m;
//   * v_mfma_f32_16x16x32_bf16 with A = 16 weight rows and B = 16 tokens;
//     one MX block is one MFMA's K, so its E8M0 scale applies to the whole
//     operand through the scaled fp4 -> bf16 conversion;
//   * the slices' partial sums go to LDS and are added in slice order by the
//     first two waves (one wave when K <= 320), which apply bias and epilogue
//     (deterministic).
// One barrier per 32-row tile.
//
// Activations arrive as bf16 (mlp1: the normalised tokens) or as a pair of
// bf16 planes hi + lo whose sum is the fp32 activation (mlp2: the SwiGLU
// output); the pair is multiplied twice, which keeps each product within
// 2^-17 of the fp32 one (a single bf16 rounding of the activation does not
// meet the block-output tolerance).
#include "moe_common.h"

namespace moe {

constexpr int kMaxG = 96;      // K <= 3072
constexpr int kS = 10;         // MX blocks per K-slice (one wave)
constexpr int kMaxSlices = 10; // ceil(kMaxG / kS)
constexpr int kTileRows = 32;  // weight rows per tile
constexpr int kAst = 44;       // LDS row stride of a wave's weight tile, dwords (40 used)
constexpr int kMaxRowsWG = 192;  // weight rows per workgroup: 192 (6 tiles) or 96 (3 tiles)

enum BRow : int { kBRowToken = 0, kBRowPair = 1, kBRowSorted = 2 };
enum ORow : int { kORowPair = 0, kORowSorted = 1 };
enum Epi : int { kEpiRaw = 0, kEpiSwigluSplit = 1 };

// Clamped SwiGLU of one (glu, linear) pair, model/mlp.py:29-60.
__device__ __forceinline__ float swiglu1(float glu, float lin, float alpha, float limit) {
  const float xg = fminf(glu, limit);
  const float xl = fminf(fmaxf(lin, -limit), limit);
  const float z = __fmul_rn(alpha, xg);
  const float sig = 1.0f / (1.0f + expf(-z));
  return __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
}

// bf16 hi/lo split of one fp32 value (hi = RNE(a), lo = RNE(a - hi)).
__device__ __forceinline__ void split1(float a, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(a);
  lo = f2bf(__fsub_rn(a, bf2f(hi)));
}

template <bool kSplit, int kEpi>
__global__ __launch_bounds__(64 * kMaxSlices) void moe_expert_gemv_kernel(
    const uint16_t* __restrict__ xh, const uint16_t* __restrict__ xl, int x_ld,
    const int32_t* __restrict__ indptr, const int32_t* __restrict__ sorted_pairs, int k_top,
    int brow_mode, int orow_mode, const uint8_t* __restrict__ blocks,
    const uint8_t* __restrict__ scales, const uint16_t* __restrict__ bias, int N, int K,
    float alpha, float limit, void* __restrict__ out, void* __restrict__ out_lo, int out_ld,
    int rows_wg) {
  constexpr int kPlanes = kSplit ? 2 : 1;
  __shared__ __align__(16) uint32_t w_lds[kMaxSlices * kTileRows * kAst];
  __shared__ __align__(16) f32x4 part[2][kMaxSlices][2][64];
  __shared__ __align__(16) uint8_t sc_lds[kMaxRowsWG * kMaxG];
  __shared__ float bias_lds[kMaxRowsWG];

  const int e = blockIdx.y;
  const int beg = indptr[e];
  const int cnt = indptr[e + 1] - beg;
  if (cnt <= 0) return;
  const int tb = blockIdx.z * 16;           // token tile
  if (tb >= cnt) return;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nw = blockDim.x >> 6;           // K-slices
  const int m = lane & 15, q = lane >> 4;
  const int G = K >> 5;
  const int g0 = wave * kS;                 // first block of this wave's slice
  const int nb = min(kS, G - g0);           // blocks in this slice (>= 1)
  const int rwg = blockIdx.x * rows_wg;     // workgroup's first row
  const int nrows = min(rows_wg, N - rwg);  // rows of the workgroup inside N (multiple of 32)
  const size_t wrow0 = (size_t)e * N + rwg;
  uint32_t* wt = w_lds + wave * kTileRows * kAst;

  // scales of the workgroup's rows -> LDS (contiguous; 32-row multiples keep
  // the region and its offset 16-byte aligned)
  {
    const u32x4* src = (const u32x4*)(scales + wrow0 * G);
    u32x4* dst = (u32x4*)sc_lds;
    for (int i = tid; i < nrows * G / 16; i += blockDim.x) dst[i] = src[i];
    // bias too: a global load inside the tile loop would drain the weight
    // prefetch (the load counter completes in issue order)
    for (int i = tid; i < nrows; i += blockDim.x) bias_lds[i] = bf2f(bias[wrow0 + i]);
  }

  // activation fragment of the slice: lane (n, q), block u -> 8 elements of token n
  const bool tv = tb + m < cnt;
  const int j = beg + (tv ? tb + m : tb);
  const int p = sorted_pairs[j];
  const int brow = brow_mode == kBRowToken ? p / k_top : (brow_mode == kBRowPair ? p : j);
  u32x4 bf[kPlanes][kS];
  {
    const uint16_t* bh = xh + (size_t)brow * x_ld + 8 * q;
#pragma unroll
    for (int u = 0; u < kS; ++u) {
      const int g = min(g0 + u, G - 1);
      bf[0][u] = *(const u32x4*)(bh + g * 32);
      if constexpr (kSplit) bf[1][u] = *(const u32x4*)(bh + (xl - xh) + g * 32);
    }
  }

  // Weight loader: chunk i = lane + 64 c (c < 5) of the tile is row i / 10,
  // block i % 10 of the slice.  Blocks past the slice end (last slice when
  // G % 10 != 0) read the slice's first block and are never used.
  const uint8_t* wbase = blocks + wrow0 * G * 16;
  int woff[5];
#pragma unroll
  for (int c = 0; c < 5; ++c) {
    const int i = lane + 64 * c;
    const int r = i / kS, b = i - (i / kS) * kS;
    woff[c] = (r * G + g0 + (b < nb ? b : 0)) * 16;
  }
  const int kTiles = rows_wg / kTileRows;   // 3 or 6
  const int kValid = nrows / kTileRows;     // tiles inside N
  auto load = [&](int k, u32x4 (&f)[5]) {
    const int kk = k < kValid ? k : 0;      // past the last valid tile: cache-hot dummy
    const uint8_t* base = wbase + (size_t)kk * kTileRows * G * 16;
#pragma unroll
    for (int c = 0; c < 5; ++c) f[c] = *(const u32x4*)(base + woff[c]);
  };
  auto stage = [&](const u32x4 (&f)[5]) {
#pragma unroll
    for (int c = 0; c < 5; ++c) {
      const int i = lane + 64 * c;
      const int r = i / kS, b = i - (i / kS) * kS;
      *(u32x4*)&wt[r * kAst + 4 * b] = f[c];
    }
  };

  __syncthreads();  // scales staged

  // Tile k: wait for its loads (two tiles stay in flight), stage, multiply,
  // write the slice's partial sums, barrier, and the first two waves reduce.
  // The partial buffer written at tile k was last read at tile k-2, before
  // those waves passed the barrier of tile k-1.  The loop is unrolled by
  // three over three register groups and has no branches around loads.
  u32x4 f0[5], f1[5], f2[5];
  load(0, f0);
  load(1, f1);
  auto tile = [&](int k, const u32x4 (&f)[5]) {
    stage(f);
    // LDS instructions of one wave execute in order: the reads below see the
    // writes above without a barrier.
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const bool kv = k < kValid;             // tiles past N compute on a dummy and store nothing
    const int rbase = (kv ? k : 0) * kTileRows;
#pragma unroll
    for (int u = 0; u < kS; ++u) {
      if (u < nb) {                         // wave-uniform
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const uint32_t adw = wt[(16 * rt + m) * kAst + 4 * u + q];
          const uint32_t sbyte = sc_lds[(rbase + 16 * rt + m) * G + g0 + u];
          const bf16x8 a = dequant8(adw, __uint_as_float(sbyte << 23));
          acc[rt] = mfma16x16x32(a, as_bf16x8(bf[0][u]), acc[rt]);
          if constexpr (kSplit) acc[rt] = mfma16x16x32(a, as_bf16x8(bf[1][u]), acc[rt]);
        }
      }
    }
    part[k & 1][wave][0][lane] = acc[0];
    part[k & 1][wave][1][lane] = acc[1];
    __syncthreads();
    // lane (token column m, group q) of row tile rt: rows 4q..4q+3
    for (int rt = wave; rt < 2; rt += nw) {
      const int row = rwg + rbase + 16 * rt + 4 * q;
      f32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bias_lds[rbase + 16 * rt + 4 * q + i];
      for (int w = 0; w < nw; ++w) {
        const f32x4 pv = part[k & 1][w][rt][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(v[i], pv[i]);
      }
      if (tv && kv) {
        const int orow = orow_mode == kORowPair ? p : j;
        if constexpr (kEpi == kEpiRaw) {
          *(f32x4*)((float*)out + (size_t)orow * out_ld + row) = v;
        } else {
          uint16_t h0, l0, h1, l1;
          split1(swiglu1(v[0], v[1], alpha, limit), h0, l0);
          split1(swiglu1(v[2], v[3], alpha, limit), h1, l1);
          const size_t o = (size_t)orow * out_ld + row / 2;
          *(uint32_t*)((uint16_t*)out + o) = (uint32_t)h0 | ((uint32_t)h1 << 16);
          *(uint32_t*)((uint16_t*)out_lo + o) = (uint32_t)l0 | ((uint32_t)l1 << 16);
        }
      }
    }
  };
  for (int k = 0; k < kTiles; k += 3) {
    load(k + 2, f2);
    __builtin_amdgcn_sched_barrier(0);
    tile(k, f0);
    __builtin_amdgcn_sched_barrier(0);
    load(k + 3, f0);
    __builtin_amdgcn_sched_barrier(0);
    tile(k + 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    load(k + 4, f1);
    __builtin_amdgcn_sched_barrier(0);
    tile(k + 2, f2);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// fp32 [rows, K] -> bf16 hi/lo planes (the split the kernel above expects).
__global__ __launch_bounds__(256) void moe_split_kernel(const f32x4* __restrict__ x, int64_t n4,
                                                        uint2* __restrict__ hi,
                                                        uint2* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const f32x4 v = x[i];
  uint16_t h[4], l[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) split1(v[k], h[k], l[k]);
  hi[i] = uint2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
  lo[i] = uint2{(uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16)};
}

template <bool kSplit, int kEpi>
static void launch(dim3 grid, int threads, hipStream_t stream, const void* xh, const void* xl,
                   int x_ld, const void* indptr, const void* sp, int k_top, int brow_mode,
                   int orow_mode, const void* blocks, const void* scales, const void* bias, int N,
                   int K, float alpha, float limit, void* out, void* out_lo, int out_ld,
                   int rows_wg) {
  hipLaunchKernelGGL((moe_expert_gemv_kernel<kSplit, kEpi>), grid, dim3(threads), 0, stream,
                     (const uint16_t*)xh, (const uint16_t*)xl, x_ld, (const int32_t*)indptr,
                     (const int32_t*)sp, k_top, brow_mode, orow_mode, (const uint8_t*)blocks,
                     (const uint8_t*)scales, (const uint16_t*)bias, N, K, alpha, limit, out, out_lo,
                     out_ld, rows_wg);
}

}  // namespace moe

// Grid (ceil(N / rows_wg), E, token tiles): one workgroup per rows_wg weight
// rows of an expert (192 when N divides, else 96; N % 32 == 0) and 16-token
// tile, ceil(K / 320) waves.  max_tokens bounds the per-expert pair count
// (n covers every case: a token routes to an expert at most once); token
// tiles past an expert's count exit at once.
// x: bf16 [rows, K] (x_lo == NULL) or bf16 hi/lo planes (x_lo != NULL).
// swiglu == 0: fp32 out [rows, out_ld]; swiglu == 1: bf16 hi/lo planes
// [rows, out_ld] with out_ld = N / 2.
extern "C" int moe_launch_expert_gemv(const void* x, const void* x_lo, int x_ld,
                                      const void* indptr, const void* sorted_pairs, int k_top,
                                      int brow_mode, int orow_mode, const void* blocks,
                                      const void* scales, const void* bias, int E, int N, int K,
                                      int max_tokens, int swiglu, float alpha, float limit,
                                      void* out, void* out_lo, int out_ld, hipStream_t stream) {
  if (N % 32 || K % 32 || K / 32 > moe::kMaxG) return moe::kErrUnsupported;
  if (max_tokens <= 0) return moe::kOk;
  const int rows_wg = N % 192 == 0 ? 192 : 96;
  const int G = K / 32;
  const int nw = (G + moe::kS - 1) / moe::kS;
  const dim3 grid((N + rows_wg - 1) / rows_wg, E, (max_tokens + 15) / 16);
#define MOE_GEMV_ARGS                                                                          \
  grid, 64 * nw, stream, x, x_lo, x_ld, indptr, sorted_pairs, k_top, brow_mode, orow_mode, \
      blocks, scales, bias, N, K, alpha, limit, out, out_lo, out_ld, rows_wg
  if (!x_lo && !swiglu) moe::launch<false, moe::kEpiRaw>(MOE_GEMV_ARGS);
  else if (!x_lo) moe::launch<false, moe::kEpiSwigluSplit>(MOE_GEMV_ARGS);
  else if (!swiglu) moe::launch<true, moe::kEpiRaw>(MOE_GEMV_ARGS);
  else moe::launch<true, moe::kEpiSwigluSplit>(MOE_GEMV_ARGS);
#undef MOE_GEMV_ARGS
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

extern "C" int moe_launch_split(const void* x, int64_t count, void* hi, void* lo,
                                hipStream_t stream) {
  if (count == 0) return moe::kOk;
  const int64_t n4 = count / 4;
  hipLaunchKernelGGL(moe::moe_split_kernel, dim3((uint32_t)((n4 + 255) / 256)), dim3(256), 0,
                     stream, (const moe::f32x4*)x, n4, (uint2*)hi, (uint2*)lo);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
