// Grouped expert matmul for small per-expert token counts (decode).
//
// Computes, for every expert e and every (token, slot) pair routed to it,
//   out[pair][c] = bias[e][c] + sum_i x[row(pair)][i] * W_e[c][i]
// where W_e is MXFP4 in the checkpoint layout blocks [E, N, K/32, 16] +
// scales [E, N, K/32] (model/mlp.py:100-144).  This is the arithmetic of the
// reference's moe_einsum_fused (model/mlp.py:267-326) and of the decode
// kernels mxfp4_moe_mlp{1,2}_decode (model/mlp_optimized.py:462-660).
//
// Mapping: one wave per (expert, 64 weight rows).  The wave streams its rows
// once, K-major, with one 16-byte load per lane per 16-row tile per step, and
// reuses each dequantised fragment for up to 32 tokens with
// v_mfma_f32_16x16x32_bf16 (A = 16 weight rows, B = 16 tokens).
//
// K order inside a step: lane (row m, group q) owns MX block g = 4*step + q
// of its row and feeds its 32 values to four MFMAs, 8 per MFMA; the token
// operand uses the same (q, sub-step, i) -> k map, so every product pairs the
// right weight with the right activation while each lane's weight load is a
// whole 16-byte block.  Steps past the last block load nothing (zeros).
//
// Inputs are bf16 (mlp1: the normalised tokens) or fp32 (mlp2: the SwiGLU
// output).  fp32 activations are split into bf16 hi + lo and multiplied
// twice, which keeps the products within 2^-17 of fp32 (a single bf16 rounding
// of the activations does not meet the block-output tolerance).
#include "moe_common.h"

namespace moe {

constexpr int kMaxG = 96;  // K <= 3072

enum BRow : int { kBRowToken = 0, kBRowPair = 1, kBRowSorted = 2 };
enum ORow : int { kORowPair = 0, kORowSorted = 1 };
enum Epi : int { kEpiRaw = 0, kEpiSwiglu = 1 };

// Clamped SwiGLU of one (glu, linear) pair, model/mlp.py:29-60.
__device__ __forceinline__ float swiglu1(float glu, float lin, float alpha, float limit) {
  const float xg = fminf(glu, limit);
  const float xl = fminf(fmaxf(lin, -limit), limit);
  const float z = __fmul_rn(alpha, xg);
  const float sig = 1.0f / (1.0f + expf(-z));
  return __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
}

template <bool kF32In, int kEpi>
__global__ __launch_bounds__(64) void moe_expert_gemv_kernel(
    const void* __restrict__ xin, const int32_t* __restrict__ indptr,
    const int32_t* __restrict__ sorted_pairs, int k_top, int brow_mode, int orow_mode,
    const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
    const uint16_t* __restrict__ bias, int N, int K, float alpha, float limit,
    float* __restrict__ out, int out_ld) {
  constexpr int R = 4;  // 16-row tiles per wave
  __shared__ __align__(16) uint8_t sc_lds[64 * kMaxG];

  const int e = blockIdx.y;
  const int r0 = blockIdx.x * 64;
  const int beg = indptr[e];
  const int cnt = indptr[e + 1] - beg;
  if (cnt <= 0) return;

  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  const int G = K >> 5;
  const size_t wrow0 = (size_t)e * N + r0;

  {
    const u32x4* src = (const u32x4*)(scales + wrow0 * G);
    u32x4* dst = (u32x4*)sc_lds;
    for (int i = lane; i < 4 * G; i += kWave) dst[i] = src[i];
  }
  __syncthreads();

  f32x4 bias4[R];
#pragma unroll
  for (int rt = 0; rt < R; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) bias4[rt][i] = bf2f(bias[wrow0 + 16 * rt + 4 * q + i]);

  const int nsteps = (G + 3) >> 2;

  for (int tb = 0; tb < cnt; tb += 32) {
    int brow[2];
    bool tv[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int jt = tb + 16 * tt + m;
      tv[tt] = jt < cnt;
      brow[tt] = 0;
      if (tv[tt]) {
        const int j = beg + jt;
        const int p = sorted_pairs[j];
        brow[tt] = brow_mode == kBRowToken ? p / k_top : (brow_mode == kBRowPair ? p : j);
      }
    }
    const bool two = (tb + 16) < cnt;

    f32x4 acc[R][2];
#pragma unroll
    for (int rt = 0; rt < R; ++rt) {
      acc[rt][0] = bias4[rt];
      acc[rt][1] = bias4[rt];
    }

    for (int s = 0; s < nsteps; ++s) {
      const int g = 4 * s + q;
      const bool gv = g < G;
      u32x4 w[R];
      float scf[R];
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        w[rt] = gv ? *(const u32x4*)(blocks + ((wrow0 + 16 * rt + m) * G + g) * 16)
                   : u32x4{0u, 0u, 0u, 0u};
        scf[rt] = e8m0_to_f32(sc_lds[(16 * rt + m) * G + (gv ? g : 0)]);
      }
      if constexpr (!kF32In) {
        u32x4 b[2][4];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const bool ld = tv[tt] && gv && (tt == 0 || two);
          const u32x4* src = (const u32x4*)((const uint16_t*)xin + (size_t)brow[tt] * K + g * 32);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) b[tt][jj] = ld ? src[jj] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
          for (int rt = 0; rt < R; ++rt) {
            const bf16x8 a = dequant8(w[rt][jj], scf[rt]);
            acc[rt][0] = mfma16x16x32(a, as_bf16x8(b[0][jj]), acc[rt][0]);
            if (two) acc[rt][1] = mfma16x16x32(a, as_bf16x8(b[1][jj]), acc[rt][1]);
          }
        }
      } else {
        u32x4 b[2][8];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const bool ld = tv[tt] && gv && (tt == 0 || two);
          const u32x4* src = (const u32x4*)((const float*)xin + (size_t)brow[tt] * K + g * 32);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) b[tt][jj] = ld ? src[jj] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          bf16x8 hi[2], lo[2];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              f[i] = __uint_as_float(b[tt][2 * jj][i]);
              f[4 + i] = __uint_as_float(b[tt][2 * jj + 1][i]);
            }
            split8(f, hi[tt], lo[tt]);
          }
#pragma unroll
          for (int rt = 0; rt < R; ++rt) {
            const bf16x8 a = dequant8(w[rt][jj], scf[rt]);
            acc[rt][0] = mfma16x16x32(a, hi[0], acc[rt][0]);
            acc[rt][0] = mfma16x16x32(a, lo[0], acc[rt][0]);
            if (two) {
              acc[rt][1] = mfma16x16x32(a, hi[1], acc[rt][1]);
              acc[rt][1] = mfma16x16x32(a, lo[1], acc[rt][1]);
            }
          }
        }
      }
    }

    // Lane (token column m, group q) holds rows 4q..4q+3 of each 16-row tile.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      if (!tv[tt]) continue;
      const int j = beg + tb + 16 * tt + m;
      const int orow = orow_mode == kORowPair ? sorted_pairs[j] : j;
      float* o = out + (size_t)orow * out_ld;
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        const int row = r0 + 16 * rt + 4 * q;
        const f32x4 v = acc[rt][tt];
        if constexpr (kEpi == kEpiRaw) {
          *(f32x4*)(o + row) = v;
        } else {
          float2 r2;
          r2.x = swiglu1(v[0], v[1], alpha, limit);
          r2.y = swiglu1(v[2], v[3], alpha, limit);
          *(float2*)(o + row / 2) = r2;
        }
      }
    }
  }
}

}  // namespace moe

// x: bf16 [rows, K] (x_f32 = 0) or fp32 [rows, K] (x_f32 = 1); rows are
// selected per pair by brow_mode.  Grid: (N / 64, E) waves.
extern "C" int moe_launch_expert_gemv(const void* x, int x_f32, const void* indptr,
                                      const void* sorted_pairs, int k_top, int brow_mode,
                                      int orow_mode, const void* blocks, const void* scales,
                                      const void* bias, int E, int N, int K, int swiglu,
                                      float alpha, float limit, void* out, int out_ld,
                                      hipStream_t stream) {
  const dim3 grid(N / 64, E), block(64);
  const int32_t* ip = (const int32_t*)indptr;
  const int32_t* sp = (const int32_t*)sorted_pairs;
  const uint8_t* bl = (const uint8_t*)blocks;
  const uint8_t* sc = (const uint8_t*)scales;
  const uint16_t* bi = (const uint16_t*)bias;
  float* o = (float*)out;
  if (!x_f32 && !swiglu)
    hipLaunchKernelGGL((moe::moe_expert_gemv_kernel<false, moe::kEpiRaw>), grid, block, 0, stream,
                       x, ip, sp, k_top, brow_mode, orow_mode, bl, sc, bi, N, K, alpha, limit, o,
                       out_ld);
  else if (!x_f32 && swiglu)
    hipLaunchKernelGGL((moe::moe_expert_gemv_kernel<false, moe::kEpiSwiglu>), grid, block, 0,
                       stream, x, ip, sp, k_top, brow_mode, orow_mode, bl, sc, bi, N, K, alpha,
                       limit, o, out_ld);
  else if (x_f32 && !swiglu)
    hipLaunchKernelGGL((moe::moe_expert_gemv_kernel<true, moe::kEpiRaw>), grid, block, 0, stream,
                       x, ip, sp, k_top, brow_mode, orow_mode, bl, sc, bi, N, K, alpha, limit, o,
                       out_ld);
  else
    hipLaunchKernelGGL((moe::moe_expert_gemv_kernel<true, moe::kEpiSwiglu>), grid, block, 0,
                       stream, x, ip, sp, k_top, brow_mode, orow_mode, bl, sc, bi, N, K, alpha,
                       limit, o, out_ld);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
