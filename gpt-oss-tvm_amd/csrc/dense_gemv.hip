// Decode-sized dense projections of the gpt-oss layer (M <= 8 tokens): the
// fused QKV nn.Linear with its bias, YaRN RoPE and the KV-cache append; the
// attention output nn.Linear with its bias and the residual add; the
// unembedding (model/attention.py:204,254-256; model/transformer.py:95-100).
// The QKV projection and the unembedding can also apply the RMSNorm before
// them (attention.py:80, transformer.py:63) to the rows they stage.
//
// y[m][n] = sum_k x[m][k] W[n][k], bf16 operands, fp32 accumulation, one bf16
// rounding (the matmul's output dtype), then the epilogue's own bf16 ops.
// HBM-bound on W.  A workgroup takes RW rows of W; its 4 waves split K (wave
// w takes the 16-byte chunks w * 64 + lane + 256 i of each row), so a row's
// bytes stream from four waves at once; the four partial sums are added in
// wave order through LDS (deterministic).  The tokens x are staged in LDS.
// Loads complete in issue order, so everything small that the workgroup
// needs (its x chunks, the epilogue's bias, residual, positions, slots and
// RoPE frequencies) is loaded before the W rows, and the epilogue's cos and
// sin are taken while W streams: the RMSNorm and the epilogue then wait for
// nothing behind the W loads.
#include "moe_common.h"

namespace gemv {

using moe::bf2f;
using moe::f2bf;
using moe::u32x4;

constexpr int kThreads = 256;  // 4 waves
constexpr int kWaves = 4;
constexpr int kMaxM = 8;
constexpr int kIters = 2;  // 16-byte chunk rounds per lane: K <= 4096 = 2 x 256 x 8

// gpt-oss attention shapes (the QKV epilogue)
constexpr int kD = 64, kHq = 64, kHkv = 8, kPage = 16;
constexpr int kHeadBlock = kPage * kD * 2;
constexpr int kPageBytes = 2 * kHkv * kHeadBlock;

__device__ __forceinline__ float dot8(u32x4 w, u32x4 x, float acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc = fmaf(__uint_as_float(w[j] << 16), __uint_as_float(x[j] << 16), acc);
    acc = fmaf(__uint_as_float(w[j] & 0xFFFF0000u), __uint_as_float(x[j] & 0xFFFF0000u), acc);
  }
  return acc;
}

enum Epi { kPlain = 0, kBiasResidual = 1, kQkv = 2 };

struct Args {
  const uint16_t* x;
  int M, K;
  const uint16_t* W;
  int N;
  uint16_t* out;
  const uint16_t* norm_w;  // non-null: RMSNorm the staged rows first
  float eps;
  const uint16_t* bias;
  const uint16_t* res;
  // QKV epilogue
  const int* positions;
  const int* slots;
  const float* inv_freq;
  float conc;
  uint8_t* cache;
  int num_pages;
  uint16_t* q_out;
};

template <int RW, int EPI, int MM>
__global__ __launch_bounds__(kThreads) void gemv_kernel(Args a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint16_t xs[];  // the M token rows, M * K bf16
  __shared__ float part[kWaves][RW][kMaxM];
  __shared__ double ssq[kWaves][kMaxM];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int M = a.M, K = a.K, N = a.N;
  const int chunks = K / 8;
  // this workgroup's rows
  int rows[RW];
  if constexpr (EPI == kQkv) {
    // rope pairs (j, j + 32) of head h: workgroup g takes pairs
    // j = (RW / 2) * (g % (32 / (RW / 2))) .. + RW / 2 - 1
    constexpr int kPairs = RW / 2, kBlocks = 32 / kPairs;
    const int h = blockIdx.x / kBlocks, jb = blockIdx.x % kBlocks;
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      rows[2 * i] = h * kD + jb * kPairs + i;
      rows[2 * i + 1] = h * kD + jb * kPairs + i + 32;
    }
  } else {
#pragma unroll
    for (int i = 0; i < RW; ++i) rows[i] = blockIdx.x * RW + i;
  }
  // x's chunks of this thread (one token: at eight, holding them would cost
  // occupancy) and the epilogue's operands first (they are needed first),
  // then every W load of this lane (K <= 4096: at most two rounds of 256
  // 16-byte chunks) with the norm weight's chunks when the rows are
  // normalised.  Every load is unconditional (indices clamped into range,
  // values past the row never used, raw bits converted where they are
  // used): a load under a branch made the compiler wait for it inside the
  // branch, which split the weight loads into three rounds with a full wait
  // between them.
  const bool norm = a.norm_w != nullptr;
  const uint16_t* const nw = norm ? a.norm_w : a.W;  // (loaded, unused, without a norm)
  constexpr bool kEarlyX = MM == 1;
  u32x4 xr[kEarlyX ? 1 : 0 + 1][kIters];
  if constexpr (kEarlyX) {
#pragma unroll
    for (int it = 0; it < kIters; ++it)
      xr[0][it] = *(const u32x4*)(a.x + min(it * kThreads + t, chunks - 1) * 8);
  }
  // the epilogue task of this thread (one per row or rope pair, and token)
  constexpr int kTasks = EPI == kQkv ? RW / 2 : RW;
  const bool task = t < kTasks * M;
  const int ti = task ? t / M : 0, tm = task ? t % M : 0;
  uint16_t eb0r = 0, eb1r = 0, err = 0;
  float cs = 0.f, sn = 0.f, ifq = 0.f;
  int eslot = -1, epos = 0;
  if constexpr (EPI == kBiasResidual) {
    const int n = min(rows[ti], N - 1);
    eb0r = a.bias[n];
    err = a.res[(size_t)tm * N + n];
  } else if constexpr (EPI == kQkv) {
    const int nlo = rows[2 * ti], nhi = rows[2 * ti + 1];
    eb0r = a.bias[nlo];
    eb1r = a.bias[nhi];
    eslot = a.slots[tm];
    epos = a.positions[tm];
    ifq = a.inv_freq[nlo % kD];
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[kIters][RW];
  u32x4 nwv[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int cc = min(it * kThreads + wave * 64 + lane, chunks - 1);
#pragma unroll
    for (int i = 0; i < RW; ++i)
      wv[it][i] = *(const u32x4*)(a.W + (size_t)min(rows[i], N - 1) * K + cc * 8);
    nwv[it] = *(const u32x4*)(nw + cc * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the RoPE factors while W streams
  if constexpr (EPI == kQkv) {
    if (task && rows[2 * ti] / kD < kHq + kHkv) {
      const float freq = (float)epos * ifq;
      const double fd = (double)freq;
      cs = bf2f(f2bf((float)cos(fd))) * a.conc;
      sn = bf2f(f2bf((float)sin(fd))) * a.conc;
    }
  }
  // Stage x; for the RMSNorm, the sum of squares of the bf16 values in fp64
  // (exact for rows spanning less than 2^37) on the way, as the standalone
  // kernel: r = fp32(1 / sqrt(ss / K + eps)), t = bf16(fp32(x r) w)
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m >= M) break;
    double ss = 0.0;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int c = it * kThreads + t;
      if (c >= chunks) continue;
      const u32x4 v = kEarlyX ? xr[0][it] : *(const u32x4*)(a.x + (size_t)m * K + c * 8);
      *(u32x4*)(xs + m * K + c * 8) = v;
      if (norm) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const double lo = (double)__uint_as_float(v[j] << 16);
          const double hi = (double)__uint_as_float(v[j] & 0xFFFF0000u);
          ss += lo * lo + hi * hi;
        }
      }
    }
    if (norm) {
      ss = moe::wave_sum(ss);
      if (lane == 0) ssq[wave][m] = ss;
    }
  }
  __syncthreads();
  float rn[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    rn[m] = 1.0f;
    if (norm && m < M) {
      const double tot = (ssq[0][m] + ssq[1][m]) + (ssq[2][m] + ssq[3][m]);
      rn[m] = (float)(1.0 / sqrt(tot / (double)K + (double)a.eps));
    }
  }
  float acc[RW][MM];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[i][m] = 0.f;
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int c = it * kThreads + wave * 64 + lane;
    if (c < chunks) {
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (m < M) {
          u32x4 xv = *(const u32x4*)(xs + m * K + c * 8);
          if (norm) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t lo = f2bf(__fmul_rn(__fmul_rn(__uint_as_float(xv[j] << 16), rn[m]),
                                                 __uint_as_float(nwv[it][j] << 16)));
              const uint32_t hi = f2bf(__fmul_rn(__fmul_rn(__uint_as_float(xv[j] & 0xFFFF0000u),
                                                           rn[m]),
                                                 __uint_as_float(nwv[it][j] & 0xFFFF0000u)));
              xv[j] = lo | (hi << 16);
            }
          }
#pragma unroll
          for (int i = 0; i < RW; ++i) acc[i][m] = dot8(wv[it][i], xv, acc[i][m]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int m = 0; m < MM; ++m)
      if (m < M) {
        const float v = moe::wave_sum(acc[i][m]);
        if (lane == 0) part[wave][i][m] = v;
      }
  __syncthreads();
  // epilogue: one thread per (row or rope pair, token); partials in wave order
  auto total = [&](int i, int m) {
    return ((part[0][i][m] + part[1][i][m]) + part[2][i][m]) + part[3][i][m];
  };
  if constexpr (EPI == kPlain || EPI == kBiasResidual) {
    if (task) {
      const int i = ti, m = tm, n = rows[i];
      if (n < N) {
        const uint16_t y = f2bf(total(i, m));
        if constexpr (EPI == kPlain) {
          a.out[(size_t)m * N + n] = y;
        } else {
          const float tb = bf2f(f2bf(bf2f(y) + bf2f(eb0r)));
          a.out[(size_t)m * N + n] = f2bf(bf2f(err) + tb);
        }
      }
    }
  } else {
    // bias (its own bf16 rounding), then YaRN RoPE of q / k heads exactly as
    // the standalone append kernel does, then q out or the cache slot
    if (task) {
      const int i = ti, m = tm;
      const int nlo = rows[2 * i];
      const int head = nlo / kD, d = nlo % kD;
      float lo = bf2f(f2bf(bf2f(f2bf(total(2 * i, m))) + bf2f(eb0r)));
      float hi = bf2f(f2bf(bf2f(f2bf(total(2 * i + 1, m))) + bf2f(eb1r)));
      if (head < kHq + kHkv) {
        const float nl = lo * cs - hi * sn;
        const float nh = lo * sn + hi * cs;
        lo = nl;
        hi = nh;
      }
      const uint16_t blo = f2bf(lo), bhi = f2bf(hi);
      const int slot = eslot;
      if (head < kHq) {
        uint16_t* qo = a.q_out + ((size_t)m * kHq + head) * kD;
        qo[d] = blo;
        qo[d + 32] = bhi;
      } else if (slot >= 0 && slot < a.num_pages * kPage) {
        const int kv = head < kHq + kHkv ? 0 : 1;
        const int hk = head - kHq - kv * kHkv;
        uint16_t* row = (uint16_t*)(a.cache + (size_t)(slot / kPage) * kPageBytes +
                                    (size_t)(kv * kHkv + hk) * kHeadBlock +
                                    (slot % kPage) * (kD * 2));
        row[d] = blo;
        row[d + 32] = bhi;
      }
    }
  }
}

}  // namespace gemv

extern "C" {

int attn_launch_gemv(const void* x, int M, int K, const void* W, int N, void* out,
                     const void* norm_w, float eps, const void* bias, const void* res,
                     hipStream_t s) {
  using namespace gemv;
  Args a{};
  a.x = (const uint16_t*)x;
  a.M = M;
  a.K = K;
  a.W = (const uint16_t*)W;
  a.N = N;
  a.out = (uint16_t*)out;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  a.bias = (const uint16_t*)bias;
  a.res = (const uint16_t*)res;
  const size_t lds = (size_t)M * K * 2;
  // one token (batch-1 decode): accumulators for one row of x only
  if (bias) {
    constexpr int RW = 4;
    const dim3 grid((N + RW - 1) / RW);
    if (M == 1)
      hipLaunchKernelGGL((gemv_kernel<RW, kBiasResidual, 1>), grid, dim3(kThreads), lds, s, a);
    else
      hipLaunchKernelGGL((gemv_kernel<RW, kBiasResidual, kMaxM>), grid, dim3(kThreads), lds, s, a);
  } else if (M == 1) {
    constexpr int RW = 16;
    hipLaunchKernelGGL((gemv_kernel<RW, kPlain, 1>), dim3((N + RW - 1) / RW), dim3(kThreads), lds,
                       s, a);
  } else {
    constexpr int RW = 8;
    hipLaunchKernelGGL((gemv_kernel<RW, kPlain, kMaxM>), dim3((N + RW - 1) / RW), dim3(kThreads),
                       lds, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_qkv_gemv(const void* x, int M, int K, const void* W, const void* norm_w,
                         float eps, const void* bias, const int* positions, const int* slots,
                         const float* inv_freq, float conc, void* cache, int num_pages,
                         void* q_out, hipStream_t s) {
  using namespace gemv;
  constexpr int heads = kHq + 2 * kHkv;
  constexpr int RW = 4;  // two rope pairs per workgroup
  Args a{};
  a.x = (const uint16_t*)x;
  a.M = M;
  a.K = K;
  a.W = (const uint16_t*)W;
  a.N = heads * kD;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  a.bias = (const uint16_t*)bias;
  a.positions = positions;
  a.slots = slots;
  a.inv_freq = inv_freq;
  a.conc = conc;
  a.cache = (uint8_t*)cache;
  a.num_pages = num_pages;
  a.q_out = (uint16_t*)q_out;
  const dim3 grid(heads * (32 / (RW / 2)));
  if (M == 1)
    hipLaunchKernelGGL((gemv_kernel<RW, kQkv, 1>), grid, dim3(kThreads), (size_t)K * 2, s, a);
  else
    hipLaunchKernelGGL((gemv_kernel<RW, kQkv, kMaxM>), grid, dim3(kThreads), (size_t)M * K * 2, s,
                       a);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // extern "C"
