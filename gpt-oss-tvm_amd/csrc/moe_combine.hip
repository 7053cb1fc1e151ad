// Gate-weighted combine of the k expert outputs (+ residual), and the
// standalone SwiGLU.
//
// Combine: moe_gemv_gating, model/mlp.py:328-369 -- fp32 sum over slots
// r = 0..k-1 in order, starting from 0, of y[s,r,c] * w[s,r], rounded to bf16;
// then the residual of model/mlp.py:402, bf16(x + moe).  The multiply and the
// add round separately, as written.
// SwiGLU: model/mlp.py:29-60 with out_dtype float32.
#include "moe_common.h"

namespace moe {

// One thread per 4 output columns of one token; grid (ceil(N/1024), n).
// status (if not null): nonzero when the producer of y reported incomplete
// results (the decode launch's bounded wait gave up); every output is then
// written as NaN, so a wrong result cannot pass for a right one.
// KT > 0: k == KT known at compile time (the loads of every slot issued
// without a branch between them); KT == 0: any k <= 8.
template <int KT>
__global__ __launch_bounds__(256) void moe_gating_kernel(const float* __restrict__ y,
                                                         const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ x, int k,
                                                         int N, uint16_t* __restrict__ out,
                                                         const int* __restrict__ status) {
  // multiply and add round separately, as the reference writes them: no
  // contraction into fma (__fmul_rn / __fadd_rn alone do not prevent it)
#pragma clang fp contract(off)
  const int tok = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= N) return;
  // Every load in one round: the k rows and weights, the residual and the
  // status word, so the kernel waits for one memory round trip, not for the
  // status before the rows.  Then the in-order sum.  (With k known only at
  // run time the compiler waits for each slot's weight inside its branch.)
  if constexpr (KT > 0) k = KT;
  constexpr int kMax = KT > 0 ? KT : 8;
  f32x4 v[kMax];
  uint16_t wraw[kMax];
#pragma unroll
  for (int r = 0; r < kMax; ++r) {
    if (KT > 0 || r < k) {
      v[r] = *(const f32x4*)(y + ((size_t)tok * k + r) * N + c);
      wraw[r] = w[(size_t)tok * k + r];
    }
  }
  uint16_t xr[4] = {0, 0, 0, 0};
  if (x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[i] = x[(size_t)tok * N + c + i];
  }
  const int st = status ? *status : 0;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < kMax; ++r) {
    if (KT > 0 || r < k) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + v[r][i] * bf2f(wraw[r]);
    }
  }
  uint16_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t g = f2bf(acc[i]);
    o[i] = x ? f2bf(__fadd_rn(bf2f(xr[i]), bf2f(g))) : g;
  }
  uint2 pk;
  pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
  pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
  if (st != 0) pk = make_uint2(0x7FC07FC0u, 0x7FC07FC0u);
  *(uint2*)(out + (size_t)tok * N + c) = pk;
}

__global__ __launch_bounds__(256) void moe_swiglu_kernel(const float2* __restrict__ x,
                                                         int64_t pairs, float alpha, float limit,
                                                         float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= pairs) return;
  const float2 v = x[i];
  const float xg = fminf(v.x, limit);
  const float xl = fminf(fmaxf(v.y, -limit), limit);
  const float z = __fmul_rn(alpha, xg);
  const float sig = 1.0f / (1.0f + expf(-z));
  out[i] = __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
}

}  // namespace moe

extern "C" int moe_launch_gating(const void* y, const void* w, const void* x, int n, int k, int N,
                                 void* out, const void* status, hipStream_t stream) {
  if (n == 0) return moe::kOk;
  const dim3 grid((N / 4 + 255) / 256, n);
  if (k == 4)
    hipLaunchKernelGGL(moe::moe_gating_kernel<4>, grid, dim3(256), 0, stream, (const float*)y,
                       (const uint16_t*)w, (const uint16_t*)x, k, N, (uint16_t*)out,
                       (const int*)status);
  else
    hipLaunchKernelGGL(moe::moe_gating_kernel<0>, grid, dim3(256), 0, stream, (const float*)y,
                       (const uint16_t*)w, (const uint16_t*)x, k, N, (uint16_t*)out,
                       (const int*)status);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}

extern "C" int moe_launch_swiglu(const void* x, int64_t pairs, float alpha, float limit, void* out,
                                 hipStream_t stream) {
  if (pairs == 0) return moe::kOk;
  hipLaunchKernelGGL(moe::moe_swiglu_kernel, dim3((uint32_t)((pairs + 255) / 256)), dim3(256), 0,
                     stream, (const float2*)x, pairs, alpha, limit, (float*)out);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
