// Standalone MXFP4 -> bf16 dequantisation.
//
// moe_dequant_kernel restates the reference's dequant_mxfp4 prim_func
// (model/mlp.py:172-234): out[r, 2j] = bf16(LUT[lo(b)] * 2^(s-127)),
// out[r, 2j+1] = bf16(LUT[hi(b)] * 2^(s-127)), product in fp32.  It is exact
// for every (byte, scale) pair including the subnormal (s <= 1) and
// infinite (s = 255) corners.
//
// moe_dequant_fast_kernel produces the same output through dequant8(), the
// hardware conversion the expert matmuls use, so that tests can pin the fused
// path's dequantisation bit for bit.
#include "moe_common.h"

namespace moe {

__global__ __launch_bounds__(256) void moe_dequant_kernel(const u32x4* __restrict__ blocks,
                                                          const uint8_t* __restrict__ scales,
                                                          u32x4* __restrict__ out, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const u32x4 b = blocks[r];
  const float sc = e8m0_to_f32(scales[r]);
  uint32_t packed[16];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = (b[d] >> (8 * j)) & 0xFFu;
      const uint16_t lo = f2bf(__fmul_rn(e2m1_to_f32(byte & 0xFu), sc));
      const uint16_t hi = f2bf(__fmul_rn(e2m1_to_f32(byte >> 4), sc));
      packed[4 * d + j] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    out[r * 4 + q] = u32x4{packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]};
}

__global__ __launch_bounds__(256) void moe_dequant_fast_kernel(const u32x4* __restrict__ blocks,
                                                               const uint8_t* __restrict__ scales,
                                                               u32x4* __restrict__ out, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const u32x4 b = blocks[r];
  const float sc = e8m0_to_f32(scales[r]);
#pragma unroll
  for (int d = 0; d < 4; ++d) out[r * 4 + d] = __builtin_bit_cast(u32x4, dequant8(b[d], sc));
}

}  // namespace moe

extern "C" int moe_launch_dequant(const void* blocks, const void* scales, void* out, int64_t rows,
                                  int fast, hipStream_t stream) {
  if (rows == 0) return moe::kOk;
  const int threads = 256;
  const int64_t grid = (rows + threads - 1) / threads;
  if (fast)
    hipLaunchKernelGGL(moe::moe_dequant_fast_kernel, dim3((uint32_t)grid), dim3(threads), 0, stream,
                       (const moe::u32x4*)blocks, (const uint8_t*)scales, (moe::u32x4*)out, rows);
  else
    hipLaunchKernelGGL(moe::moe_dequant_kernel, dim3((uint32_t)grid), dim3(threads), 0, stream,
                       (const moe::u32x4*)blocks, (const uint8_t*)scales, (moe::u32x4*)out, rows);
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
