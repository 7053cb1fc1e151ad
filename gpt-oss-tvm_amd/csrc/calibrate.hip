// HBM read calibration: a plain streaming read of a large buffer, the
// achievable-bandwidth ceiling the MoE kernels' HBM fractions are read
// against (the datasheet's 8 TB/s is not reached by any access pattern).
// No reference counterpart: a measurement hook.
//
// Grid-stride loop: workgroup b, iteration i reads U consecutive 4 KB pieces
// (256 lanes x 16 bytes, one global_load_dwordx4 per lane each), all U
// issued before any is used; the values are folded into one word that is
// stored only if it equals a constant no data produces, so the loads stay.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "moe_common.h"

namespace moe {

template <int U>
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                       uint32_t* __restrict__ sink) {
  uint32_t acc = 0u;
  const size_t step = (size_t)gridDim.x * 256 * U;
  for (size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x; i < n16; i += step) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + (size_t)u * 256;
      v[u] = j < n16 ? p[j] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

}  // namespace moe

extern "C" int moe_launch_hbm_read(const void* src, size_t bytes, int grid, int unroll,
                                   uint32_t* sink, hipStream_t stream) {
  if (!src || !sink) return moe::kErrUnsupported;
  if (grid < 1 || bytes < 16 || (bytes & 15) || ((uintptr_t)src & 15)) return moe::kErrUnsupported;
  const size_t n16 = bytes / 16;
  const moe::u32x4* p = (const moe::u32x4*)src;
  if (unroll == 4)
    hipLaunchKernelGGL(moe::hbm_read_kernel<4>, dim3(grid), dim3(256), 0, stream, p, n16, sink);
  else if (unroll == 8)
    hipLaunchKernelGGL(moe::hbm_read_kernel<8>, dim3(grid), dim3(256), 0, stream, p, n16, sink);
  else if (unroll == 16)
    hipLaunchKernelGGL(moe::hbm_read_kernel<16>, dim3(grid), dim3(256), 0, stream, p, n16, sink);
  else
    return moe::kErrUnsupported;
  return hipGetLastError() == hipSuccess ? moe::kOk : moe::kErrLaunch;
}
