// Shared device helpers for the gfx950 MXFP4 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

constexpr int kWave = 64;

// Status codes returned across the C ABI (mirrored in include/moe_gfx950.h).
enum Status : int {
  kOk = 0,
  kErrNull = -1,
  kErrShape = -2,
  kErrAlign = -3,
  kErrUnsupported = -4,
  kErrLaunch = -5,
  kErrWorkspace = -6,
  kErrIncomplete = -7,
};

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// fp64 -> fp32 (RNE) -> bf16 (RNE): two roundings, as an fp32 result stored
// to bf16.  The opaque fp32 step keeps the compiler from folding the pair
// into one fp64 -> bf16 conversion, which rounds differently when the fp32
// value lands on a bf16 tie.
__device__ __forceinline__ uint16_t f64_to_bf16_via_f32(double v) {
  float f = (float)v;
  asm volatile("" : "+v"(f));
  return f2bf(f);
}

// E8M0 byte -> fp32 2^(s-127); s = 0 is the fp32 subnormal 2^-127 and s = 255
// is +inf, as exp2(float(s - 127)) gives (model/mlp.py:297-298).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return s == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(s << 23);
}

// e2m1 code -> fp32 value (model/mlp.py:9-26), by construction from the bits:
// exponent field e = (c>>1)&3, mantissa bit m = c&1; e = 0 is the subnormal
// 0.5*m, otherwise 2^(e-1) * (1 + m/2); bit 3 is the sign.
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
  const uint32_t e = (c >> 1) & 3u, m = c & 1u;
  const float mag = e == 0 ? 0.5f * (float)m : __uint_as_float((126u + e) << 23) * (1.0f + 0.5f * (float)m);
  return (c & 8u) ? -mag : mag;
}

// Eight e2m1 codes (one dword, element 2b from the low nibble of byte b) ->
// eight bf16 values scaled by 2^(s-127) via gfx950's scaled fp4 conversion.
// Exact for scales whose products stay normal in bf16.
__device__ __forceinline__ bf16x8 dequant8(uint32_t w, float scale) {
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Split eight fp32 values into bf16 hi + bf16 lo with a = hi + lo + O(2^-17 |a|).
__device__ __forceinline__ void split8(const float* a, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const __bf16 h = (__bf16)a[i];
    hi[i] = h;
    lo[i] = (__bf16)(a[i] - (float)h);
  }
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// fp8 e4m3 (OCP: bias 7, no infinities, max 448), through gfx950's
// conversions: v_cvt_pk_fp8_f32 rounds to nearest even (subnormals included),
// v_cvt_f32_fp8 is exact.  Four values -> four codes, value j in byte j.
__device__ __forceinline__ uint32_t e4m3_pack4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Value of byte J of a word of e4m3 codes.
template <int J>
__device__ __forceinline__ float e4m3_byte(uint32_t w) {
  return __builtin_amdgcn_cvt_f32_fp8((int)w, J);
}

// Eight values r (each |r| * inv < 256) -> eight e4m3 codes of r * inv in
// (lo, hi), and r minus the value each code stands for (times sc = 1 / inv;
// exact: the code's value is a rounding of r * inv).
__device__ __forceinline__ void e4m3_piece8(float* r, float inv, float sc, uint32_t& lo,
                                            uint32_t& hi) {
  lo = e4m3_pack4(r[0] * inv, r[1] * inv, r[2] * inv, r[3] * inv);
  hi = e4m3_pack4(r[4] * inv, r[5] * inv, r[6] * inv, r[7] * inv);
  r[0] -= e4m3_byte<0>(lo) * sc;
  r[1] -= e4m3_byte<1>(lo) * sc;
  r[2] -= e4m3_byte<2>(lo) * sc;
  r[3] -= e4m3_byte<3>(lo) * sc;
  r[4] -= e4m3_byte<0>(hi) * sc;
  r[5] -= e4m3_byte<1>(hi) * sc;
  r[6] -= e4m3_byte<2>(hi) * sc;
  r[7] -= e4m3_byte<3>(hi) * sc;
}

// E8M0 exponent byte for a group whose largest magnitude is amax: the smallest
// scale 2^(s-127) with amax / scale < 256, i.e. s = floor(log2(amax)) - 7 + 127
// (s = 0 when amax is zero or tiny), so the group's codes stay below 256.
__device__ __forceinline__ uint32_t e8m0_for_amax(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu);  // biased exponent of amax
  const int s = e - 7;
  return (uint32_t)(s < 0 ? 0 : s);
}

// v_mfma_scale_f32_16x16x128_f8f6f4, A = fp4 e2m1 (cbsz 4), B = fp8 e4m3
// (blgp 0), one E8M0 byte per lane for each operand (byte 0 of the VGPR).
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
__device__ __forceinline__ f32x4 mfma_mx(const i32x8& a, const i32x8& b, f32x4 c, int sa,
                                         int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, 0, sa, 0, sb);
}

// x of lane l ^ 1 and of lane l ^ 2: DPP quad permutes [1,0,3,2] and
// [2,3,0,1], a register move with no LDS round trip (a shuffle through
// ds_bpermute waits for the LDS).  All lanes of the quad must be active.
__device__ __forceinline__ float lane_xor1(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor2(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
}

// A 64-bit value moved between lanes by one DPP pattern (two 32-bit moves);
// lanes outside ROW_MASK get 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK,
                                                            0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL,
                                                            ROW_MASK, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum of v over the 64 lanes in a fixed order (DPP tree: pairs, quads,
// half-rows, rows, then rows 0+1 and 2+3, then all four), returned to every
// lane.  All lanes must be active.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_f64<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_f64<0x141>(v);       // row_half_mirror
  v += dpp_f64<0x140>(v);       // row_mirror
  v += dpp_f64<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f64<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// LDS pointer type of the direct global-to-LDS loads (global_load_lds).
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Workgroup barrier for LDS hand-offs that leaves global loads in flight:
// waits for this wave's LDS operations only, then s_barrier.  __syncthreads'
// release fence would also wait for every outstanding global load (vmcnt(0)),
// which drains a load pipeline at each barrier.  The memory clobber keeps the
// compiler from moving memory accesses across it.  LDS written by
// global_load_lds must be covered by a vmcnt wait before it.
// Ranking keys of bf16 logits: the order-preserving unsigned image of the
// value in the high 16 bits, 0xFFFF - expert in the low 16, so that a larger
// key means (value larger, or value equal and expert lower).  Logits are bf16
// values (low 16 bits zero); -inf pads rank below every finite logit.
__device__ __forceinline__ uint32_t rank_key(float v, int e) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (u & 0xFFFF0000u) | (uint32_t)(0xFFFF - e);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  const uint32_t hi = key & 0xFFFF0000u;
  return __uint_as_float((hi & 0x80000000u) ? (hi ^ 0x80000000u) : (~hi & 0xFFFF0000u));
}

// Cache-policy operand of the global_load_lds builtin: sc1 = device scope.
constexpr int kCpolSc1 = 16;  // also the aux operand of the buffer-load builtins
// Word 3 of a raw buffer resource (32-bit data format; byte offsets, no
// swizzle): loads past num_records return zero.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Device-scope (agent) relaxed stores and loads: on gfx950 the stores write
// through (sc1) and the loads bypass the non-coherent caches, so data passes
// between workgroups on different XCDs (each XCD has its own L2) within one
// launch.  The writer waits for its stores (vmcnt) before the release count.
template <class T>
__device__ __forceinline__ void store_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T load_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// s_waitcnt with only the vector-memory count: vmcnt(n), n < 64
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace moe
