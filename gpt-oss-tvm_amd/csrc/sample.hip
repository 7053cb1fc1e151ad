// Top-p sampling of the next token on the GPU (engine.py:165-167: TVM's
// vm.builtin.sample_top_p_from_logits, called with temperature 0.7, top_p 0.9
// and a fixed uniform sample 0.5 at engine.py:40).
//
// The algorithm sorts the logits in descending order, takes e = exp((l - max)
// / T) and p = e / sum(e); it returns the largest element at once when the
// uniform sample is below p_max / top_p, and otherwise the first element whose
// cumulative probability over the top-p mass exceeds the uniform sample, where
// the top-p mass is the sum up to and including the element at which the
// running sum reaches top_p.
//
// The model's logits are bf16 values (the unembedding's bf16 output cast to
// fp32, model/transformer.py:95-100), so a sequence has at most 65536 distinct
// logit values.  Instead of a sort:
//   1. count the elements of each value in a 65536-bin histogram (integer
//      atomics: deterministic) and take the maximum; each workgroup counts
//      its 16384 elements in LDS first and adds one global atomic per value
//      it saw;
//   2. the masses of 64 segments of 1024 bins (descending values): mass of a
//      bin = count x exp((v - max) / T), summed per segment in a fixed order;
//   3. one workgroup finds the two crossings (top_p, then u times the top-p
//      mass): the segment from the 64 segment masses, the bin from a scan of
//      that segment's 1024 masses, the element inside the bin in fp64; the
//      result is a value v* and a rank j* among the elements of that value
//      (equal logits are taken in index order);
//   4. the j*-th element of value v* in index order: matches counted per
//      index range by 64 workgroups, then the owning range searched by one.
// The histogram is left zeroed after each call (it must be zero before the
// first): nothing is cleared with a memset, so the calls can be captured.
//
// Numerics: the exponent's argument in fp32 as written, exp rounded once to
// fp32, masses summed in fp64 (exact to far below an element's share); the
// restated algorithm adds fp32 values serially in an order TVM does not
// expose, whose error at this vocabulary size (about 1e-3 relative) can move
// the choice by a rank, so the exact sums are the definition here.
#include "moe_common.h"

namespace smp {

using moe::bf2f;
using moe::u32x4;

constexpr int kBins = 65536;
constexpr int kSegBins = 1024;           // bins per mass segment (one thread each)
constexpr int kSegs = kBins / kSegBins;  // 64

// exp((v - max) * scale): the argument in fp32 as written, exp rounded once
// to fp32 (through fp64), carried as fp64 for the exact sums
__device__ __forceinline__ double weight(float v, float m, float scale) {
  const float arg = (v - m) * scale;
  return (double)(float)exp((double)arg);
}

// order-preserving key of a bf16 value: larger value -> larger key
__device__ __forceinline__ uint32_t key16(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__device__ __forceinline__ float value_of(uint32_t k) {
  const uint32_t b = (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
  return bf2f((uint16_t)b);
}

struct State {  // per sequence, after the histogram
  uint32_t counts[kBins];
  uint32_t max_key;
  uint32_t pick_key;  // value of the chosen element
  uint32_t pick_rank; // 1-based rank among the elements of that value
  uint32_t pad;
  uint32_t part_count[64];  // matches of the chosen value per index range
  double seg_mass[kSegs];   // mass of bins 65535 - 1024 p - [0, 1024) per segment p
};

// 1. histogram and maximum.  Grid (ceil(V / 16384), batch), 1024 threads x 16
// elements.  The workgroup's counts go to LDS first as 16-bit counters, two
// per word (a workgroup sees at most 16384 elements, so a count never carries
// into its neighbour), then one global atomic per nonzero bin.
constexpr int kHistThreads = 1024;
constexpr int kHistElems = kHistThreads * 16;
constexpr size_t kHistLds = kBins * 2;  // 128 KB

__global__ __launch_bounds__(kHistThreads) void hist_kernel(const uint16_t* __restrict__ logits,
                                                            int V, State* __restrict__ st) {
  extern __shared__ __align__(16) uint32_t h[];  // kBins / 2 words
  const int b = blockIdx.y, t = threadIdx.x;
  const uint16_t* l = logits + (size_t)b * V;
  State& s = st[b];
  for (int i = t; i < kBins / 8; i += kHistThreads) ((u32x4*)h)[i] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
  uint32_t mk = 0;
  auto add = [&](uint32_t k) {
    atomicAdd(&h[k >> 1], 1u << ((k & 1u) << 4));
    mk = max(mk, k);
  };
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i0 = blockIdx.x * kHistElems + (j * kHistThreads + t) * 8;
    if (i0 + 8 <= V && (V & 7) == 0) {
      const u32x4 v = *(const u32x4*)(l + i0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        add(key16(v[q] & 0xFFFFu));
        add(key16(v[q] >> 16));
      }
    } else {
      for (int i = i0; i < min(i0 + 8, V); ++i) add(key16(l[i]));
    }
  }
  __syncthreads();
  for (int i = t; i < kBins / 8; i += kHistThreads) {
    const u32x4 v = ((const u32x4*)h)[i];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (v[q] & 0xFFFFu) atomicAdd(&s.counts[8 * i + 2 * q], v[q] & 0xFFFFu);
      if (v[q] >> 16) atomicAdd(&s.counts[8 * i + 2 * q + 1], v[q] >> 16);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mk = max(mk, (uint32_t)__shfl_xor((int)mk, off, 64));
  if ((t & 63) == 0 && mk) atomicMax(&s.max_key, mk);
}

// Fixed-order sums over a 1024-thread workgroup: exclusive prefix of v in
// thread order (lane scan, then the 16 wave totals in order) and the total.
__device__ double block_exclusive_scan(double v, double* tmp, double* total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  double incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) tmp[w] = incl;
  __syncthreads();
  if (t == 0) {
    double acc = 0.0;
    for (int i = 0; i < kSegBins / 64; ++i) {
      const double x = tmp[i];
      tmp[i] = acc;
      acc += x;
    }
    *total = acc;
  }
  __syncthreads();
  const double r = tmp[w] + incl - v;
  __syncthreads();
  return r;
}

// The mass of bin key k (0 for an empty bin).
__device__ __forceinline__ double bin_mass(uint32_t c, uint32_t k, float m, float scale) {
  return c ? (double)c * weight(value_of(k), m, scale) : 0.0;
}

// 2. segment masses.  Grid (64, batch), 1024 threads: thread t of segment p
// holds bin 65535 - 1024 p - t.
__global__ __launch_bounds__(kSegBins) void mass_kernel(State* __restrict__ st,
                                                        float temperature) {
  __shared__ double tmp[kSegBins / 64];
  __shared__ double tot;
  if (temperature < 1e-6f) return;  // argmax: no masses
  State& s = st[blockIdx.y];
  const int p = blockIdx.x;
  const uint32_t k = 65535u - kSegBins * p - threadIdx.x;
  const double v = bin_mass(s.counts[k], k, value_of(s.max_key), 1.0f / temperature);
  block_exclusive_scan(v, tmp, &tot);
  if (threadIdx.x == 0) s.seg_mass[p] = tot;
}

// 3. the two crossings.  One 1024-thread workgroup per sequence.
__global__ __launch_bounds__(kSegBins) void select_kernel(State* __restrict__ st,
                                                          float temperature, float top_p,
                                                          float uniform) {
  __shared__ double tmp[kSegBins / 64];
  __shared__ double segm[kSegs];
  __shared__ double segpre[kSegs + 1];  // exclusive prefix of the segment masses
  __shared__ double tot_s, crossing_s;
  __shared__ int seg_s, owner, last_nz;
  State& s = st[blockIdx.x];
  const int t = threadIdx.x;
  const uint32_t mk = s.max_key;
  const float m = value_of(mk);
  if (temperature < 1e-6f) {
    // argmax: the first element of the largest value
    if (t == 0) {
      s.pick_key = mk;
      s.pick_rank = 1;
    }
  } else {
    const float scale = 1.0f / temperature;
    if (t < kSegs) segm[t] = s.seg_mass[t];
    __syncthreads();
    if (t == 0) {
      double acc = 0.0;
      for (int p = 0; p < kSegs; ++p) {
        segpre[p] = acc;
        acc += segm[p];
      }
      segpre[kSegs] = acc;
    }
    __syncthreads();
    // TVM's short cut (SampleTopPFromProb): uniform < p_max / top_p returns
    // the argmax before the top-p mass is formed.  The largest value's weight
    // is exp(0) = 1, so p_max = 1 / total.  Uniform over the workgroup.
    if ((double)uniform < (1.0 / segpre[kSegs]) / (double)top_p) {
      if (t == 0) {
        s.pick_key = mk;
        s.pick_rank = 1;
      }
      return;
    }
    // The segment whose range [segpre[p], segpre[p + 1]) holds a crossing
    // (strict: the first with segpre[p] <= x < segpre[p + 1], else the first
    // with segpre[p] < x <= segpre[p + 1]), then the bin: the segment's 1024
    // masses scanned in bin order from segpre[p]; owner = the first bin whose
    // range holds x.  A rounding difference between the segment's own sum and
    // its scan leaves the owner at kSegBins (none).
    auto locate = [&](double x, bool strict, uint32_t& c, uint32_t& k, double& before,
                      double& mass) -> int {
      if (t == 0) {
        seg_s = -1;
        owner = kSegBins;
        last_nz = -1;
        for (int p = 0; p < kSegs; ++p) {
          const bool in = strict ? (segpre[p] <= x && x < segpre[p + 1])
                                 : (segpre[p] < x && x <= segpre[p + 1]);
          if (in) {
            seg_s = p;
            break;
          }
        }
      }
      __syncthreads();
      const int p = seg_s;
      if (p < 0) return -1;  // uniform
      k = 65535u - kSegBins * p - t;
      c = s.counts[k];
      mass = bin_mass(c, k, m, scale);
      before = segpre[p] + block_exclusive_scan(mass, tmp, &tot_s);
      const bool in = strict ? (before <= x && x < before + mass)
                             : (before < x && x <= before + mass);
      if (in) atomicMin(&owner, t);
      if (c) atomicMax(&last_nz, t);
      __syncthreads();
      return p;
    };
    uint32_t c = 0, k = 0;
    double before = 0.0, mass = 0.0;
    // crossing 1: the element at which the running sum reaches top_p x total;
    // the top-p mass runs up to and including it
    const double tp = (double)top_p * segpre[kSegs];
    const int p1 = locate(tp, false, c, k, before, mass);
    if (t == 0) crossing_s = p1 < 0 ? segpre[kSegs] : segpre[p1 + 1];  // none: everything
    __syncthreads();
    if (p1 >= 0 && t == owner) {
      const double w = mass / c;
      const double j = ceil((tp - before) / w);  // elements with sum before < tp
      crossing_s = before + fmin(fmax(j, 1.0), (double)c) * w;
    }
    __syncthreads();
    // crossing 2: the first element whose cumulative mass exceeds u x top-p mass
    const double x = (double)uniform * crossing_s;
    const int p2 = locate(x, true, c, k, before, mass);
    if (p2 < 0) {
      // past the top-p mass: the first element of the largest value
      if (t == 0) {
        s.pick_key = mk;
        s.pick_rank = 1;
      }
    } else if (owner < kSegBins) {
      if (t == owner) {
        const double w = mass / c;
        const double j = floor((x - before) / w) + 1.0;
        s.pick_key = k;
        s.pick_rank = (uint32_t)fmin(fmax(j, 1.0), (double)c);
      }
    } else if (t == last_nz) {  // rounding put the crossing past the bins: the last element
      s.pick_key = k;
      s.pick_rank = c;
    }
  }
}

// 4. the pick_rank-th element of value pick_key, in index order, in two
// launches: count_kernel counts the matches of each of kFindParts contiguous
// ranges (16-byte loads) and leaves the histogram zeroed for the next call
// (part p clears bins [1024 p, 1024 p + 1024)), locate_kernel finds the range
// holding the wanted rank and the element inside it (a block-wide prefix over
// that range).
constexpr int kFindParts = 64;
constexpr int kFindThreads = 256;
constexpr int kLocThreads = 1024;
static_assert(kBins == kFindParts * kFindThreads * 4, "one 16-byte clear per thread");

__device__ __forceinline__ int part_begin(int V, int p) {
  // ranges of whole 8-element groups (the last one takes the remainder)
  const int groups = (V + 7) / 8;
  return min(V, (int)(((int64_t)groups * p / kFindParts) * 8));
}

__global__ __launch_bounds__(kFindThreads) void count_kernel(const uint16_t* __restrict__ logits,
                                                             int V, State* __restrict__ st) {
  __shared__ int wsum[kFindThreads / 64];
  const int b = blockIdx.y, p = blockIdx.x, t = threadIdx.x;
  const uint16_t* l = logits + (size_t)b * V;
  const uint32_t want = st[b].pick_key;
  ((u32x4*)st[b].counts)[p * kFindThreads + t] = u32x4{0u, 0u, 0u, 0u};
  if (p == 0 && t == 0) st[b].max_key = 0u;
  const int i0 = part_begin(V, p), i1 = part_begin(V, p + 1);
  int c = 0;
  for (int i = i0 + t * 8; i < i1; i += kFindThreads * 8) {
    if (i + 8 <= i1 && (V & 7) == 0) {
      const u32x4 v = *(const u32x4*)(l + i);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c += (key16(v[j] & 0xFFFFu) == want) + (key16(v[j] >> 16) == want);
    } else {
      for (int k = i; k < min(i + 8, i1); ++k) c += key16(l[k]) == want;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((t & 63) == 0) wsum[t >> 6] = c;
  __syncthreads();
  if (t == 0) st[b].part_count[p] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

__global__ __launch_bounds__(kLocThreads) void locate_kernel(const uint16_t* __restrict__ logits,
                                                             int V, const State* __restrict__ st,
                                                             int* __restrict__ out) {
  __shared__ int base_s, part_s;
  __shared__ int wsum[kLocThreads / 64];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint16_t* l = logits + (size_t)b * V;
  const State& s = st[b];
  const uint32_t want = s.pick_key;
  const int rank = (int)s.pick_rank;
  if (t == 0) {
    int acc = 0, p = 0;
    for (; p < kFindParts - 1 && acc + (int)s.part_count[p] < rank; ++p) acc += s.part_count[p];
    base_s = acc;
    part_s = p;
    out[b] = -1;  // replaced below
  }
  __syncthreads();
  const int i0 = part_begin(V, part_s), i1 = part_begin(V, part_s + 1);
  // chunks of kLocThreads elements in index order; a running count across them
  int before_chunk = base_s;
  for (int c0 = i0; c0 < i1; c0 += kLocThreads) {
    const int i = c0 + t;
    const int hit = i < i1 && key16(l[i]) == want;
    int incl = hit;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int pre = 0, total = 0;
    for (int k = 0; k < kLocThreads / 64; ++k) {
      pre += k < w ? wsum[k] : 0;
      total += wsum[k];
    }
    if (hit && before_chunk + pre + incl == rank) out[b] = i;
    before_chunk += total;
    __syncthreads();
    if (before_chunk >= rank) break;  // uniform: every thread has the same count
  }
}

}  // namespace smp

extern "C" {

size_t attn_sample_state_bytes() { return sizeof(smp::State); }

int attn_launch_sample(const void* logits, int batch, int V, float temperature, float top_p,
                       float uniform, int* out, void* state, hipStream_t s) {
  smp::State* st = (smp::State*)state;
  static const bool lds_ok =  // more than 64 KB of dynamic LDS, once
      hipFuncSetAttribute((const void*)smp::hist_kernel,
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)smp::kHistLds) == hipSuccess;
  if (!lds_ok) return -6;
  hipLaunchKernelGGL(smp::hist_kernel, dim3((V + smp::kHistElems - 1) / smp::kHistElems, batch),
                     dim3(smp::kHistThreads), smp::kHistLds, s, (const uint16_t*)logits, V, st);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::mass_kernel, dim3(smp::kSegs, batch), dim3(smp::kSegBins), 0, s, st,
                     temperature);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::select_kernel, dim3(batch), dim3(smp::kSegBins), 0, s, st,
                     temperature, top_p, uniform);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::count_kernel, dim3(smp::kFindParts, batch), dim3(smp::kFindThreads), 0,
                     s, (const uint16_t*)logits, V, st);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::locate_kernel, dim3(batch), dim3(smp::kLocThreads), 0, s,
                     (const uint16_t*)logits, V, (const smp::State*)st, out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // extern "C"
