// Top-p sampling of the next token on the GPU (engine.py:165-167: TVM's
// vm.builtin.sample_top_p_from_logits, called with temperature 0.7, top_p 0.9
// and a fixed uniform sample 0.5 at engine.py:40).
//
// The algorithm sorts the logits in descending order, takes e = exp((l - max)
// / T), and returns the first element whose cumulative probability over the
// top-p mass exceeds the uniform sample, where the top-p mass is the sum up to
// and including the element at which the running sum reaches top_p.
//
// The model's logits are bf16 values (the unembedding's bf16 output cast to
// fp32, model/transformer.py:95-100), so a sequence has at most 65536 distinct
// logit values.  Instead of a sort:
//   1. count the elements of each value in a 65536-bin histogram (integer
//      atomics: deterministic) and take the maximum;
//   2. one workgroup walks the bins in descending value order: mass of a bin =
//      count x exp((v - max) / T); the two crossings (top_p, then u times the
//      top-p mass) are found at element granularity inside their bins, in
//      fp64; the result is a value v* and a rank j* among the elements of that
//      value (equal logits are taken in index order);
//   3. the j*-th element of value v* in index order: matches counted per
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
};

// 1. histogram and maximum.  Grid (ceil(V / 2048), batch), 256 threads x 8.
__global__ __launch_bounds__(256) void hist_kernel(const uint16_t* __restrict__ logits, int V,
                                                   State* __restrict__ st) {
  const int b = blockIdx.y;
  const uint16_t* l = logits + (size_t)b * V;
  State& s = st[b];
  const int i0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  uint32_t mk = 0;
  if (i0 + 8 <= V && (V & 7) == 0) {
    const u32x4 v = *(const u32x4*)(l + i0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k0 = key16(v[j] & 0xFFFFu), k1 = key16(v[j] >> 16);
      atomicAdd(&s.counts[k0], 1u);
      atomicAdd(&s.counts[k1], 1u);
      mk = max(mk, max(k0, k1));
    }
  } else {
    for (int i = i0; i < min(i0 + 8, V); ++i) {
      const uint32_t k = key16(l[i]);
      atomicAdd(&s.counts[k], 1u);
      mk = max(mk, k);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mk = max(mk, (uint32_t)__shfl_xor((int)mk, off, 64));
  if ((threadIdx.x & 63) == 0 && mk) atomicMax(&s.max_key, mk);
}

// 2. the two crossings.  One 1024-thread workgroup per sequence; thread t owns
// the 64 bins of keys [65535 - 64 t - 63, 65535 - 64 t] (descending values).
constexpr int kSelThreads = 1024;
constexpr int kPerThread = kBins / kSelThreads;

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
    for (int i = 0; i < kSelThreads / 64; ++i) {
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

__global__ __launch_bounds__(kSelThreads) void select_kernel(State* __restrict__ st,
                                                             float temperature, float top_p,
                                                             float uniform) {
  __shared__ double tmp[kSelThreads / 64];
  __shared__ double tot_s, crossing_s;
  __shared__ int found, owner1, owner2;
  State& s = st[blockIdx.x];
  const int t = threadIdx.x;
  const uint32_t mk = s.max_key;
  const float m = value_of(mk);
  const int top_bin = 65535 - kPerThread * t;  // this thread's bins: top_bin down to top_bin - 63
  if (t == 0) {
    found = 0;
    owner1 = owner2 = kSelThreads;
  }
  if (temperature < 1e-6f) {
    // argmax: the first element of the largest value
    if (t == 0) {
      s.pick_key = mk;
      s.pick_rank = 1;
    }
  } else {
    const float scale = 1.0f / temperature;
    double mass = 0.0;
    for (int i = 0; i < kPerThread; ++i) {
      const int k = top_bin - i;
      const uint32_t c = s.counts[k];
      if (c) mass += (double)c * weight(value_of(k), m, scale);
    }
    const double before = block_exclusive_scan(mass, tmp, &tot_s);
    const double total = tot_s;
    // crossing 1: the element at which the running sum reaches top_p; the
    // top-p mass runs up to and including it
    const double tp = (double)top_p * total;
    // the first segment holding a crossing does the element-level search
    // (rounding of the scan could let two neighbours both claim it)
    if (before < tp && before + mass >= tp) atomicMin(&owner1, t);
    __syncthreads();
    if (t == owner1) {
      double run = before;
      int i = 0;
      for (; i < kPerThread; ++i) {
        const int k = top_bin - i;
        const uint32_t c = s.counts[k];
        if (!c) continue;
        const double p = weight(value_of(k), m, scale);
        if (run + c * p >= tp) {
          const double j = ceil((tp - run) / p);          // elements with sum before < tp
          run += fmin(fmax(j, 1.0), (double)c) * p;
          break;
        }
        run += c * p;
      }
      crossing_s = run;  // (the segment's end if rounding put the crossing past it)
      found = 1;
    }
    __syncthreads();
    if (t == 0 && !found) crossing_s = total;  // top_p >= 1: everything
    __syncthreads();
    // crossing 2: the first element whose cumulative mass exceeds u x top-p mass
    const double x = (double)uniform * crossing_s;
    if (t == 0) found = 0;
    if (before <= x && before + mass > x) atomicMin(&owner2, t);
    __syncthreads();
    if (t == owner2) {
      double run = before;
      int last = -1;
      for (int i = 0; i < kPerThread; ++i) {
        const int k = top_bin - i;
        const uint32_t c = s.counts[k];
        if (!c) continue;
        last = k;
        const double p = weight(value_of(k), m, scale);
        if (run + c * p > x) {
          const double j = floor((x - run) / p) + 1.0;
          s.pick_key = (uint32_t)k;
          s.pick_rank = (uint32_t)fmin(fmax(j, 1.0), (double)c);
          last = -2;
          break;
        }
        run += c * p;
      }
      if (last >= 0) {  // rounding put the crossing past the segment: its last element
        s.pick_key = (uint32_t)last;
        s.pick_rank = s.counts[last];
      }
      found = 1;
    }
    __syncthreads();
    if (t == 0 && !found) {  // past the top-p mass: the first element of the largest value
      s.pick_key = mk;
      s.pick_rank = 1;
    }
  }
  __syncthreads();
  // leave the histogram zeroed for the next call
  for (int i = t; i < kBins; i += kSelThreads) s.counts[i] = 0u;
  if (t == 0) s.max_key = 0u;
}

// 3. the pick_rank-th element of value pick_key, in index order, in two
// launches: count_kernel counts the matches of each of kFindParts contiguous
// ranges (16-byte loads), locate_kernel finds the range holding the wanted
// rank and the element inside it (a block-wide prefix over that range).
constexpr int kFindParts = 64;
constexpr int kFindThreads = 256;

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

__global__ __launch_bounds__(kFindThreads) void locate_kernel(const uint16_t* __restrict__ logits,
                                                              int V, const State* __restrict__ st,
                                                              int* __restrict__ out) {
  __shared__ int base_s, part_s;
  __shared__ int wsum[kFindThreads / 64];
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
  // chunks of kFindThreads elements in index order; a running count across them
  int before_chunk = base_s;
  for (int c0 = i0; c0 < i1; c0 += kFindThreads) {
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
    int pre = 0;
    for (int k = 0; k < w; ++k) pre += wsum[k];
    const int total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
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
  hipLaunchKernelGGL(smp::hist_kernel, dim3((V + 2047) / 2048, batch), dim3(256), 0, s,
                     (const uint16_t*)logits, V, st);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::select_kernel, dim3(batch), dim3(smp::kSelThreads), 0, s, st,
                     temperature, top_p, uniform);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::count_kernel, dim3(smp::kFindParts, batch), dim3(smp::kFindThreads), 0,
                     s, (const uint16_t*)logits, V, st);
  if (hipGetLastError() != hipSuccess) return -6;
  hipLaunchKernelGGL(smp::locate_kernel, dim3(batch), dim3(smp::kFindThreads), 0, s,
                     (const uint16_t*)logits, V, (const smp::State*)st, out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // extern "C"
