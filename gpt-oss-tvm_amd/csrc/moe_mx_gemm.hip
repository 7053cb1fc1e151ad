// Grouped expert GEMM for many tokens per expert (prefill), on the same
// block-scaled instruction as the GEMV (v_mfma_scale_f32_16x16x128_f8f6f4):
// fp8 activation pieces (A) times MXFP4 weights as stored (B), fp32 out.
//
// Reference operators: mxfp4_moe_mlp1_prefill / mxfp4_moe_mlp2_prefill
// (model/mlp_optimized.py:214-460) with the fp32 semantics of
// model/mlp.py:387-395 (einsum + bias, interleaved clamped SwiGLU on mlp1).
//
// Tiles.  A work unit is one (expert, token tile, column tile): 192 A rows
// (192 / P tokens, P pieces each) against 192 weight rows over the whole K.
// Eight waves split it 4 x 2: each wave owns 48 A rows x 96 columns, i.e.
// 3 x 6 MFMA tiles of 16 x 16, and keeps their 18 accumulators for all of K.
//
// Staging.  The unit's scale bytes (A: 112 per row, B: G per column) are
// staged once.  Per 128-wide K chunk a stage holds the tile's A codes
// (192 x 128 bytes) and B codes (192 x 64).  Both come by direct
// global-to-LDS loads (no registers), 16 bytes per lane; three code stages
// form a ring, so while chunk c is multiplied the loads of chunks c + 1 and
// c + 2 are in flight.  A wave's loads complete in issue order, so "chunk c
// has landed" is vmcnt <= (its loads per chunk) on each wave plus a barrier.
// A and B code rows are stored with their 16-byte parts XOR-swizzled so that
// the MFMA operand reads of 16 lanes hit distinct LDS banks.
//
// Operand layout per K chunk c (lane l = 16 g + r), as in the GEMV:
//   A  row r: bytes 0..15 -> k = 16 g + 0..15, bytes 16..31 -> k = 64 + 16 g + 0..15
//   B  column r: MX block 4 c + g of that weight row (low nibble first)
//   scales: lane (r, g) gives the E8M0 of block 4 c + g of its row / column
//   D  column r, elements i = 0..3 -> A rows 4 g + i
// A token's P piece rows share one lane's four accumulator rows, so the
// pieces are summed in registers in the epilogue, as the GEMV does.
#include <type_traits>

#include "moe_common.h"

namespace moe {

constexpr int kGmRows = 192;                       // A rows per tile
constexpr int kGmCols = 192;                       // weight rows (output columns) per tile
constexpr int kGmWaves = 8;                        // 4 (A rows) x 2 (columns)
constexpr int kGmThreads = 64 * kGmWaves;
constexpr int kGmStages = 3;
constexpr int kGmAInst = kGmRows * 8 / 64;         // 24 A-code loads per chunk (3 per wave)
constexpr int kGmBInst = kGmCols * 4 / 64;         // 12 B-code loads per chunk
constexpr int kGmAo = 0;                           // in a stage: A codes, then B codes
constexpr int kGmBo = kGmRows * 128;
constexpr int kGmStage = kGmBo + kGmCols * 64;     // 36864 bytes
constexpr int kGmSclRow = 112;                     // scale bytes per piece row (4 runs of 28)
constexpr int kGmMaxG = 96;                        // K <= 3072
constexpr int kGmASc = kGmStages * kGmStage;       // A scales of the unit [rows][112]
constexpr int kGmBSc = kGmASc + kGmRows * kGmSclRow;  // B scales of the unit [cols][G]
constexpr int kGmBScBytes = kGmCols * kGmMaxG;     // 192 G, G <= 96, in whole 1 KB loads
constexpr int kGmBias = kGmBSc + kGmBScBytes;      // bias of the unit's columns (bf16)
constexpr int kGmFixedLds = kGmBias + 1024;        // 152064 bytes
constexpr int kGmCUs = 256;                        // MI355X
constexpr int kGmXcds = 8;                         // 8 XCDs of 32 CUs, one L2 each

// dynamic part: unit prefix and indptr, E + 1 ints each
// dynamic part: unit prefix and indptr, E + 1 ints each, then two buffers of
// a unit's sorted_pairs entries (kGmSpMax ints each)
constexpr int kGmSpMax = kGmRows / 2;
__host__ __device__ constexpr int gm_lds_bytes(int E) { return 2 * (E + 1) * 4 + 2 * kGmSpMax * 4; }
static_assert(kGmFixedLds + gm_lds_bytes(256) <= 160 * 1024, "LDS");


template <int S, int E, class F>
__device__ __forceinline__ void gm_static_for(F&& f) {
  if constexpr (S < E) {
    f(std::integral_constant<int, S>{});
    gm_static_for<S + 1, E>(f);
  }
}


// LDS reads of the staged operands, issued as inline asm: the compiler does
// not count them against the direct loads in flight (it would otherwise wait
// for all of those before any LDS read).  Their results pass through
// lgkm_wait, whose operand ties keep every use after the wait.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}
template <int OFF>
__device__ __forceinline__ u32x4 lds_b128(uint32_t a) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_u8(uint32_t a) {
  uint32_t v;
  asm volatile("ds_read_u8 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

// The value of lane l + 16 for lane groups g = 0..2 (x's next 16-lane row)
// and of lane l - 48 for g = 3 (y's row 0): one row down across the pair
// (x, y).  v_permlane16_swap(D, S) swaps D's odd rows with S's even rows
// (D' = [D0 S0 D2 S2], S' = [D1 S1 D3 S3]); v_permlane32_swap(D, S) swaps
// D's upper half with S's lower half (D' = [D0 D1 S0 S1], S' = [D2 D3 S2 S3]).
__device__ __forceinline__ float gm_row_down(float x, float y, int g) {
  const int xi = __float_as_int(x), yi = __float_as_int(y);
  const auto s16 = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);  // S' = [x1 x1 x3 x3]
  const auto s32 = __builtin_amdgcn_permlane32_swap(xi, yi, false, false);  // [x0 x1 y0 y1], [x2 x3 y2 y3]
  const auto a = __builtin_amdgcn_permlane16_swap(s32[0], s32[1], false, false);  // D' = [x0 x2 y0 y2]
  const auto c = __builtin_amdgcn_permlane16_swap(s32[1], s32[0], false, false);  // D' = [x2 x0 y2 y0]
  return __int_as_float(g == 1 ? (int)a[0] : g == 3 ? (int)c[0] : (int)s16[1]);
}

template <int P, int kEpi>
__global__ __launch_bounds__(kGmThreads) void moe_mx_gemm_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ qs, int Kp,
    const int* __restrict__ indptr, const int* __restrict__ sorted_pairs, int k_top,
    int arow_mode, int orow_mode, const uint8_t* __restrict__ blocks,
    const uint8_t* __restrict__ scales, const uint16_t* __restrict__ bias, int N, int G, int E,
    float alpha, float limit, float* __restrict__ out, int out_ld, int xcds,
    uint8_t* __restrict__ oqs) {
  __shared__ __align__(16) uint8_t ring[kGmFixedLds];
  extern __shared__ __align__(16) uint8_t lds[];  // unit prefix
  constexpr int TPT = kGmRows / P;  // tokens per tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, wn = wave >> 2;
  const int r = lane & 15, g = lane >> 4;
  const int NT = N / kGmCols;
  const int NC = Kp >> 7;
  // B-code loads per chunk: instruction k < 12 belongs to wave k % 8
  const bool two_b = wave < kGmBInst - kGmWaves;
  // Per-lane LDS read bases of each stage; the operand index goes into the
  // instructions' immediate offsets.  Lane (r, g): B column 96 wn + 16 b + r
  // (part g, swizzled by (column >> 1) & 3 = (r >> 1) & 3); A row
  // 48 wm + 16 f + r (parts g and g + 4, swizzled by row & 7 = r & 7).
  const uint32_t rbase = lds_addr(ring);
  uint32_t vb[kGmStages], va0[kGmStages], va1[kGmStages];
#pragma unroll
  for (int S = 0; S < kGmStages; ++S) {
    const uint32_t st = rbase + S * kGmStage;
    vb[S] = st + kGmBo + (96 * wn + r) * 64 + ((g ^ ((r >> 1) & 3)) << 4);
    va0[S] = st + kGmAo + (48 * wm + r) * 128 + ((g ^ (r & 7)) << 4);
    va1[S] = st + kGmAo + (48 * wm + r) * 128 + (((g + 4) ^ (r & 7)) << 4);
  }
  // scale bytes: A row 48 wm + 16 f + r, run g; B column 96 wn + 16 b + r
  const uint32_t vas = rbase + kGmASc + (48 * wm + r) * kGmSclRow + g * 28;
  const uint32_t vbs = rbase + kGmBSc + (96 * wn + r) * G;
  int* const pre = (int*)lds;
  int* const ipl = pre + (E + 1);  // indptr, read once
  // A unit's sorted_pairs entries (token tt at [tt]) in LDS, double-buffered:
  // each unit's epilogue loads the next unit's before any of its stores, so
  // no global load in the address chains or the stores waits behind stores
  // (vmcnt counts loads and stores together, in issue order).
  int* const spb = ipl + (E + 1);
  const bool need_sp = arow_mode != 2 || orow_mode == 0;
  int par = 0;
  bool first_unit = true;

  // Exclusive prefix of the unit counts: ceil(cnt_e / TPT) * NT.
  if (wave == 0) {
    int carry = 0;
    if (lane == 0) pre[0] = 0;
    for (int i = lane; i <= E; i += 64) ipl[i] = indptr[i];
    for (int b = 0; b < E; b += 64) {
      const int i = b + lane;
      int v = 0;
      if (i < E) v = (indptr[i + 1] - indptr[i] + TPT - 1) / TPT * NT;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, kWave);
        if (lane >= o) v += t;
      }
      if (i < E) pre[i + 1] = carry + v;
      carry += __shfl(v, 63, kWave);
    }
  }
  __syncthreads();
  const int total = pre[E];
  // Units go round-robin over the workgroups in XCD-major numbering: at each
  // step the workgroups of one XCD take consecutive units, the column tiles
  // of one token tile, so that tile's A rows are fetched into that XCD's L2
  // once and read from there by all of them.
  const int vwg = xcds > 1 ? (int)(blockIdx.x % xcds) * (int)(gridDim.x / xcds) +
                                 (int)(blockIdx.x / xcds)
                           : (int)blockIdx.x;
  auto expert_of = [&](int u) {  // largest e with pre[e] <= u
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= u) lo = mid; else hi = mid - 1;
    }
    return lo;
  };

  for (int u = vwg; u < total; u += gridDim.x) {
    // An opaque copy of the lane index for this unit's address arithmetic:
    // the compiler would otherwise hoist lane-dependent addresses out of the
    // unit loop and spill them, and reloading a spill waits for every load in
    // flight (vmcnt counts them in issue order), serialising the prologue.
    int lane_u = lane;
    asm volatile("" : "+v"(lane_u));
    const int e = expert_of(u);
    const int off = u - pre[e];
    const int mt = off / NT, nt = off - mt * NT;
    const int start = ipl[e];
    const int m0 = mt * TPT;
    const int ntok = min(TPT, ipl[e + 1] - start - m0);
    const int n0 = nt * kGmCols;
    int* const spu = spb + par * kGmSpMax;
    if (need_sp && first_unit) {
      if (tid < ntok) spu[tid] = sorted_pairs[start + m0 + tid];
      __syncthreads();  // (the first unit: nothing else in flight)
    }
    first_unit = false;
    auto src_row = [&](int tt) {  // activation row of token tt of this tile
      return arow_mode == 0 ? spu[tt] / k_top : arow_mode == 1 ? spu[tt] : start + m0 + tt;
    };
    // Rows past the tile's tokens load token 0's row: their MFMA rows are
    // computed and never stored (a D row depends on its A row only).
    auto piece_row = [&](int R) {  // packed-pieces row of tile A row R
      if constexpr (P == 3) asm volatile("" : "+v"(R));  // (not hoisted: see the epilogue)
      const int tt = R / P, p = R - tt * P;
      return (uint32_t)(src_row(tt < ntok ? tt : 0) * P + p);
    };

    // The unit's scales, 16 bytes per lane_u: A rows (7 loads of 16 per row;
    // loads past the last row repeat it), then the B columns' G bytes each
    // (192 G contiguous checkpoint bytes; the tail repeats the last 16).
    {
      constexpr int kAU = kGmRows * 7;                        // 1344 A-scale loads
      const int nbu = kGmCols * G / 16;                       // B-scale loads
      for (int i0 = 64 * wave; i0 < kAU; i0 += kGmThreads) {
        const int uu = min(i0 + lane_u, kAU - 1), R = uu / 7;
        __builtin_amdgcn_global_load_lds(
            (const void*)(qs + piece_row(R) * kGmSclRow + (uu - R * 7) * 16),
            (lds_ptr_t)(ring + kGmASc + i0 * 16), 16, 0, 0);
      }
      const uint8_t* bsrc = scales + ((size_t)e * N + n0) * G;
      for (int i0 = 64 * wave; i0 < nbu; i0 += kGmThreads)
        __builtin_amdgcn_global_load_lds((const void*)(bsrc + min(i0 + lane_u, nbu - 1) * 16),
                                         (lds_ptr_t)(ring + kGmBSc + i0 * 16), 16, 0, 0);
      // the columns' bias: 384 bytes, 24 loads of 16 (the rest repeat the last)
      if (wave == kGmWaves - 1)
        __builtin_amdgcn_global_load_lds(
            (const void*)((const uint8_t*)(bias + (size_t)e * N + n0) + min(lane_u, 23) * 16),
            (lds_ptr_t)(ring + kGmBias), 16, 0, 0);
    }

    // This wave's code loads of a chunk (lane_u l), 32-bit offsets from q and
    // blocks (the launcher checks the ranges):
    //  A 3: instruction 3 w + m, rows 8 (3 w + m) + l / 8, global part
    //       (l % 8) ^ (l / 8)
    //  B 1 or 2: instruction k = w (+ 8), columns 16 k + l / 4, global part
    //       (l % 4) ^ ((column >> 1) & 3)
    uint32_t ap[3], bp[2];
    int bpart[2];
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      const int R = 8 * (3 * wave + m) + (lane_u >> 3);
      ap[m] = piece_row(R) * (uint32_t)Kp + (((lane_u & 7) ^ (lane_u >> 3)) << 4);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int C = 16 * (wave + kGmWaves * m) + (lane_u >> 2);
      bp[m] = (uint32_t)(((size_t)e * N + n0 + min(C, kGmCols - 1)) * G * 16);
      bpart[m] = (lane_u & 3) ^ ((C >> 1) & 3);
    }
    auto issue_chunk = [&](int c, int S) {
      uint8_t* st = ring + S * kGmStage;
#pragma unroll
      for (int m = 0; m < 3; ++m)
        __builtin_amdgcn_global_load_lds((const void*)(q + ap[m] + c * 128),
                                         (lds_ptr_t)(st + kGmAo + (3 * wave + m) * 1024), 16, 0,
                                         0);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        if (m == 0 || two_b) {
          // past K a column re-reads block G - 1 (finite; its A codes are zero)
          const uint32_t blk = (uint32_t)min(4 * c + bpart[m], G - 1);
          __builtin_amdgcn_global_load_lds((const void*)(blocks + bp[m] + blk * 16),
                                           (lds_ptr_t)(st + kGmBo + (wave + kGmWaves * m) * 1024),
                                           16, 0, 0);
        }
      }
    };

    // Chunks 0..2 in flight; chunk 0's operands go to registers first.
    issue_chunk(0, 0);
    if (NC > 1) issue_chunk(1, 1);
    if (NC > 2) issue_chunk(2, 2);

    f32x4 acc[3][6];
#pragma unroll
    for (int f = 0; f < 3; ++f)
#pragma unroll
      for (int b = 0; b < 6; ++b) acc[f][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // A operand groups holding no token of the tile are skipped (uniform)
    int nf = 0;
#pragma unroll
    for (int f = 0; f < 3; ++f) nf += (48 * wm + 16 * f) / P < ntok ? 1 : 0;

    // Operands of one chunk in registers: six B groups (16 bytes + scale) and
    // three A groups (32 bytes + scale).
    struct Ops {
      u32x4 b[6];
      uint32_t bs[6];
      u32x4 a0[3], a1[3];
      uint32_t as[3];
    };
    auto read_b = [&](Ops& o, int c, auto sv) {
      constexpr int S = decltype(sv)::value;
      const uint32_t bsc = vbs + (uint32_t)min(4 * c + g, G - 1);
      gm_static_for<0, 6>([&](auto bv) {
        constexpr int b = decltype(bv)::value;
        o.b[b] = lds_b128<b * 1024>(vb[S]);
        o.bs[b] = lds_u8<0>(bsc + b * 16 * G);
      });
    };
    auto read_a = [&](Ops& o, int c, auto sv, auto fv) {
      constexpr int S = decltype(sv)::value, f = decltype(fv)::value;
      o.a0[f] = lds_b128<f * 2048>(va0[S]);
      o.a1[f] = lds_b128<f * 2048>(va1[S]);
      o.as[f] = lds_u8<f * 16 * kGmSclRow>(vas + c);
    };
    auto wait_ops = [&](Ops& o) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(o.b[0]), "+v"(o.b[1]), "+v"(o.b[2]), "+v"(o.b[3]), "+v"(o.b[4]),
                     "+v"(o.b[5]), "+v"(o.bs[0]), "+v"(o.bs[1]), "+v"(o.bs[2]), "+v"(o.bs[3]),
                     "+v"(o.bs[4]), "+v"(o.bs[5]), "+v"(o.a0[0]), "+v"(o.a0[1]), "+v"(o.a0[2]),
                     "+v"(o.a1[0]), "+v"(o.a1[1]), "+v"(o.a1[2]), "+v"(o.as[0]), "+v"(o.as[1]),
                     "+v"(o.as[2]));
    };
    auto mfma_group = [&](const Ops& o, auto fv) {
      constexpr int f = decltype(fv)::value;
      const i32x8 A = {(int)o.a0[f][0], (int)o.a0[f][1], (int)o.a0[f][2], (int)o.a0[f][3],
                       (int)o.a1[f][0], (int)o.a1[f][1], (int)o.a1[f][2], (int)o.a1[f][3]};
#pragma unroll
      for (int b = 0; b < 6; ++b) {
        const i32x8 B = {(int)o.b[b][0], (int)o.b[b][1], (int)o.b[b][2], (int)o.b[b][3],
                         0, 0, 0, 0};
        acc[f][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[f][b], 0, 4, 0,
                                                                     (int)o.as[f], 0,
                                                                     (int)o.bs[b]);
      }
    };

    // wait until at most `pending` later chunks' loads are outstanding (a
    // wave issues 4 or 5 loads per chunk; its loads complete in order)
    auto wait_chunks = [&](int pending) {
      if (pending >= 2) {
        if (two_b) wait_vmcnt<10>(); else wait_vmcnt<8>();
      } else if (pending == 1) {
        if (two_b) wait_vmcnt<5>(); else wait_vmcnt<4>();
      } else {
        wait_vmcnt<0>();
      }
    };
    Ops cur, nxt;
    // chunk 0 landed (and the unit's scales: issued before it)
    wait_chunks(min(NC - 1, 2));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_b(cur, 0, std::integral_constant<int, 0>{});
    gm_static_for<0, 3>([&](auto fv) { read_a(cur, 0, std::integral_constant<int, 0>{}, fv); });
    wait_ops(cur);

    // Step c: chunk c + 1 landed everywhere (its waves' vmcnt + barrier; the
    // barrier also certifies that every wave has read chunk c out of stage
    // c % 3), issue chunk c + 3 into that stage, then multiply chunk c from
    // registers while chunk c + 1's operands are read from LDS.  The barrier
    // carries no memory fence: a fence would wait for the loads in flight.
    // Issue order within the step: the first six MFMAs straight after the
    // barrier (their operands are in registers), then the B and first A
    // operand reads, six more MFMAs, then the chunk loads and the other A
    // reads, the last six MFMAs.  (Measured against the loads and reads
    // ahead of the MFMAs, and against one MFMA between each pair of memory
    // instructions: both are slower.)
    auto step = [&](int c, Ops& cu, Ops& nx, auto sv) {
      constexpr int S = decltype(sv)::value;           // stage of chunk c
      constexpr int S1 = (S + 1) % kGmStages;          // stage of chunk c + 1
      const bool more = c + 1 < NC;
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using SS1 = std::integral_constant<int, S1>;
      if (more) {
        wait_chunks(c + 2 < NC ? 1 : 0);
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      if (0 < nf) mfma_group(cu, I0{});
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
        read_b(nx, c + 1, SS1{});
        read_a(nx, c + 1, SS1{}, I0{});
      }
      __builtin_amdgcn_sched_barrier(0);
      if (1 < nf) mfma_group(cu, I1{});
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
        if (c + 3 < NC) issue_chunk(c + 3, S);
        read_a(nx, c + 1, SS1{}, I1{});
        read_a(nx, c + 1, SS1{}, I2{});
      }
      __builtin_amdgcn_sched_barrier(0);
      if (2 < nf) mfma_group(cu, I2{});
      __builtin_amdgcn_sched_barrier(0);
      if (more) wait_ops(nx);
    };
    // Register sets alternate with the chunk parity and stages with c % 3,
    // so the loop is unrolled by six.
    for (int c = 0; c < NC; c += 6) {
      step(c, cur, nxt, std::integral_constant<int, 0>{});
      if (c + 1 < NC) step(c + 1, nxt, cur, std::integral_constant<int, 1>{});
      if (c + 2 < NC) step(c + 2, cur, nxt, std::integral_constant<int, 2>{});
      if (c + 3 < NC) step(c + 3, nxt, cur, std::integral_constant<int, 0>{});
      if (c + 4 < NC) step(c + 4, cur, nxt, std::integral_constant<int, 1>{});
      if (c + 5 < NC) step(c + 5, nxt, cur, std::integral_constant<int, 2>{});
    }
    // The MFMAs combine all 64 lanes; the LDS writes below are per-lane.  The
    // empty asm keeps the compiler from sinking the chains into them.
#pragma unroll
    for (int f = 0; f < 3; ++f)
#pragma unroll
      for (int b = 0; b < 6; ++b) asm volatile("" : "+v"(acc[f][b]));
    // every wave is done with the stages: the output tile reuses them
    __syncthreads();
    // the next unit's sorted_pairs entries, loaded before this unit's stores
    int spn = 0;
    bool spn_lane = false;
    if (need_sp && u + (int)gridDim.x < total) {
      const int un = u + (int)gridDim.x;
      const int e2 = expert_of(un);
      const int st2 = ipl[e2], m02 = (un - pre[e2]) / NT * TPT;
      if (tid < min(TPT, ipl[e2 + 1] - st2 - m02)) {
        spn = sorted_pairs[st2 + m02 + tid];
        spn_lane = true;
      }
    }

    // Epilogue: bias (+ SwiGLU) into an LDS tile of the unit's outputs, then
    // row-contiguous 16-byte stores.  mlp1 with SwiGLU: [TPT][96] act columns
    // n0 / 2 ..; otherwise [TPT][192] columns n0 ...
    constexpr int TW = kEpi >= 1 ? kGmCols / 2 : kGmCols;
    constexpr int TWp = TW + 4;
    float* const tile = (float*)ring;
    static_assert(TPT * TWp * 4 <= kGmStages * kGmStage, "output tile");
    const uint16_t* const bias_l = (const uint16_t*)(ring + kGmBias);
    if constexpr (P == 3) {
      // The wave's 48 rows 48 wm + 4 q + i (q = 4 f + g, i < 4) hold 16
      // tokens, row 3 t + p piece p of token t.  Every third quad repeats:
      // q = 3k holds token 4k and piece 0 of token 4k + 1, q = 3k + 1 pieces
      // 1, 2 of token 4k + 1 and 0, 1 of 4k + 2, q = 3k + 2 piece 2 of token
      // 4k + 2 and token 4k + 3.  The quad holding a token's piece 0 sums it;
      // the share of the next quad (q + 1: lane + 16, or for g = 3 the next
      // f's lane group 0) comes by shuffle.  Sums run smallest piece first,
      // ((p2 + p1) + p0) + bias, as for the other piece counts.
      // Branch-free (q % 3 varies with the lane group): operands by select,
      // and the second token's value of a q % 3 = 0 quad is written by every
      // lane, the others' into the spare row TPT, which is never read.  The
      // exchange is by lane-row swaps (register moves, no LDS round trip).
      static_assert((TPT + 1) * TWp * 4 <= kGmStages * kGmStage, "spare row");
#pragma unroll
      for (int b = 0; b < 6; ++b) {
        const int cl = 96 * wn + 16 * b + r;
        const float bn = bf2f(bias_l[cl]);
        float send[3];
#pragma unroll
        for (int f = 0; f < 3; ++f)
          send[f] = (4 * f + g) % 3 == 1 ? acc[f][b][1] + acc[f][b][0] : acc[f][b][0];
#pragma unroll
        for (int f = 0; f < 3; ++f) {
          const f32x4 a = acc[f][b];
          const float rv = gm_row_down(send[f], f < 2 ? send[f < 2 ? f + 1 : f] : 0.0f, g);
          const int q = 4 * f + g, qm = q % 3;
          const int tb = 16 * wm + (4 * q) / 3;
          const float v1 = qm == 0 ? a[2] : qm == 1 ? rv : a[3];
          const float v2 = qm == 0 ? a[1] : qm == 1 ? a[3] : a[2];
          const float v3 = qm == 0 ? a[0] : qm == 1 ? a[2] : a[1];
          tile[(qm == 0 ? tb : tb + 1) * TWp + cl] = ((v1 + v2) + v3) + bn;
          tile[(qm == 0 ? tb + 1 : TPT) * TWp + cl] = (rv + a[3]) + bn;
        }
      }
    } else {
#pragma unroll
    for (int b = 0; b < 6; ++b) {
      const int cl = 96 * wn + 16 * b + r;  // column within the tile
      const float bn = bf2f(bias_l[cl]);
#pragma unroll
      for (int f = 0; f < 3; ++f) {
        const f32x4 a = acc[f][b];
        if constexpr (P == 4) {
          const int tt = 12 * wm + 4 * f + g;
          tile[tt * TWp + cl] = (((a[3] + a[2]) + a[1]) + a[0]) + bn;
        } else {
          const float y0 = (a[1] + a[0]) + bn;
          const float y1 = (a[3] + a[2]) + bn;
          const int tt0 = 24 * wm + 8 * f + 2 * g;
          if constexpr (kEpi >= 1) {
            // columns 2 j (glu) and 2 j + 1 (linear) sit in lanes r and r ^ 1;
            // the even lane takes token tt0, the odd lane token tt0 + 1
            const bool odd = (r & 1) != 0;
            const float send = odd ? y0 : y1;  // what the partner needs
            const float recv = lane_xor1(send);
            const float glu = odd ? recv : y0;
            const float lin = odd ? y1 : recv;
            const float xg = fminf(glu, limit);
            const float xl = fminf(fmaxf(lin, -limit), limit);
            const float z = __fmul_rn(alpha, xg);
            // sigmoid from the hardware exp2 and reciprocal (v_exp_f32 of
            // -z log2(e), v_rcp_f32: a few ulp of the correctly rounded value;
            // the epilogue is VALU-bound and the library expf and division
            // cost about 25 instructions per element)
            const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-z));
            tile[(tt0 + (odd ? 1 : 0)) * TWp + (cl >> 1)] =
                __fmul_rn(__fmul_rn(xg, sig), __fadd_rn(xl, 1.0f));
          } else {
            tile[tt0 * TWp + cl] = y0;
            tile[(tt0 + 1) * TWp + cl] = y1;
          }
        }
      }
    }
    }
    if (spn_lane) spb[(par ^ 1) * kGmSpMax + tid] = spn;
    __syncthreads();
    if constexpr (kEpi == 2) {
      // SwiGLU output straight into three fp8 pieces (the mlp2 operand), the
      // encoding of moe_pieces_kernel: the tile holds act columns n0 / 2 ..
      // n0 / 2 + 95 of its tokens, three whole 32-element blocks per row;
      // four threads per block (8 values each) share its maximum by lane
      // exchange.  out is the packed q of the act rows (length N / 2, padded
      // to 128), oqs their scale runs.  The trip count is uniform so every
      // quad exchanges with all four lanes; extra tasks store nothing.
      constexpr int PO = 3;
      const int Ka = N / 2, NCa = (Ka + 127) / 128, Kpa = NCa * 128;
      uint8_t* const oq = (uint8_t*)out;
      const int cbase = n0 / 2;
      const int tasks = ntok * 12;
      for (int i0 = 0; i0 < tasks; i0 += kGmThreads) {
        const int id = i0 + tid;
        const bool valid = id < tasks;
        const int idc = valid ? id : (id & 3);
        const int quarter = idc & 3, rb = idc >> 2;
        const int tt = rb / 3, bk = rb - tt * 3;
        const f32x4 v0 = *(const f32x4*)(tile + tt * TWp + bk * 32 + quarter * 8);
        const f32x4 v1 = *(const f32x4*)(tile + tt * TWp + bk * 32 + quarter * 8 + 4);
        float rr[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        const int orow = orow_mode == 0 ? spu[tt] : start + m0 + tt;
        const int blk = cbase / 32 + bk, ch = blk >> 2, gg = blk & 3;
#pragma unroll
        for (int p = 0; p < PO; ++p) {
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
          const size_t prow = (size_t)orow * PO + p;
          if (valid) {
            *(uint2*)(oq + prow * Kpa + cbase + bk * 32 + quarter * 8) = make_uint2(lo, hi);
            if (quarter == 0) oqs[prow * kGmSclRow + gg * 28 + ch] = (uint8_t)sc;
          }
        }
      }
      // The last column tile also writes the rows' tails: zero codes past
      // Ka, zero scales for the blocks past Ka and for the runs' unused
      // chunks [NCa, 28).
      if (nt == NT - 1) {
        for (int rp = tid; rp < ntok * PO; rp += kGmThreads) {
          const int tt = rp / PO, p = rp - tt * PO;
          const int orow = orow_mode == 0 ? spu[tt] : start + m0 + tt;
          const size_t prow = (size_t)orow * PO + p;
          for (int c = Ka; c < Kpa; c += 16) *(u32x4*)(oq + prow * Kpa + c) = u32x4{0u, 0u, 0u, 0u};
          uint8_t* const run = oqs + prow * kGmSclRow;
          for (int b = Ka / 32; b < 4 * NCa; ++b) run[(b & 3) * 28 + (b >> 2)] = 0;
          for (int g4 = 0; g4 < 4; ++g4)
            for (int z = NCa; z < 28; ++z) run[g4 * 28 + z] = 0;
        }
      }
    } else {
      constexpr int U = TW / 4;  // 16-byte units per row
      const int cbase = kEpi == 1 ? n0 / 2 : n0;
      for (int uu = tid; uu < ntok * U; uu += kGmThreads) {
        const int row = uu / U, cu4 = uu - row * U;
        const int j = start + m0 + row;
        const int orow = orow_mode == 0 ? spu[row] : j;
        *(f32x4*)(out + (size_t)orow * out_ld + cbase + 4 * cu4) =
            *(const f32x4*)(tile + row * TWp + 4 * cu4);
      }
    }
    // The next unit's loads may not overwrite the tile still being read:
    // a plain barrier (the tile's LDS reads have been consumed by the stores;
    // the stores themselves need not complete).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    par ^= 1;
  }
}

template <int P, int kEpi>
int launch_gm(dim3 grid, size_t lds, hipStream_t stream, const uint8_t* q, const uint8_t* qs,
              int Kp, const int* indptr, const int* sp, int k_top, int arow, int orow,
              const uint8_t* blocks, const uint8_t* scales, const uint16_t* bias, int N, int G,
              int E, float alpha, float limit, float* out, int out_ld, int xcds, uint8_t* oqs) {
  static const bool lds_ok = [] {  // more than 64 KB of dynamic LDS, once per kernel
    return hipFuncSetAttribute((const void*)moe_mx_gemm_kernel<P, kEpi>,
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               gm_lds_bytes(256)) == hipSuccess;
  }();
  if (!lds_ok) return kErrLaunch;
  hipLaunchKernelGGL((moe_mx_gemm_kernel<P, kEpi>), grid, dim3(kGmThreads), lds, stream, q, qs,
                     Kp, indptr, sp, k_top, arow, orow, blocks, scales, bias, N, G, E, alpha,
                     limit, out, out_ld, xcds, oqs);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace moe

extern "C" {

size_t moe_pieces_q_bytes(int64_t rows, int64_t K, int pieces);

// Same contract as moe_launch_mx_gemv (packed pieces, grouping arrays,
// checkpoint weights); requires N % 192 == 0 and K <= 3072.
int moe_launch_mx_gemm(const void* packed, int rows, int pieces, const void* indptr,
                       const void* sorted_pairs, int k_top, int arow_mode, int orow_mode,
                       const void* blocks, const void* scales, const void* bias, int E, int N,
                       int K, int rows_active, int swiglu, float alpha, float limit, void* out,
                       int out_ld, void* out_qs, hipStream_t stream) {
  if (rows_active <= 0) return moe::kOk;
  if (N % moe::kGmCols || K % 32 || K > 32 * moe::kGmMaxG || E > 256)
    return moe::kErrUnsupported;
  // 32-bit offsets into the pieces and the weights
  if ((int64_t)rows * pieces * ((K + 127) / 128 * 128) >= ((int64_t)1 << 31) ||
      (int64_t)E * N * (K / 32) * 16 >= ((int64_t)1 << 31))
    return moe::kErrUnsupported;
  const int NC = (K + 127) / 128, Kp = NC * 128, G = K / 32;
  const uint8_t* q = (const uint8_t*)packed;
  const uint8_t* qs = q + moe_pieces_q_bytes(rows, K, pieces);
  const int tpt = moe::kGmRows / pieces;
  const int64_t units_max = (int64_t)(N / moe::kGmCols) *
                            ((int64_t)max(1, min(E, rows_active)) + rows_active / tpt);
  if (units_max >= ((int64_t)1 << 31)) return moe::kErrUnsupported;
  const int nwg = (int)(units_max < moe::kGmCUs ? units_max : moe::kGmCUs);
  const int xcds = nwg % moe::kGmXcds == 0 ? moe::kGmXcds : 1;
  const size_t lds = moe::gm_lds_bytes(E);
  const int* ip = (const int*)indptr;
  const int* sp = (const int*)sorted_pairs;
  const uint8_t* b = (const uint8_t*)blocks;
  const uint8_t* s = (const uint8_t*)scales;
  const uint16_t* bi = (const uint16_t*)bias;
  float* o = (float*)out;
  const dim3 grid(nwg);
  if (pieces == 2 && swiglu == 2) {  // SwiGLU straight into 3 act pieces (out = their q)
    if (!out_qs || ((uintptr_t)out & 15u)) return moe::kErrUnsupported;
    return moe::launch_gm<2, 2>(grid, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode, orow_mode,
                                b, s, bi, N, G, E, alpha, limit, o, out_ld, xcds,
                                (uint8_t*)out_qs);
  }
  if (pieces == 2 && swiglu)
    return moe::launch_gm<2, 1>(grid, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode, orow_mode,
                                b, s, bi, N, G, E, alpha, limit, o, out_ld, xcds, nullptr);
  if (pieces == 2)
    return moe::launch_gm<2, 0>(grid, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode, orow_mode,
                                b, s, bi, N, G, E, alpha, limit, o, out_ld, xcds, nullptr);
  if (pieces == 3 && !swiglu)
    return moe::launch_gm<3, 0>(grid, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode, orow_mode,
                                b, s, bi, N, G, E, alpha, limit, o, out_ld, xcds, nullptr);
  if (pieces == 4 && !swiglu)
    return moe::launch_gm<4, 0>(grid, lds, stream, q, qs, Kp, ip, sp, k_top, arow_mode, orow_mode,
                                b, s, bi, N, G, E, alpha, limit, o, out_ld, xcds, nullptr);
  return moe::kErrUnsupported;
}

}  // extern "C"
