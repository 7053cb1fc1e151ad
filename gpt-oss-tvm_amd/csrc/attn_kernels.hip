// gpt-oss attention block kernels (gfx950): RMSNorm, QKV bias + YaRN RoPE +
// paged KV append, decode attention (split over pages, merged with the sink
// scaling), prefill / extend attention on bf16 MFMA, bias + residual, and the
// embedding gather.
//
// Reference: model/attention.py:182-256 (AttentionBlock.forward), the masks of
// tvm_fix.patch:36-47, mlc-llm's PagedKVCache page layout
// [pages, 2 (k, v), kv_heads, page_size, head_dim] (model/transformer.py:
// 153-175 creates it with page_size 16, engine.py:97-107).
//
// Shapes fixed by gpt-oss: head_dim 64, 64 query heads, 8 key/value heads
// (GQA groups of 8), pages of 16 tokens.  The host checks them.
#include "moe_common.h"

namespace attn {

using moe::bf16x8;
using moe::bf2f;
using moe::f2bf;
using moe::f32x4;
using moe::kWave;
using moe::load_dev;
using moe::store_dev;
using moe::u32x4;

constexpr int kD = 64;          // head_dim
constexpr int kHq = 64;         // query heads
constexpr int kHkv = 8;         // key/value heads
constexpr int kGroup = kHq / kHkv;
constexpr int kPage = 16;       // tokens per page
constexpr int kQkvHeads = kHq + 2 * kHkv;
// bytes of one (page, k or v, head) block: 16 tokens x 64 dims x bf16
constexpr int kHeadBlock = kPage * kD * 2;
constexpr int kPageBytes = 2 * kHkv * kHeadBlock;  // 32 KB per page per layer

__device__ __forceinline__ const uint16_t* kv_row(const uint8_t* cache, int page, int kv, int hk,
                                                  int slot) {
  return (const uint16_t*)(cache + (size_t)page * kPageBytes + (size_t)(kv * kHkv + hk) * kHeadBlock +
                           slot * (kD * 2));
}

// A sequence's page list: the page holding position pos.  The list index is
// clamped to the sequence's pages and the page id to the pool, so a page table
// that does not cover kv_len reads wrong keys instead of foreign memory (the
// host sizes the tables; this only keeps a bad table from faulting).
struct PageList {
  const int* ids;
  int count, pool;
  // a table entry clamped into the pool (callers that read entries ahead
  // clamp them at use)
  __device__ __forceinline__ int clamp(int id) const { return min(max(id, 0), pool - 1); }
  __device__ __forceinline__ int page_of(int pos) const {
    return clamp(ids[max(min(pos / kPage, count - 1), 0)]);
  }
};

// ---------------------------------------------------------------------------
// RMSNorm (attention.py:80, nn.RMSNorm): sum of squares of the bf16 inputs in
// fp64 (exact for inputs spanning less than 2^37), r = fp32(1/sqrt(ss/H +
// eps)) in fp64, t = bf16(fp32(x r) w).  One 256-thread workgroup per token.
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* __restrict__ x, int H,
                                                       const uint16_t* __restrict__ w, float eps,
                                                       uint16_t* __restrict__ out) {
  __shared__ double part[4];
  const int tok = blockIdx.x;
  const uint16_t* xr = x + (size_t)tok * H;
  double ss = 0.0;
  for (int i = threadIdx.x; i < H; i += 256) {
    const double v = (double)bf2f(xr[i]);
    ss += v * v;
  }
  ss = moe::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const double tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = (float)(1.0 / sqrt(tot / (double)H + (double)eps));
  for (int i = threadIdx.x; i < H; i += 256) {
    const float xv = __fmul_rn(bf2f(xr[i]), r);
    out[(size_t)tok * H + i] = f2bf(__fmul_rn(xv, bf2f(w[i])));
  }
}

// ---------------------------------------------------------------------------
// QKV epilogue: bias (a second bf16 rounding after the matmul's, nn.Linear),
// YaRN RoPE of q and k (attention.py:126-165), the new k and v written to
// their cache slots (append_mha_kv), q written [token][head][dim].
// cos/sin of fp32(position) * inv_freq are evaluated in fp64, rounded to fp32
// and then to bf16 (the rope's .astype(dtype)), then scaled by the fp32
// concentration; the rotation rounds each product and the difference / sum
// separately (no contraction).  One thread per rotation pair (d, d + 32):
// 256 threads = 8 heads of one token; grid (10, n).
__global__ __launch_bounds__(256) void qkv_rope_append_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ bias,
    const int* __restrict__ positions, const int* __restrict__ slots,
    const float* __restrict__ inv_freq, float conc, uint8_t* __restrict__ cache, int num_pages,
    uint16_t* __restrict__ q_out) {
#pragma clang fp contract(off)
  const int tok = blockIdx.y;
  const int head = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int d = threadIdx.x & 31;
  const size_t base = (size_t)tok * (kQkvHeads * kD) + head * kD;
  float lo = bf2f(f2bf(bf2f(qkv[base + d]) + bf2f(bias[head * kD + d])));
  float hi = bf2f(f2bf(bf2f(qkv[base + d + 32]) + bf2f(bias[head * kD + d + 32])));
  const int slot = slots[tok];
  if (head < kHq + kHkv) {
    const float freq = (float)positions[tok] * inv_freq[d];
    const double fd = (double)freq;
    const float c = bf2f(f2bf((float)cos(fd))) * conc;
    const float s = bf2f(f2bf((float)sin(fd))) * conc;
    const float nlo = lo * c - hi * s;
    const float nhi = lo * s + hi * c;
    lo = nlo;
    hi = nhi;
  }
  const uint16_t blo = f2bf(lo), bhi = f2bf(hi);
  if (head < kHq) {
    uint16_t* qo = q_out + ((size_t)tok * kHq + head) * kD;
    qo[d] = blo;
    qo[d + 32] = bhi;
  } else if (slot >= 0 && slot < num_pages * kPage) {  // other slots are not written
    const int kv = head < kHq + kHkv ? 0 : 1;
    const int hk = head - kHq - kv * kHkv;
    uint16_t* row = (uint16_t*)kv_row(cache, slot / kPage, kv, hk, slot % kPage);
    row[d] = blo;
    row[d + 32] = bhi;
  }
}

// ---------------------------------------------------------------------------
// Decode attention, phase 1: workgroup (split s, kv head hk, sequence b)
// takes keys [lo + S s, lo + S (s + 1)) of the sequence's attended range
// [lo, kv_len), S = 128 cps (cps chunks of 128 keys), for the 8 query heads of
// hk, and writes the partial softmax state of each head: m (max score), l (sum
// of exp(score - m)) and o[64] = sum exp(score - m) v.  The split's page ids
// are read once; each chunk's K rows and V (transposed) are staged in LDS
// from registers loaded while the previous chunk's products ran (256 threads
// x 8 16-byte loads, all in flight), with an online softmax across chunks.
// Both products run on v_mfma_f32_16x16x32_bf16, with the lane facts the
// prefill kernel below relies on (operand row / column = lane % 16; result
// element i of lane l = row 4 (l / 16) + i, column l % 16; A and B pair their
// operand slots by position): wave w takes the keys at positions 32 w ..
// 32 w + 31 of the chunk's V^T tile (dec_key_at: each 64-key half holds keys
// i and i + 32 side by side),
//  * S^T = K Q^T (A = 16 keys x 32 dims, B = 32 dims x 16 "queries": the 8
//    heads, repeated): A row r of tile kk is the key at position 32 w + 8 (r /
//    4) + 4 kk + r % 4, so lane l holds S[head l % 16][the keys at positions
//    32 w + 8 (l / 16) + 4 kk + i] for kk = 0, 1; scores in fp32 (times
//    sm_scale), the chunk's maximum per head through LDS;
//  * O^T = V^T P^T over the wave's 32 keys (P as two bf16 pieces, about 16
//    bits, as in the prefill kernel): P's slot 4 kk + i of lane l carries
//    that score, V^T's slot j of lane l position 32 w + 8 (l / 16) + j, the
//    same key; at the end the four waves' partial o are summed in wave order.
constexpr int kDecChunk = 128;
// the key of a chunk at V^T position p: each 64-key half interleaved,
// position 2i key i, 2i + 1 key i + 32
__device__ __forceinline__ int dec_key_at(int p) {
  const int q = p & 63;
  return (p & ~63) + ((q & 1) ? 32 + (q >> 1) : (q >> 1));
}
constexpr int kDecMaxCps = 8;
constexpr int kDecKRow = kD + 8;         // padded K row (bf16)
constexpr int kDecVRow = kDecChunk + 8;  // padded V^T row (bf16)

// Sink scaling of attention.py:235-245: lse (natural log) -> s =
// bf16(sigmoid(lse - sink)), out = bf16(bf16(o) * s).
__device__ __forceinline__ float sink_factor(float lse, uint16_t sink) {
  const float z = lse - bf2f(sink);
  return bf2f(f2bf((float)(1.0 / (1.0 + exp(-(double)z)))));
}

__device__ void decode_merge_group(const float* part_o, const float* part_ml, int splits,
                                   int used, bool bad, int b, int hk, const uint16_t* sinks,
                                   uint16_t* out);

__device__ __forceinline__ f32x4 dec_mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void decode_partial_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ cache,
    const int* __restrict__ page_indptr, const int* __restrict__ page_indices, int num_pages,
    const int* __restrict__ kv_len, int window, float sm_scale, int splits, int cps,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ arrive,
    const uint16_t* __restrict__ sinks, uint16_t* __restrict__ out) {
  // K rows [key][dim]; after the last chunk, the waves' partial o [wave][head][dim]
  __shared__ __align__(16) uint16_t ks[kDecChunk * kDecKRow];
  __shared__ __align__(16) uint16_t vt[kD * kDecVRow];  // V^T [dim][key]
  __shared__ float red_m[4][16], red_l[4][16], hm[kGroup];
  __shared__ int pid[kDecChunk * kDecMaxCps / kPage + 1];
  const int s = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x;
  const int wave = t >> 6, lane = t & 63, r = lane & 15, g = lane >> 4;
  const int L = kv_len[b];
  const int lo = window > 0 ? max(0, L - window) : 0;
  const int span = L - lo;
  // keys per split: cps chunks, except that a span of at most two chunks is
  // one split (its chunks in sequence cost less than publishing and merging
  // partials); covered = the keys the caller's bound gives the splits
  const int skeys =
      kDecChunk * (span <= 2 * kDecChunk ? max(cps, (span + kDecChunk - 1) / kDecChunk) : cps);
  const int covered = splits * kDecChunk * cps;
  const int k0 = lo + s * skeys;
  const int nks = max(0, min(skeys, L - k0));
  const size_t pidx = ((size_t)b * kHq + hk * kGroup) * splits + s;  // head h: + h * splits
  // the splits holding keys: the first ceil(span / skeys) (at most splits)
  const int used = min((span + skeys - 1) / skeys, splits);
  // a split past the attended range holds no keys and writes nothing (the
  // merge reads only the used splits); an empty range gives NaN outputs
  if (nks == 0) {
    if (span <= 0 && s == 0)
      decode_merge_group(part_o, part_ml, splits, 0, true, b, hk, sinks, out);
    return;
  }
  const PageList pages{page_indices + page_indptr[b], page_indptr[b + 1] - page_indptr[b],
                       num_pages};
  // the split's pages (it need not start on a page boundary)
  const int pg0 = k0 / kPage, npg = (k0 + nks - 1) / kPage - pg0 + 1;
  for (int i = t; i < npg; i += 256) pid[i] = pages.page_of(min((pg0 + i) * kPage, L - 1));
  // Q operand: head r % 8 of the group, dims 32 ks + 8 g .. + 7
  bf16x8 qb[2];
  {
    const u32x4* src = (const u32x4*)(q + ((size_t)b * kHq + hk * kGroup + (r & 7)) * kD);
    qb[0] = moe::as_bf16x8(src[g]);
    qb[1] = moe::as_bf16x8(src[4 + g]);
  }
  // the sinks of this thread's two output heads (t / 64 and t / 64 + 4),
  // loaded now: read at the end they cost a memory round trip of their own
  const uint16_t sink0 = sinks[hk * kGroup + (t >> 6)], sink1 = sinks[hk * kGroup + (t >> 6) + 4];
  __syncthreads();
  // A chunk's loads, K and V alike: 16-byte unit u = t + 256 j, key u / 8 =
  // c + 32 j (c = t / 8), part t % 8 -- a wave reads eight whole 128-byte rows
  // per instruction.  Keys past the chunk repeat its last key (finite;
  // masked).  V is written transposed, each 64-key half interleaved: position
  // 2i holds key i, 2i + 1 key i + 32 (the pair a thread holds, one 32-bit
  // store), the 16-byte units of a V^T row XOR-swizzled by its 8-row group
  // (the V part) so that the stores of a wave spread over the banks.
  const int vc = t >> 3, vpart = t & 7;
  u32x4 kv[4], vv[4];
  auto load_chunk = [&](int c) {
    const int kc0 = k0 + c * kDecChunk, last = min(kDecChunk, nks - c * kDecChunk) - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = kc0 + min(vc + 32 * j, last);
      const uint16_t* kr = kv_row(cache, pid[pos / kPage - pg0], 0, hk, pos % kPage) + vpart * 8;
      kv[j] = *(const u32x4*)kr;
      vv[j] = *(const u32x4*)(kr + kHkv * kHeadBlock / 2);  // the V row of the same key
    }
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int j = 0; j < 4; ++j) *(u32x4*)(ks + (vc + 32 * j) * kDecKRow + vpart * 8) = kv[j];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t a0 = (vv[2 * h2][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        const uint32_t a1 = (vv[2 * h2 + 1][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        const int unit = (8 * h2 + (vc >> 2)) ^ vpart;  // rows vpart * 8 + e: group vpart
        *(uint32_t*)(vt + (vpart * 8 + e) * kDecVRow + unit * 8 + ((2 * vc) & 7)) = a0 | (a1 << 16);
      }
  };
  load_chunk(0);
  store_chunk();
  __syncthreads();
  const int nch = (nks + kDecChunk - 1) / kDecChunk;
  float m_run = -INFINITY, l_run = 0.f;  // this lane's head r; l over its keys
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; ++c) {
    const int nkc = min(kDecChunk, nks - c * kDecChunk);
    if (c + 1 < nch) load_chunk(c + 1);  // in flight during this chunk's products
    // scores of the keys at V^T positions 32 w .. 32 w + 31: A row r of tile
    // kk is the key at position 32 w + 8 (r / 4) + 4 kk + r % 4, so result
    // element i of lane (r, g) is the key at position 32 w + 8 g + 4 kk + i,
    // the one V^T's operand slot 4 kk + i of the lane carries
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint16_t* kr = ks + dec_key_at(32 * wave + 8 * (r >> 2) + 4 * kk + (r & 3)) * kDecKRow + 8 * g;
      f32x4 st = dec_mfma(moe::as_bf16x8(*(const u32x4*)kr), qb[0], f32x4{0.f, 0.f, 0.f, 0.f});
      st = dec_mfma(moe::as_bf16x8(*(const u32x4*)(kr + 32)), qb[1], st);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = dec_key_at(32 * wave + 8 * g + 4 * kk + i);
        sv[4 * kk + i] = key < nkc ? st[i] * sm_scale : -INFINITY;
        mx = fmaxf(mx, sv[4 * kk + i]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    if (g == 0) red_m[wave][r] = mx;
    __syncthreads();
    // the running maximum (every chunk holds a key, so mn is finite) and the
    // rescaling of what the earlier chunks added
    const float mn = fmaxf(m_run, fmaxf(fmaxf(red_m[0][r], red_m[1][r]),
                                        fmaxf(red_m[2][r], red_m[3][r])));
    const float alpha = m_run == -INFINITY ? 0.0f : __expf(m_run - mn);
    m_run = mn;
    l_run *= alpha;
    bf16x8 ph, pl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = sv[j] == -INFINITY ? 0.0f : __expf(sv[j] - mn);
      l_run += p;
      ph[j] = (__bf16)p;
      pl[j] = (__bf16)(p - (float)ph[j]);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int row = 16 * dt + r;  // positions 32 w + 8 g .. + 7: one swizzled unit
      const bf16x8 va = moe::as_bf16x8(
          *(const u32x4*)(vt + row * kDecVRow + ((4 * wave + g) ^ ((row >> 3) & 7)) * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
      o[dt] = dec_mfma(va, ph, o[dt]);
      o[dt] = dec_mfma(va, pl, o[dt]);
    }
    __syncthreads();  // every wave is done with this chunk's tiles and maxima
    if (c + 1 < nch) {
      store_chunk();
      __syncthreads();
    }
  }
  // l over the wave's keys, then the waves' partial o in LDS (the K tile's
  // space: every wave passed the last chunk's barrier)
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  if (g == 0) red_l[wave][r] = l_run;
  if (wave == 0 && g == 0 && r < kGroup) hm[r] = m_run;
  float* const obuf = (float*)ks;
  if (r < kGroup) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) obuf[(wave * kGroup + r) * kD + 16 * dt + 4 * g + i] = o[dt][i];
  }
  __syncthreads();
  {
    // o[h][d]: thread -> dim t % 64, heads t / 64 and t / 64 + 4, waves summed in order
    const int d = t & 63, h0 = t >> 6;
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      o0 += obuf[(w * kGroup + h0) * kD + d];
      o1 += obuf[(w * kGroup + h0 + 4) * kD + d];
    }
    if (used == 1 && span <= covered) {
      // the only split: the merge's arithmetic for one split (its weight is
      // exp(0) = 1), done here without publishing the partial
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int hl = h0 + 4 * j, h = hk * kGroup + hl;
        const float l = ((red_l[0][hl] + red_l[1][hl]) + red_l[2][hl]) + red_l[3][hl];
        const float lse = hm[hl] + __logf(l);
        const float ob = bf2f(f2bf((j == 0 ? o0 : o1) / l));
        out[((size_t)b * kHq + h) * kD + d] = f2bf(ob * sink_factor(lse, j == 0 ? sink0 : sink1));
      }
      return;
    }
    // device scope (sc1): the merge may run in a workgroup on another XCD
    store_dev(part_o + (pidx + (size_t)h0 * splits) * kD + d, o0);
    store_dev(part_o + (pidx + (size_t)(h0 + 4) * splits) * kD + d, o1);
    if (t < kGroup) {
      const float lh = ((red_l[0][t] + red_l[1][t]) + red_l[2][t]) + red_l[3][t];
      store_dev(part_ml + (pidx + (size_t)t * splits) * 2 + 0, hm[t]);
      store_dev(part_ml + (pidx + (size_t)t * splits) * 2 + 1, lh);
    }
  }
  // The last of the group's used splits to finish merges them: each wave's
  // stores complete (vmcnt), the workgroup meets, one thread counts the
  // arrival (agent-scope atomic) and the one that completes the count resets
  // it to zero for the next call.
  __shared__ int is_last;
  moe::wait_vmcnt<0>();
  __syncthreads();
  if (t == 0) {
    int* cnt = arrive + b * kHkv + hk;
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == used - 1;
    if (is_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (is_last)
    decode_merge_group(part_o, part_ml, splits, used, span > covered, b, hk, sinks,
                       out);
}


// Decode attention, merge: the group's 8 query heads of sequence b over the
// used splits (max, rescaled sums in split order), then lse, the sink factor
// and the bf16 output.  The partials are read with device scope (written by
// other workgroups), and every load is issued without waiting on another:
// the maxima by 32 threads per head, then per tile of 32 splits the weights
// exp(m_s - m) and the l_s by one thread each into LDS, and the o values by
// the (dim, head) threads, eight loads in flight before their sums.  The
// sums run in split order.  `bad` (the attended range is empty or longer
// than the splits cover: the caller's bound was too small) gives NaN outputs.
// Called by all 256 threads of the workgroup.
__device__ void decode_merge_group(const float* part_o, const float* part_ml, int splits,
                                   int used, bool bad, int b, int hk, const uint16_t* sinks,
                                   uint16_t* out) {
  constexpr int kTile = 32;
  __shared__ float wgt[kGroup][kTile];   // exp(m_s - m) in [0, 1], or -1 for a skipped split
  __shared__ float lval[kGroup][kTile];  // l_s
  __shared__ float lsum[kGroup];
  __shared__ float hmax[kGroup];
  const int t = threadIdx.x;
  const int d = t & 63;
  if (bad) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      out[((size_t)b * kHq + hk * kGroup + (t >> 6) + 4 * j) * kD + d] = 0x7FC0;
    return;
  }
  // this thread's two output heads' sinks first (read at the end, they would
  // cost a memory round trip of their own)
  const uint16_t sk[2] = {sinks[hk * kGroup + (t >> 6)], sinks[hk * kGroup + (t >> 6) + 4]};
  // maxima: thread (head t / 32, lane i = t % 32) over splits i, i + 32, ...
  const int mh = t >> 5, mi = t & 31;
  const size_t mbase = ((size_t)b * kHq + hk * kGroup + mh) * splits;
  {
    float m = -INFINITY;
    for (int s = mi; s < used; s += kTile) m = fmaxf(m, load_dev(part_ml + (mbase + s) * 2));
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if (mi == 0) {
      hmax[mh] = m;
      lsum[mh] = 0.0f;
    }
  }
  float o[2] = {0.0f, 0.0f};
  size_t obase[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    obase[j] = ((size_t)b * kHq + hk * kGroup + (t >> 6) + 4 * j) * splits;
  for (int s0 = 0; s0 < used; s0 += kTile) {
    const int nt = min(kTile, used - s0);
    __syncthreads();  // hmax written; the previous tile's weights consumed
    if (mi < nt) {
      const float ms = load_dev(part_ml + (mbase + s0 + mi) * 2);
      lval[mh][mi] = load_dev(part_ml + (mbase + s0 + mi) * 2 + 1);
      wgt[mh][mi] = ms == -INFINITY ? -1.0f : __expf(ms - hmax[mh]);
    }
    __syncthreads();
    if (mi == 0) {  // l in split order (one thread per head)
      float l = lsum[mh];
      for (int i = 0; i < nt; ++i) {
        const float w = wgt[mh][i];
        if (!(w < 0.0f)) l = fmaf(lval[mh][i], w, l);
      }
      lsum[mh] = l;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = (t >> 6) + 4 * j;
      for (int i0 = 0; i0 < nt; i0 += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = i0 + i < nt ? load_dev(part_o + (obase[j] + s0 + i0 + i) * kD + d) : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float w = i0 + i < nt ? wgt[h][i0 + i] : -1.0f;
          if (!(w < 0.0f)) o[j] = fmaf(v[i], w, o[j]);
        }
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int hl = (t >> 6) + 4 * j, h = hk * kGroup + hl;
    const float l = lsum[hl];
    const float lse = hmax[hl] + __logf(l);
    const float ob = bf2f(f2bf(o[j] / l));
    out[((size_t)b * kHq + h) * kD + d] = f2bf(ob * sink_factor(lse, sk[j]));
  }
}

// ---------------------------------------------------------------------------
// Prefill / extend attention on v_mfma_f32_16x16x32_bf16.
//
// Workgroup = (query tile of 64 rows of one sequence, kv head hk, half h of
// its GQA group): 4 waves, wave w = query head 8 hk + 4 h + w, so 4 heads share
// each key/value block staged in LDS.  At 256 VGPRs a SIMD holds two
// waves: two independent workgroups per CU, whose barriers and phases do not
// line up, rather than one of 8 waves.  Keys in blocks of 64 (four pages),
// double buffered: the next block's global loads are in flight while the
// current block's MFMAs run, one barrier per block.
//
// The products are arranged so that only two facts of the MFMA's lane layout
// matter: operand row (A) / column (B) = lane % 16, and result element i of
// lane l = row 4 (l / 16) + i, column l % 16.  Which k each of a lane's 8
// operand slots carries is the same for A and B, so pairing slot j of A with
// slot j of B always multiplies matching k.
//  * S^T = K Q^T (A = 16 keys x 32 dims, B = 32 dims x 16 queries): lane l of
//    key subblock kk holds S[query l % 16][key 16 kk + 4 (l / 16) + i].
//  * O^T += V^T P^T per 32 keys (A = 16 dims x 32 keys, B = 32 keys x 16
//    queries, P as two bf16 pieces): P's operand slot j of lane l carries key
//    4 (l / 16) + j / 2 (j even) or 16 + 4 (l / 16) + (j - 1) / 2 (j odd) --
//    scores lane l holds -- and V^T's slot j of lane l carries the same key,
//    read from a transposed LDS tile whose 32-key halves are interleaved
//    (position 2i key i, 2i + 1 key i + 16), so that a lane's 8 keys are one
//    16-byte read.
constexpr int kPfQ = 64;              // query rows per wave
constexpr int kPfSub = kPfQ / 16;     // 16-row subtiles per wave
constexpr int kPfKeys = 64;           // keys per block
constexpr int kKRow = kD + 8;         // K tile row (bf16), padded
constexpr int kVRow = kPfKeys + 8;    // V^T tile row (bf16), padded
constexpr int kPfWaves = 4;           // waves (query heads) per workgroup
constexpr float kPfSlack = 8.0f;      // log2 headroom of the lazy softmax rescale
constexpr int kPfHalves = kGroup / kPfWaves;  // workgroups per GQA group

// max of x over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows) in
// registers: swapping x with itself, v_permlane32_swap returns x of lanes
// l & 31 and l | 32, v_permlane16_swap x of rows 2 (l / 32) and 2 (l / 32) + 1
__device__ __forceinline__ float group_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(
    const uint16_t* __restrict__ q, const int* __restrict__ q_indptr,
    const uint8_t* __restrict__ cache, const int* __restrict__ page_indptr,
    const int* __restrict__ page_indices, int num_pages, const int* __restrict__ kv_len,
    int window, float sm_scale, const uint16_t* __restrict__ sinks, int tiles_per_seq,
    uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint16_t kt[2][kPfKeys * kKRow];
  __shared__ __align__(16) uint16_t vt[2][kD * kVRow];
  // each lane's Q operands, parked in LDS (a lane reads back only what it
  // wrote), leaving registers for two subtiles' scores at once
  __shared__ __align__(16) u32x4 qs[kPfWaves][2 * kPfSub][kWave];
  // Workgroups are dispatched in linear order (x, then y): the linear index
  // walks query tiles from the last, which under the causal mask attends to
  // the most keys, so the longest tiles start first and the short ones fill
  // the CUs they free (the tiles of one sequence otherwise ran as rounds each
  // as long as its longest tile).  Within a tile: (sequence, half, kv head),
  // so the two halves of a kv head's group are 8 workgroups apart and share
  // an XCD (workgroups go round-robin over the 8 XCDs) and its L2.
  const int lin = (int)(blockIdx.x + blockIdx.y * gridDim.x);
  const int per_tile = (int)(gridDim.x / tiles_per_seq) * kPfHalves * kHkv;
  const int tile = tiles_per_seq - 1 - lin / per_tile;
  const int rest = lin % per_tile;
  const int b = rest / (kPfHalves * kHkv), half = rest / kHkv % kPfHalves, hk = rest % kHkv;
  const int qb = q_indptr[b], qn = q_indptr[b + 1] - qb;
  const int q0 = tile * kPfQ;
  if (q0 >= qn) return;
  const int L = kv_len[b];
  const int P = L - qn;  // positions of the sequence's queries: P .. L - 1
  const int t = threadIdx.x;
  const int wave = t >> 6, lane = t & 63;
  const int r = lane & 15, g = lane >> 4;
  const int head = hk * kGroup + half * kPfWaves + wave;
  const PageList pages{page_indices + page_indptr[b], page_indptr[b + 1] - page_indptr[b],
                       num_pages};

  // this wave's Q operands: [query subtile][k step] (rows past the sequence
  // repeat its last query; their results are not stored)
#pragma unroll
  for (int qt = 0; qt < kPfSub; ++qt) {
    const int row = qb + min(q0 + qt * 16 + r, qn - 1);
    const u32x4* src = (const u32x4*)(q + ((size_t)row * kHq + head) * kD);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qs[wave][qt * 2 + ks][lane] = src[ks * 4 + g];
  }
  const float c2 = sm_scale * 1.4426950408889634f;  // scores in log2 units
  f32x4 o[kPfSub][4];
  float m[kPfSub], l[kPfSub];
#pragma unroll
  for (int qt = 0; qt < kPfSub; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int qlast = min(q0 + kPfQ, qn) - 1;
  const int kmax = P + qlast;                                     // last key any row sees
  const int kmin = window > 0 ? max(0, P + q0 - window + 1) : 0;  // first key any row sees
  const int kfirst = kmin / kPfKeys * kPfKeys;

  // Staging: load j brings page j of the block (keys 16 j .. 16 j + 15),
  // threads 0..127 its K rows, threads 128..255 its V rows, 16-byte part
  // t % 8 of key 16 j + c (c = (t % 128) / 8).  A load's page is the same for
  // every lane: a scalar base (the page ids are scalar loads issued one block
  // ahead, pid) plus a fixed lane offset.  V is written transposed, each
  // 32-key half interleaved: position 2i holds key i, 2i + 1 key i + 16, the
  // pair (loads 2h, 2h + 1) in one 32-bit store.  In a block that runs past
  // kv_len, keys beyond it read key L - 1 (finite, masked).
  const int kvsel = t >> 7, c = (t & 127) >> 3, part = t & 7;
  const unsigned lane_base = (unsigned)((kvsel * kHkv + hk) * kHeadBlock) + part * 16;
  const unsigned lane_off = lane_base + c * (kD * 2);
  // page list index clamped to the page holding key L - 1: a page of the
  // block wholly past kv_len resolves to that page
  const int last_page = min(pages.count - 1, (L - 1) / kPage);
  int pid[4];
  auto fetch_pages = [&](int kb0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) pid[j] = pages.ids[max(min(kb0 / kPage + j, last_page), 0)];
  };
  u32x4 sr[4];
  auto load = [&](int kb0) {
    const unsigned lim = (unsigned)(L - 1 - kb0);  // the block starts before kv_len
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      unsigned off = lane_off;
      if (lim < (unsigned)(kPfKeys - 1)) {  // keys past L - 1 read key L - 1
        const unsigned pj = min((unsigned)j, lim / kPage);
        off = lane_base + (min((unsigned)(kPage * j + c), lim) - kPage * pj) * (kD * 2);
      }
      const uint8_t* pbase = cache + (size_t)(unsigned)pages.clamp(pid[j]) * kPageBytes;
      sr[j] = *(const u32x4*)(pbase + off);
    }
  };
  auto store = [&](int buf) {
    if (kvsel == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) *(u32x4*)(kt[buf] + (kPage * j + c) * kKRow + part * 8) = sr[j];
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t a0 = (sr[2 * h][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          const uint32_t a1 = (sr[2 * h + 1][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          *(uint32_t*)(vt[buf] + (part * 8 + e) * kVRow + 32 * h + 2 * c) = a0 | (a1 << 16);
        }
    }
  };

  if (kfirst <= kmax) {
    fetch_pages(kfirst);
    load(kfirst);
    if (kfirst + kPfKeys <= kmax) fetch_pages(kfirst + kPfKeys);
    store(0);
  }
  // every load before the loop (Q, the first block, the next page ids) done:
  // inside the loop the compiler then waits only for the block prefetch
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  int buf = 0;
  for (int kb0 = kfirst; kb0 <= kmax; kb0 += kPfKeys) {
    const bool more = kb0 + kPfKeys <= kmax;
    if (more) {
      load(kb0 + kPfKeys);  // in flight during this block's MFMAs
      if (kb0 + 2 * kPfKeys <= kmax) fetch_pages(kb0 + 2 * kPfKeys);
    }
    bf16x8 ka[4][2];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        ka[kk][ks] =
            moe::as_bf16x8(*(const u32x4*)(kt[buf] + (kk * 16 + r) * kKRow + ks * 32 + g * 8));
    // V^T operand: positions 8g .. 8g + 7 of the half, keys 4g + i (slots 2i)
    // and 16 + 4g + i (slots 2i + 1)
    bf16x8 va[2][4];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        va[s2][dt] = moe::as_bf16x8(*(const u32x4*)(vt[buf] + (dt * 16 + r) * kVRow + s2 * 32 + 8 * g));
    // The 16-row subtiles, software-pipelined: subtile qt + 1's scores
    // (its Q operands read from LDS first) are issued in the same stretch of
    // code as subtile qt's exponentials and P V products, so the MFMAs of one
    // run while the vector ALUs work on the other.  A subtile whose rows see
    // none of the block is not skipped: its mask sets every score to -inf, so
    // p = 0 and o, l and m are unchanged.
    bf16x8 q2[2];
    f32x4 sa[4], sb[4];
    auto read_q = [&](int qt) {
      q2[0] = moe::as_bf16x8(qs[wave][qt * 2][lane]);
      q2[1] = moe::as_bf16x8(qs[wave][qt * 2 + 1][lane]);
    };
    auto scores = [&](f32x4 (&st)[4]) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        st[kk] = mfma_bf16(ka[kk][0], q2[0], f32x4{0.f, 0.f, 0.f, 0.f});
        st[kk] = mfma_bf16(ka[kk][1], q2[1], st[kk]);
      }
    };
    read_q(0);
    scores(sa);
#pragma unroll
    for (int qt = 0; qt < kPfSub; ++qt) {
      f32x4 (&st)[4] = (qt & 1) ? sb : sa;
      f32x4 (&sn)[4] = (qt & 1) ? sa : sb;
      if (qt < kPfSub - 1) read_q(qt + 1);
      const int qpos0 = P + q0 + qt * 16;  // this subtile's positions: qpos0 .. qpos0 + 15
      // mask: key kb0 + 16 kk + 4 g + i for the query at position qpos; a
      // block that every row of the subtile sees whole (all blocks of a
      // causal row but its diagonal one) skips it
      const bool whole = kb0 + kPfKeys - 1 <= qpos0 && kb0 + kPfKeys <= L &&
                         (window <= 0 || kb0 >= qpos0 + 15 - window + 1);
      if (!whole) {
        const int qpos = qpos0 + r;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb0 + kk * 16 + 4 * g + i;
            const bool ok = key <= qpos && key < L && (window <= 0 || key >= qpos - window + 1);
            st[kk][i] = ok ? st[kk][i] : -INFINITY;
          }
      }
      // the row maximum of the raw scores: scaling by c2 > 0 keeps the order
      float bm = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i) bm = fmaxf(bm, st[kk][i]);
      bm = group_max(bm);
      // The reference point m of a row moves to the new maximum only when some
      // row's maximum exceeds its m by more than kPfSlack (log2 units): until
      // then p = 2^(s c2 - m) stays below 2^kPfSlack, and o and l carry the
      // same factor, so o / l and the lse m + log2(l) are unchanged.  The
      // rescale then runs on the first blocks of a row and seldom after.
      const float mn = fmaxf(m[qt], bm * c2);
      if (__any(mn > m[qt] + kPfSlack)) {
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[qt] - mn);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[qt][dt][i] *= alpha;
        l[qt] *= alpha;
        m[qt] = mn;
      }
      if (qt < kPfSub - 1) scores(sn);
      // p = 2^(s c2 - m); masked scores (-inf) give 0, also in a row that has
      // seen no key yet (m = -inf)
      const float mneg = m[qt] == -INFINITY ? 0.0f : -m[qt];
      float ps = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        // P enters the MFMA as two bf16 pieces, p = hi + lo to about 16 bits,
        // so the products keep the fp32 probabilities' precision: hi = p
        // truncated to bf16 (its top 16 bits), lo = bf16(p - hi) (the
        // difference is exact in fp32)
        uint32_t pb[8];
        bf16x8 pl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kk = s2 * 2 + (j & 1), i = j >> 1;  // the key V^T's slot j holds
          const float p = __builtin_amdgcn_exp2f(fmaf(st[kk][i], c2, mneg));
          ps += p;
          pb[j] = __float_as_uint(p);
          pl[j] = (__bf16)(p - __uint_as_float(pb[j] & 0xFFFF0000u));
        }
        const bf16x8 ph = moe::as_bf16x8(u32x4{
            __builtin_amdgcn_perm(pb[1], pb[0], 0x07060302u), __builtin_amdgcn_perm(pb[3], pb[2], 0x07060302u),
            __builtin_amdgcn_perm(pb[5], pb[4], 0x07060302u), __builtin_amdgcn_perm(pb[7], pb[6], 0x07060302u)});
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          o[qt][dt] = mfma_bf16(va[s2][dt], ph, o[qt][dt]);
          o[qt][dt] = mfma_bf16(va[s2][dt], pl, o[qt][dt]);
        }
      }
      l[qt] += ps;
    }
    if (more) store(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  // epilogue: row sums across the 4 lane groups, lse, sink factor, bf16
#pragma unroll
  for (int qt = 0; qt < kPfSub; ++qt) {
    float lt = l[qt];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    const int qi = q0 + qt * 16 + r;
    const float lse = (m[qt] + __log2f(lt)) * 0.6931471805599453f;
    const float sf = sink_factor(lse, sinks[head]);
    const float inv = 1.0f / lt;
    if (qi < qn) {
      uint16_t* dst = out + ((size_t)(qb + qi) * kHq + head) * kD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        uint16_t v4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = f2bf(bf2f(f2bf(o[qt][dt][i] * inv)) * sf);
        *(uint2*)(dst + dt * 16 + 4 * g) =
            make_uint2((uint32_t)v4[0] | ((uint32_t)v4[1] << 16), (uint32_t)v4[2] | ((uint32_t)v4[3] << 16));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// out = bf16(x + bf16(y + bias)): the output linear's bias (nn.Linear's second
// op) and the residual add of attention.py:256.  Four columns per thread.
__global__ __launch_bounds__(256) void bias_residual_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ y,
                                                            const uint16_t* __restrict__ bias,
                                                            int64_t total, int H,
                                                            uint16_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= total) return;
  const int c = (int)(i % H);
  uint16_t o4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float t = bf2f(f2bf(bf2f(y[i + j]) + bf2f(bias[c + j])));
    o4[j] = f2bf(bf2f(x[i + j]) + t);
  }
  *(uint2*)(out + i) = make_uint2((uint32_t)o4[0] | ((uint32_t)o4[1] << 16),
                                  (uint32_t)o4[2] | ((uint32_t)o4[3] << 16));
}

// Embedding gather (transformer.py:101-105): out[i] = table[ids[i]]; ids
// outside [0, vocab) give a zero row.  One workgroup per token, 16 bytes per
// thread.
__global__ __launch_bounds__(256) void embedding_kernel(const int* __restrict__ ids,
                                                        const uint16_t* __restrict__ table,
                                                        int vocab, int H,
                                                        uint16_t* __restrict__ out) {
  const int tok = blockIdx.x;
  const int id = ids[tok];
  const bool ok = id >= 0 && id < vocab;
  for (int c = threadIdx.x * 8; c < H; c += 256 * 8) {
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (ok) v = *(const u32x4*)(table + (size_t)id * H + c);
    *(u32x4*)(out + (size_t)tok * H + c) = v;
  }
}

}  // namespace attn

// ---------------------------------------------------------------------------
// Launchers (argument checks live in the C ABI, attn_capi.hip)
extern "C" {

int attn_launch_rms_norm(const void* x, int n, int H, const void* w, float eps, void* out,
                         hipStream_t s) {
  hipLaunchKernelGGL(attn::rms_norm_kernel, dim3(n), dim3(256), 0, s, (const uint16_t*)x, H,
                     (const uint16_t*)w, eps, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_qkv_rope_append(const void* qkv, const void* bias, int n, const int* positions,
                                const int* slots, const float* inv_freq, float conc, void* cache,
                                int num_pages, void* q_out, hipStream_t s) {
  hipLaunchKernelGGL(attn::qkv_rope_append_kernel, dim3(attn::kQkvHeads / 8, n), dim3(256), 0, s,
                     (const uint16_t*)qkv, (const uint16_t*)bias, positions, slots, inv_freq, conc,
                     (uint8_t*)cache, num_pages, (uint16_t*)q_out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_decode(const void* q, int batch, const void* cache, const int* page_indptr,
                       const int* page_indices, int num_pages, const int* kv_len, int window,
                       float sm_scale, const void* sinks, int splits, int cps, float* part_o,
                       float* part_ml, int* arrive, void* out, hipStream_t s) {
  if (cps < 1 || cps > attn::kDecMaxCps) return -6;
  hipLaunchKernelGGL(attn::decode_partial_kernel, dim3(splits, attn::kHkv, batch), dim3(256), 0, s,
                     (const uint16_t*)q, (const uint8_t*)cache, page_indptr, page_indices,
                     num_pages, kv_len, window, sm_scale, splits, cps, part_o, part_ml, arrive,
                     (const uint16_t*)sinks, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_prefill(const void* q, const int* q_indptr, int batch, int max_q_len,
                        const void* cache, const int* page_indptr, const int* page_indices,
                        int num_pages, const int* kv_len, int window, float sm_scale,
                        const void* sinks, void* out, hipStream_t s) {
  const int tiles = (max_q_len + attn::kPfQ - 1) / attn::kPfQ;
  hipLaunchKernelGGL(attn::prefill_kernel, dim3(tiles * batch, attn::kHkv * attn::kPfHalves),
                     dim3(64 * attn::kPfWaves), 0, s,
                     (const uint16_t*)q, q_indptr, (const uint8_t*)cache, page_indptr, page_indices,
                     num_pages, kv_len, window, sm_scale, (const uint16_t*)sinks, tiles,
                     (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_bias_residual(const void* x, const void* y, const void* bias, int64_t n, int H,
                              void* out, hipStream_t s) {
  const int64_t total = n * H;
  const int64_t blocks = (total / 4 + 255) / 256;
  hipLaunchKernelGGL(attn::bias_residual_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)bias, total, H,
                     (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int attn_launch_embedding(const int* ids, int n, const void* table, int vocab, int H, void* out,
                          hipStream_t s) {
  hipLaunchKernelGGL(attn::embedding_kernel, dim3(n), dim3(256), 0, s, ids,
                     (const uint16_t*)table, vocab, H, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // extern "C"
