/*
 * C restatement of the reference MoE block -- TEST INFRASTRUCTURE ONLY.
 *
 * This is the CPU oracle and CPU baseline for the gpt-oss MXFP4 MoE block.  It
 * follows the loop nest of brekkylab/gpt-oss-tvm model/mlp.py, the block that
 * model/transformer.py:10 wires in:
 *
 *   run_einsum  (mlp.py:238-326)  serial fp32 accumulation from the bias, one
 *                                 multiply-add per input element, with the
 *                                 exp2(scale-127) recomputed per element
 *                                 (mlp.py:289-317) -- exactly that order;
 *   swiglu      (mlp.py:29-60)    fp32, out_dtype float32 (mlp.py:390);
 *   run_gating  (mlp.py:328-369)  fp32, slot order, then bf16;
 *   forward     (mlp.py:371-402)  norm, router, top-k, softmax, residual.
 *
 * TVM compiles that unscheduled TIR to serial loops on its llvm (CPU) target,
 * so the single-threaded build of this file is the faithful stand-in for the
 * reference's CPU path.  An OpenMP loop over (token, slot) gives an all-core
 * upper bound.  Where TVM's lowering cannot be observed (tvm is absent), this
 * file applies the same canonical choices as oracle/moe_oracle.py:
 * fp64 sum of squares and router dot, lower-index-wins top-k, fp64 softmax,
 * correctly rounded sigmoid.  Build with -ffp-contract=off so that every
 * written multiply and add rounds separately.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load the library built from this file.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* e2m1 code -> value, model/mlp.py:9-26 */
static const float kFp4[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint64_t r = ((uint64_t)u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)(r & 0xFFFFu);
}

/* model/mlp.py:81-87,375 -- canonical fp64 reduction, one fp32 rounding of r. */
static void rms_norm_row(const uint16_t* x, const uint16_t* w, int H, float eps, uint16_t* t) {
  double ss = 0.0;
  for (int i = 0; i < H; ++i) {
    double v = (double)bf2f(x[i]);
    ss += v * v;
  }
  float r = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
  for (int i = 0; i < H; ++i) {
    float xr = bf2f(x[i]) * r;
    t[i] = f2bf(xr * bf2f(w[i]));
  }
}

/* model/mlp.py:88-92,376 -- bf16(bf16(dot) + bias), dot in fp64. */
static void router_row(const uint16_t* t, const uint16_t* gw, const uint16_t* gb, int H, int E,
                       float* g) {
  for (int e = 0; e < E; ++e) {
    double acc = 0.0;
    const uint16_t* we = gw + (size_t)e * H;
    for (int i = 0; i < H; ++i) acc += (double)bf2f(t[i]) * (double)bf2f(we[i]);
    float dot = bf2f(f2bf((float)acc));
    g[e] = bf2f(f2bf(dot + bf2f(gb[e])));
  }
}

/* model/mlp.py:381-382 -- top-k descending, lower index wins ties; softmax. */
static void topk_softmax_row(const float* g, int E, int k, int32_t* idx, uint16_t* w) {
  unsigned char taken[1024];
  memset(taken, 0, (size_t)E);
  double v[16];
  for (int j = 0; j < k; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e) {
      if (taken[e]) continue;
      if (best < 0 || g[e] > g[best]) best = e;
    }
    taken[best] = 1;
    idx[j] = best;
    v[j] = (double)g[best];
  }
  double ex[16];
  double s = 0.0;
  for (int j = 0; j < k; ++j) {
    ex[j] = exp(v[j] - v[0]);
    s = (j == 0) ? ex[0] : s + ex[j];
  }
  for (int j = 0; j < k; ++j) w[j] = f2bf((float)(ex[j] / s));
}

/*
 * model/mlp.py:238-326.  x is fp32 values: [n, K] when x_is_3d == 0, else
 * [n, k, K].  Writes out [n, k, N] fp32.
 */
void moe_ref_einsum(const float* x, int x_is_3d, const int32_t* idx, int n, int k, int N, int K,
                    const uint8_t* blocks, const uint8_t* scales, const uint16_t* bias, float* out,
                    int nthreads) {
  const int G = K / 32;
  long total = (long)n * k;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (long sr = 0; sr < total; ++sr) {
    const int s = (int)(sr / k), r = (int)(sr % k);
    const int e = idx[(size_t)s * k + r];
    const float* xs = x_is_3d ? x + ((size_t)s * k + r) * K : x + (size_t)s * K;
    float* o = out + ((size_t)s * k + r) * N;
    for (int c = 0; c < N; ++c) {
      const size_t row = (size_t)e * N + c;
      float sum = bf2f(bias[row]);
      for (int in_idx = 0; in_idx < K; ++in_idx) {
        const int g = in_idx / 32;
        const int local = in_idx % 32;
        const int byte_idx = local / 2;
        const int is_high = local % 2;
        const int sv = (int)scales[row * G + g] - 127;
        const float ldexp_scale = exp2f((float)sv);
        const uint8_t bv = blocks[(row * G + g) * 16 + byte_idx];
        const int nib = (bv >> (is_high * 4)) & 0x0F;
        sum += xs[in_idx] * kFp4[nib] * ldexp_scale;
      }
      o[c] = sum;
    }
  }
  (void)nthreads;
}

/* model/mlp.py:29-60, fp32 out. */
void moe_ref_swiglu(const float* x, long pairs, float alpha, float limit, float* out) {
  for (long i = 0; i < pairs; ++i) {
    float glu = x[2 * i], lin = x[2 * i + 1];
    float xg = glu < limit ? glu : limit;
    float xl = lin < -limit ? -limit : (lin > limit ? limit : lin);
    float z = alpha * xg;
    float sig = (float)(1.0 / (1.0 + exp(-(double)z)));
    float gate = xg * sig;
    out[i] = gate * (xl + 1.0f);
  }
}

/* model/mlp.py:328-369 then mlp.py:402 (residual when x != NULL). */
void moe_ref_gating(const float* y, const uint16_t* w, const uint16_t* x, int n, int k, int N,
                    uint16_t* out) {
  for (int s = 0; s < n; ++s) {
    for (int c = 0; c < N; ++c) {
      float acc = 0.0f;
      for (int r = 0; r < k; ++r) {
        float prod = y[((size_t)s * k + r) * N + c] * bf2f(w[(size_t)s * k + r]);
        acc = acc + prod;
      }
      uint16_t t = f2bf(acc);
      out[(size_t)s * N + c] = x ? f2bf(bf2f(x[(size_t)s * N + c]) + bf2f(t)) : t;
    }
  }
}

/* Norm + router + top-k + softmax for n tokens. */
void moe_ref_route(const uint16_t* x, int n, int H, int E, int k, const uint16_t* norm_w,
                   const uint16_t* gate_w, const uint16_t* gate_b, float eps, uint16_t* t_out,
                   int32_t* idx_out, uint16_t* w_out) {
  float* g = (float*)malloc(sizeof(float) * (size_t)E);
  for (int s = 0; s < n; ++s) {
    uint16_t* t = t_out + (size_t)s * H;
    rms_norm_row(x + (size_t)s * H, norm_w, H, eps, t);
    router_row(t, gate_w, gate_b, H, E, g);
    topk_softmax_row(g, E, k, idx_out + (size_t)s * k, w_out + (size_t)s * k);
  }
  free(g);
}

/*
 * MLPBlock.forward, model/mlp.py:371-402, on x [n, H] bf16.  Scratch for the
 * fp32 intermediates is allocated here (n*k*(2I + I + H) floats).
 * Returns 0, or -1 on bad arguments / allocation failure.
 */
int moe_ref_block_forward(const uint16_t* x, int n, int H, int I, int E, int k,
                          const uint16_t* norm_w, const uint16_t* gate_w, const uint16_t* gate_b,
                          const uint8_t* m1b, const uint8_t* m1s, const uint16_t* m1bias,
                          const uint8_t* m2b, const uint8_t* m2s, const uint16_t* m2bias,
                          float eps, float limit, float alpha, int nthreads, uint16_t* out,
                          uint16_t* t_out, int32_t* idx_out, uint16_t* w_out) {
  if (n <= 0 || H % 32 || I % 32 || k <= 0 || k > 16 || E < k || E > 1024) return -1;
  float* tf = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* h1 = (float*)malloc(sizeof(float) * (size_t)n * k * 2 * I);
  float* act = (float*)malloc(sizeof(float) * (size_t)n * k * I);
  float* y = (float*)malloc(sizeof(float) * (size_t)n * k * H);
  if (!tf || !h1 || !act || !y) {
    free(tf); free(h1); free(act); free(y);
    return -1;
  }
  moe_ref_route(x, n, H, E, k, norm_w, gate_w, gate_b, eps, t_out, idx_out, w_out);
  for (size_t i = 0; i < (size_t)n * H; ++i) tf[i] = bf2f(t_out[i]);
  moe_ref_einsum(tf, 0, idx_out, n, k, 2 * I, H, m1b, m1s, m1bias, h1, nthreads);
  moe_ref_swiglu(h1, (long)n * k * I, alpha, limit, act);
  moe_ref_einsum(act, 1, idx_out, n, k, H, I, m2b, m2s, m2bias, y, nthreads);
  moe_ref_gating(y, w_out, x, n, k, H, out);
  free(tf); free(h1); free(act); free(y);
  return 0;
}
