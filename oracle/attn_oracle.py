"""CPU oracle for the gpt-oss attention block and the decode loop around the
MoE block -- TEST INFRASTRUCTURE ONLY.

Restates in numpy the arithmetic of the reference's ``AttentionBlock``
(brekkylab/gpt-oss-tvm ``model/attention.py:15-256``), the attention masks of
its TVM patch (``tvm_fix.patch:36-47``: causal plus sliding-window lower
bound), the layer loop and logits of ``model/transformer.py:21-31,54-66,
98-133``, and the top-p sampler the engine calls (``engine.py:39-40,165-167``:
TVM's ``vm.builtin.sample_top_p_from_logits``, restated below from TVM's
published source, ``src/runtime/relax_vm/lm_support.cc``, TVM as pinned by the
reference's ``tvm_fix.patch``).  It checks the HIP library: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU leg may import it.

bf16 tensors are carried as uint16 bit patterns, as in ``moe_oracle``.

Canonical numerics (TVM's lowering cannot be observed here; each choice is the
arithmetic the reference's TIR/Relax expressions state, evaluated exactly
where they leave the order open):

* RMSNorm    as ``moe_oracle.rms_norm`` (``attention.py:80``, ``nn.RMSNorm``).
* Linear     ``nn.Linear`` = matmul with a bf16 output, then ``+ bias`` as a
             second bf16 op: bf16(bf16(x @ W^T) + b); the dot products are
             summed in fp64 and rounded once to fp32 then bf16.
* RoPE       YaRN frequencies in fp32 (``attention.py:40-66``), cos/sin of
             fp32(position) * inv_freq in fp64 rounded to fp32, then to the
             activation dtype (bf16) as ``.astype(dtype)`` states, times the
             fp32 concentration 0.1 ln(factor) + 1; the rotation in fp32
             (multiply, multiply, add/sub, no fma) rounded to bf16
             (``attention.py:126-165``); half-split pairs (d, d + 32).
* Attention  scores q.k * sm_scale in fp64, masked per ``tvm_fix.patch:36-47``,
             softmax and lse (natural log) in fp64; o rounded to bf16.
* Sinks      s = bf16(sigmoid(lse - sink)), o' = bf16(o * s)
             (``attention.py:235-245``; sigmoid in fp64 rounded to fp32).
* Sampling   TVM's algorithm with exact (fp64) masses and exp rounded once to
             fp32; sort descending by logit, equal logits in index order (the
             C++ std::sort leaves their order open).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from oracle.moe_oracle import bf16_to_f32, f32_to_bf16, f64_to_bf16, rms_norm

HEAD_DIM = 64
N_Q_HEADS = 64
N_KV_HEADS = 8
SLIDING_WINDOW = 128
ROPE_THETA = 150000.0
# model/config.py:41-48 (the rope_scaling defaults); attention.py:103-110
YARN = {"factor": 32.0, "beta_fast": 32.0, "beta_slow": 1.0,
        "original_max_position_embeddings": 4096}


# ---------------------------------------------------------------------------
# YaRN RoPE (attention.py:15-66, 94-165)
# ---------------------------------------------------------------------------

def yarn_correction_range(rotary_dim: int = HEAD_DIM, theta: float = ROPE_THETA,
                          beta_fast: float = YARN["beta_fast"], beta_slow: float = YARN["beta_slow"],
                          max_pos: int = YARN["original_max_position_embeddings"]):
    """(low, high) of attention.py:24-37 as fp32 constants: the dims at which
    ``beta_fast`` and ``beta_slow`` rotations fit the original context, clamped
    to [0, rotary_dim - 1] (no truncation: ``truncate`` is False)."""
    def dim(num_rot):
        return rotary_dim * math.log(max_pos / (num_rot * 2 * math.pi)) / (2 * math.log(theta))
    low = np.float32(max(dim(beta_fast), 0.0))
    high = np.float32(min(dim(beta_slow), rotary_dim - 1))
    if low == high:  # attention.py:61
        high = np.float32(high + np.float32(0.001))
    return low, high


def yarn_inv_freq(rotary_dim: int = HEAD_DIM, theta: float = ROPE_THETA,
                  factor: float = YARN["factor"]) -> np.ndarray:
    """inv_freq[d], d = 0 .. rotary_dim/2 - 1, in fp32 (attention.py:53-64)."""
    d = np.arange(rotary_dim // 2, dtype=np.int64)
    exponent = ((d * 2) % rotary_dim).astype(np.float32) / np.float32(rotary_dim)
    freq_power = np.power(np.float32(theta), exponent).astype(np.float32)
    freq_extra = (np.float32(1.0) / freq_power).astype(np.float32)
    freq_inter = (np.float32(1.0) / (np.float32(factor) * freq_power)).astype(np.float32)
    low, high = yarn_correction_range(rotary_dim, theta)
    ramp = ((d.astype(np.float32) - low) / (high - low)).astype(np.float32)
    mask = (np.float32(1.0) - np.clip(ramp, np.float32(0.0), np.float32(1.0))).astype(np.float32)
    return (freq_inter * (np.float32(1.0) - mask) + freq_extra * mask).astype(np.float32)


def yarn_concentration(factor: float = YARN["factor"]) -> np.float32:
    """attention.py:147-148."""
    return np.float32(0.1 * math.log(factor) + 1.0 if factor > 1.0 else 1.0)


def rope_cos_sin(positions: np.ndarray, inv_freq: np.ndarray | None = None):
    """(cos, sin) [n, rotary_dim/2] as fp32 values: fp32(bf16(cos(freq))) * conc."""
    if inv_freq is None:
        inv_freq = yarn_inv_freq()
    pos = np.asarray(positions, dtype=np.int64).astype(np.float32)
    freq = (pos[:, None] * inv_freq[None, :]).astype(np.float32)
    conc = yarn_concentration()
    f64 = freq.astype(np.float64)
    c = bf16_to_f32(f64_to_bf16(np.cos(f64))) * conc
    s = bf16_to_f32(f64_to_bf16(np.sin(f64))) * conc
    return c.astype(np.float32), s.astype(np.float32)


def rope(x_bf16: np.ndarray, positions: np.ndarray, inv_freq: np.ndarray | None = None) -> np.ndarray:
    """Rotate x [n, heads, D] (bf16 bits) by position; attention.py:126-165."""
    x = bf16_to_f32(x_bf16)
    half = x.shape[-1] // 2
    c, s = rope_cos_sin(positions, inv_freq)
    c = c[:, None, :]
    s = s[:, None, :]
    lo, hi = x[..., :half], x[..., half:]
    out_lo = (lo * c).astype(np.float32) - (hi * s).astype(np.float32)
    out_hi = (lo * s).astype(np.float32) + (hi * c).astype(np.float32)
    return f32_to_bf16(np.concatenate([out_lo, out_hi], axis=-1).astype(np.float32))


# ---------------------------------------------------------------------------
# Linear, attention, sinks
# ---------------------------------------------------------------------------

def bias_add(y_bf16: np.ndarray, b_bf16: np.ndarray) -> np.ndarray:
    """bf16(y + b) over the last axis: nn.Linear's bias add, its own bf16 op."""
    return f32_to_bf16((bf16_to_f32(y_bf16) + bf16_to_f32(b_bf16)).astype(np.float32))


def linear(x_bf16: np.ndarray, w_bf16: np.ndarray, b_bf16: np.ndarray | None) -> np.ndarray:
    """bf16(bf16(x @ W^T) + b): nn.Linear's matmul then bias add."""
    x64 = bf16_to_f32(x_bf16).astype(np.float64)
    w64 = bf16_to_f32(w_bf16).astype(np.float64)
    y = f64_to_bf16(x64 @ w64.T)
    return y if b_bf16 is None else bias_add(y, b_bf16)


def allowed(q_pos: int, kv_len: int, window: int) -> np.ndarray:
    """Key positions 0..kv_len-1 a query at q_pos may attend to: causal, plus
    the sliding-window lower bound of tvm_fix.patch:36-47 (col >= row - W + 1
    with the query's row offset by kv_len - qo_len, i.e. its position)."""
    col = np.arange(kv_len)
    ok = col <= q_pos
    if window > 0:
        ok &= col >= q_pos - window + 1
    return ok


def attention(q_bf16: np.ndarray, k_bf16: np.ndarray, v_bf16: np.ndarray, q_pos: np.ndarray,
              window: int, sm_scale: float = 1.0 / math.sqrt(HEAD_DIM)):
    """q [n, Hq, D]; k, v [L, Hkv, D] (key j at position j); -> (o bf16 [n, Hq, D],
    lse fp32 [n, Hq], natural log).  GQA: q head h reads kv head h // (Hq/Hkv)."""
    q = bf16_to_f32(q_bf16).astype(np.float64)
    k = bf16_to_f32(k_bf16).astype(np.float64)
    v = bf16_to_f32(v_bf16).astype(np.float64)
    n, hq, d = q.shape
    L, hkv, _ = k.shape
    g = hq // hkv
    o = np.zeros((n, hq, d))
    lse = np.zeros((n, hq))
    for i in range(n):
        ok = allowed(int(q_pos[i]), L, window)
        kk = k[ok]
        vv = v[ok]
        for h in range(hq):
            s = kk[:, h // g, :] @ q[i, h] * sm_scale
            m = s.max()
            e = np.exp(s - m)
            z = e.sum()
            lse[i, h] = m + math.log(z)
            o[i, h] = (e / z) @ vv[:, h // g, :]
    return f64_to_bf16(o), lse.astype(np.float32)


def sink_scale(o_bf16: np.ndarray, lse: np.ndarray, sinks_bf16: np.ndarray) -> np.ndarray:
    """o * bf16(sigmoid(lse - sink)) (attention.py:235-245), bf16 out."""
    z = lse.astype(np.float64) - bf16_to_f32(sinks_bf16).astype(np.float64)[None, :]
    sig = f64_to_bf16(1.0 / (1.0 + np.exp(-z)))
    return f32_to_bf16((bf16_to_f32(o_bf16) * bf16_to_f32(sig)[..., None]).astype(np.float32))


# ---------------------------------------------------------------------------
# The block (attention.py:182-256)
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class AttnParams:
    """AttentionBlock parameters (attention.py:77-92), bf16 bits."""
    sinks: np.ndarray    # [Hq]
    norm_w: np.ndarray   # [H]
    qkv_w: np.ndarray    # [D (Hq + 2 Hkv), H]
    qkv_b: np.ndarray    # [D (Hq + 2 Hkv)]
    out_w: np.ndarray    # [H, D Hq]
    out_b: np.ndarray    # [H]


def split_qkv(qkv_bf16: np.ndarray, hq: int = N_Q_HEADS, hkv: int = N_KV_HEADS, d: int = HEAD_DIM):
    """attention.py:206-210: [n, (Hq + 2 Hkv) D] -> q [n, Hq, D], k, v [n, Hkv, D]."""
    x = qkv_bf16.reshape(qkv_bf16.shape[0], hq + 2 * hkv, d)
    return x[:, :hq], x[:, hq:hq + hkv], x[:, hq + hkv:]


def attn_block_forward(x_bf16: np.ndarray, p: AttnParams, k_cache: np.ndarray, v_cache: np.ndarray,
                       window: int, eps: float = 1e-5):
    """One AttentionBlock call on one sequence.

    x [n, H] holds the tokens at positions P .. P + n - 1, where P = len(k_cache)
    (the tokens already cached).  k_cache / v_cache [P, Hkv, D] bf16 hold the
    rotated keys and the values of positions 0 .. P-1.  n > 1 with P = 0 is the
    reference's "prefill" (self-attention over the chunk), n = 1 its "decode"
    (cross-attention over the cache, which then holds the new token), P > 0 with
    n > 1 its "extend" (attention over the cached prefix and the chunk).
    Returns (out [n, H] bf16, k_new, v_new [n, Hkv, D]).
    """
    n = x_bf16.shape[0]
    P = k_cache.shape[0]
    hq = p.sinks.shape[0]
    d = HEAD_DIM
    hkv = (p.qkv_w.shape[0] // d - hq) // 2
    t = rms_norm(x_bf16, p.norm_w, eps)
    qkv = linear(t, p.qkv_w, p.qkv_b)
    q, k, v = split_qkv(qkv, hq, hkv, d)
    pos = np.arange(P, P + n)
    q = rope(q, pos)
    k = rope(k, pos)
    kk = np.concatenate([k_cache.reshape(P, hkv, d), k], axis=0)
    vv = np.concatenate([v_cache.reshape(P, hkv, d), v], axis=0)
    o, lse = attention(q, kk, vv, pos, window)
    o = sink_scale(o, lse, p.sinks)
    y = linear(o.reshape(n, hq * d), p.out_w, p.out_b)
    out = f32_to_bf16(bf16_to_f32(x_bf16) + bf16_to_f32(y))
    return out, k, v


def _bf16_normal(rng, shape, std):
    return f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def make_attn_params(seed: int, hidden: int = 2880, hq: int = N_Q_HEADS, hkv: int = N_KV_HEADS,
                     d: int = HEAD_DIM) -> AttnParams:
    """Synthetic AttentionBlock parameters from PCG64(seed): sinks N(0, 1),
    unit norm weight, qkv / out weights N(0, 0.02), biases N(0, 0.01)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    qkv_dim = d * (hq + 2 * hkv)
    return AttnParams(
        sinks=_bf16_normal(rng, (hq,), 1.0),
        norm_w=f32_to_bf16(np.ones(hidden, dtype=np.float32)),
        qkv_w=_bf16_normal(rng, (qkv_dim, hidden), 0.02),
        qkv_b=_bf16_normal(rng, (qkv_dim,), 0.01),
        out_w=_bf16_normal(rng, (hidden, hq * d), 0.02),
        out_b=_bf16_normal(rng, (hidden,), 0.01),
    )


# ---------------------------------------------------------------------------
# Sampling: TVM vm.builtin.sample_top_p_from_logits (engine.py:39-40,165-167)
# ---------------------------------------------------------------------------

def sample_top_p_from_logits(logits: np.ndarray, temperature: float, top_p: float,
                             uniform_sample: float) -> int:
    """TVM's SampleTopPFromLogits, restated: sort descending by logit; argmax
    if temperature < 1e-6; else e = exp((l - max) * (1 / T)) and
    probabilities p = e / sum(e); the first maximum if uniform_sample <
    p_max / top_p (SampleTopPFromProb's short cut, taken before any sum); else
    the probabilities accumulated in sorted order, the top-p mass = the running
    sum up to and including the element before which it was still below
    top_p, and the first element whose cumulative probability over the top-p
    mass exceeds uniform_sample is returned (the first maximum otherwise).

    Canonical numerics: the exponent's argument in fp32 as written, exp
    rounded once to fp32 (through fp64), and the sums exact (fp64).  TVM adds
    the fp32 values serially, in an order not observable here, which over the
    201088-entry vocabulary carries a relative error near 1e-3 -- enough to
    move the chosen element by a rank or so; the exact sums are this build's
    definition.  Equal logits are taken in index order."""
    l = np.asarray(logits, dtype=np.float32).reshape(-1)
    order = np.argsort(-l, kind="stable")
    ls = l[order]
    if temperature < 1e-6:
        return int(order[0])
    scale = np.float32(1.0 / temperature)
    arg = ((ls - ls[0]) * scale).astype(np.float32)
    e = np.exp(arg.astype(np.float64)).astype(np.float32).astype(np.float64)
    total = e.sum()
    u32, tp32 = float(np.float32(uniform_sample)), float(np.float32(top_p))
    if u32 < (1.0 / total) / tp32:          # e[0] = exp(0) = 1: p_max = 1 / total
        return int(order[0])
    cums = np.cumsum(e) / total
    before = np.concatenate([[0.0], cums[:-1]])
    top = cums[np.nonzero(before < tp32)[0][-1]]
    hit = np.nonzero(u32 < cums / top)[0]
    return int(order[hit[0]] if hit.size else order[0])


# ---------------------------------------------------------------------------
# The decode loop's model (model/transformer.py:13-133)
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class ModelParams:
    """GPTOssForCausalLM parameters (bf16 bits / MXFP4 bytes)."""
    embedding: np.ndarray     # [V, H]
    layers: list              # [(AttnParams, moe_oracle.BlockParams)]
    norm_w: np.ndarray        # [H]
    unembedding: np.ndarray   # [V, H]


def make_model_params(seed: int, layers: int, vocab: int, hidden: int = 2880,
                      experts: int = 32, inter: int = 2880) -> ModelParams:
    """Per-layer seeds seed + 100 i (attention) and seed + 100 i + 1 (MoE);
    embedding and unembedding N(0, 1) and N(0, 0.02) from seed - 1."""
    from oracle.moe_oracle import make_params
    rng = np.random.Generator(np.random.PCG64(seed - 1))
    emb = _bf16_normal(rng, (vocab, hidden), 1.0)
    unemb = _bf16_normal(rng, (vocab, hidden), 0.02)
    lay = [(make_attn_params(seed + 100 * i, hidden=hidden),
            make_params(seed + 100 * i + 1, num_experts=experts, hidden=hidden, inter=inter))
           for i in range(layers)]
    return ModelParams(emb, lay, f32_to_bf16(np.ones(hidden, dtype=np.float32)), unemb)


class OracleModel:
    """Teacher-forced forward of one sequence: ``forward(ids)`` appends the
    tokens to this object's per-layer caches and returns the fp32 logits
    (bf16 values) of every appended token.  Even layers use the sliding
    window (model/attention.py:87; the engine enables it for each sequence,
    engine.py:116-125)."""

    def __init__(self, p: ModelParams, window: int = SLIDING_WINDOW, k: int = 4,
                 eps: float = 1e-5):
        self.p, self.window, self.k, self.eps = p, window, k, eps
        empty = np.zeros((0, N_KV_HEADS, HEAD_DIM), dtype=np.uint16)
        self.kc = [empty.copy() for _ in p.layers]
        self.vc = [empty.copy() for _ in p.layers]

    def forward(self, ids) -> np.ndarray:
        from oracle.moe_oracle import block_forward
        x = self.p.embedding[np.asarray(ids, dtype=np.int64)]
        for i, (ap, mp) in enumerate(self.p.layers):
            w = self.window if i % 2 == 0 else 0
            x, k, v = attn_block_forward(x, ap, self.kc[i], self.vc[i], w, self.eps)
            self.kc[i] = np.concatenate([self.kc[i], k])
            self.vc[i] = np.concatenate([self.vc[i], v])
            x = block_forward(x, mp, self.k, self.eps).out
        h = rms_norm(x, self.p.norm_w, self.eps)
        self.hidden = h  # final hidden state (bf16 bits) of the appended tokens
        return self.logits(h)

    def logits(self, h_bf16: np.ndarray) -> np.ndarray:
        """fp32 logits (bf16 values) of final hidden states (model/transformer.py:95-100)."""
        return bf16_to_f32(linear(h_bf16, self.p.unembedding, None))
