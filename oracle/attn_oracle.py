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
* Sampling   TVM's algorithm on fp32 values; sort descending by logit, equal
             logits in index order (the C++ std::sort leaves their order open).
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
    if temperature < 1e-6; else e = expf((l - max) / T) summed in sorted order,
    probabilities e / sum accumulated in sorted order, top_p_sum = the mass of
    the prefix up to and including the element at which the running sum
    reaches top_p, and the first element whose cumulative probability over
    top_p_sum exceeds uniform_sample is returned (the last one otherwise).
    fp32 throughout, serial; equal logits in index order."""
    l = np.asarray(logits, dtype=np.float32).reshape(-1)
    order = np.argsort(-l, kind="stable")
    ls = l[order]
    if temperature < 1e-6:
        return int(order[0])
    scale = np.float32(1.0 / temperature)
    e = np.exp(((ls - ls[0]) * scale).astype(np.float32)).astype(np.float32)
    # np.add.accumulate adds serially in the output dtype: the running fp32
    # sums of the serial loops
    total = np.cumsum(e, dtype=np.float32)[-1]
    prob = (e / total).astype(np.float32)
    cums = np.cumsum(prob, dtype=np.float32)
    # top_p_sum adds the same probabilities in the same order as the running
    # sum, up to and including the first one at which the sum before it is
    # not below top_p
    before = np.concatenate([[np.float32(0.0)], cums[:-1]]).astype(np.float32)
    inside = np.nonzero(before < np.float32(top_p))[0]
    top = cums[inside[-1]]
    u = np.float32(uniform_sample)
    hit = np.nonzero(u < (cums / top).astype(np.float32))[0]
    return int(order[hit[0]] if hit.size else order[0])
