"""Pins of the attention / decode-loop oracle (oracle/attn_oracle.py), CPU only.

The reference holds no golden vectors for attention, so each function is
checked against what the mathematics fixes, computed by an independent route:
the YaRN correction range and ramp from their closed forms, RoPE against
complex multiplication, attention against a brute-force loop and one-hot
values, the sink scaling against a softmax with an extra sink logit, the
sampler against a literal serial loop, and the block against its own cache
consistency (decode after prefill = prefill of the longer sequence).
"""
import math

import numpy as np
import pytest

from oracle import attn_oracle as A
from oracle import moe_oracle as O


def bf(x):
    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def f(b):
    return O.bf16_to_f32(b).astype(np.float64)


def test_yarn_correction_range_closed_form():
    # dim(r) = 64 ln(4096 / (2 pi r)) / (2 ln 150000): r = 32 -> low, r = 1 -> high
    low, high = A.yarn_correction_range()
    assert abs(float(low) - 64 * math.log(4096 / (64 * math.pi)) / (2 * math.log(150000))) < 1e-5
    assert abs(float(high) - 64 * math.log(4096 / (2 * math.pi)) / (2 * math.log(150000))) < 1e-5
    assert 8 < low < 9 and 17 < high < 18


def test_yarn_inv_freq_regions():
    inv = A.yarn_inv_freq().astype(np.float64)
    low, high = (float(v) for v in A.yarn_correction_range())
    for d in range(32):
        base = 150000.0 ** (-2 * d / 64)
        ramp = min(max((d - low) / (high - low), 0.0), 1.0)
        want = base / 32 * ramp + base * (1 - ramp)   # extrapolated below low, interpolated above
        assert abs(inv[d] - want) <= 2e-6 * want, d
    assert inv[0] == 1.0
    assert np.all(np.diff(inv) < 0)
    assert float(A.yarn_concentration()) == pytest.approx(1 + 0.1 * math.log(32), rel=1e-7)


def test_rope_is_a_scaled_rotation():
    rng = np.random.default_rng(1)
    n, heads = 6, 3
    x = bf(rng.standard_normal((n, heads, 64)))
    pos = np.array([0, 1, 7, 100, 4095, 70000])
    out = f(A.rope(x, pos))
    inv = A.yarn_inv_freq().astype(np.float64)
    conc = float(A.yarn_concentration())
    for i, p in enumerate(pos):
        ang = np.float32(p) * A.yarn_inv_freq()          # fp32 angle, as stated
        c = f(bf(np.cos(ang.astype(np.float64)))) * conc
        s = f(bf(np.sin(ang.astype(np.float64)))) * conc
        z = (f(x[i, :, :32]) + 1j * f(x[i, :, 32:])) * (c + 1j * s)   # (lo + i hi) e^{i ang}
        np.testing.assert_allclose(out[i, :, :32], z.real, rtol=8e-3, atol=1e-6)
        np.testing.assert_allclose(out[i, :, 32:], z.imag, rtol=8e-3, atol=1e-6)
    # position 0: no rotation, only the concentration
    np.testing.assert_array_equal(A.rope(x[:1], np.array([0])), bf(f(x[:1]) * np.float32(conc)))
    assert inv.shape == (32,)


def test_linear_two_roundings():
    """nn.Linear as two bf16 ops (attention.py:206,254): bf16(bf16(x W^T) + b),
    the products summed exactly.  Closed cases: x W^T = 1 + 2^-8 + 2^-10 rounds
    to 1 + 2^-7 (above the midpoint 1 + 2^-8); adding b = 2^-8 lands exactly on
    the midpoint between 1 + 2^-7 and 1 + 2^-6, which ties to the even 1 + 2^-6
    -- one rounding of the exact 1 + 2^-7 + 2^-10 would give 1 + 2^-7.  And
    [2^24, 1, -2^24] . [1, 1, 1] = 1 exactly, which an fp32 running sum (2^24 + 1
    = 2^24) would lose."""
    x = bf(np.array([[1.0, 2.0 ** -8, 2.0 ** -10], [2.0 ** 24, 1.0, -2.0 ** 24]]))
    w = bf(np.array([[1.0, 1.0, 1.0]]))
    y = f(A.linear(x, w, None)).ravel()
    assert y[0] == 1.0 + 2.0 ** -7 and y[1] == 1.0
    yb = f(A.linear(x[:1], w, bf(np.array([2.0 ** -8])))).ravel()
    assert yb[0] == 1.0 + 2.0 ** -6
    yn = f(A.linear(bf(-f(x[:1])), w, bf(np.array([-2.0 ** -8])))).ravel()
    assert yn[0] == -(1.0 + 2.0 ** -6)  # ties to even in magnitude for either sign


def _brute_attention(q, k, v, qpos, window, scale):
    n, hq, d = q.shape
    L, hkv, _ = k.shape
    o = np.zeros((n, hq, d))
    lse = np.zeros((n, hq))
    for i in range(n):
        for h in range(hq):
            ks = [j for j in range(L) if j <= qpos[i] and (window <= 0 or j > qpos[i] - window)]
            sc = [sum(q[i, h, e] * k[j, h * hkv // hq, e] for e in range(d)) * scale for j in ks]
            mx = max(sc)
            z = sum(math.exp(s - mx) for s in sc)
            lse[i, h] = mx + math.log(z)
            for j, s in zip(ks, sc):
                o[i, h] += math.exp(s - mx) / z * v[j, h * hkv // hq]
    return o, lse


@pytest.mark.parametrize("window", [0, 3])
def test_attention_brute_force(window):
    rng = np.random.default_rng(3)
    n, L, hq, hkv, d = 4, 9, 4, 2, 8
    q = bf(rng.standard_normal((n, hq, d)))
    k = bf(rng.standard_normal((L, hkv, d)))
    v = bf(rng.standard_normal((L, hkv, d)))
    qpos = np.array([5, 6, 7, 8])
    o, lse = A.attention(q, k, v, qpos, window, sm_scale=0.3)
    ro, rl = _brute_attention(f(q), f(k), f(v), qpos, window, 0.3)
    np.testing.assert_allclose(lse, rl, rtol=1e-6)
    np.testing.assert_allclose(f(o), ro, rtol=8e-3, atol=1e-6)


def test_attention_mask_with_one_hot_values():
    # q = 0: equal scores, so o = mean of the attended one-hot values -> the mask itself
    L, window = 10, 4
    q = bf(np.zeros((L, 1, 16)))
    k = bf(np.ones((L, 1, 16)))
    v = bf(np.eye(L, 16)[:, None, :])
    o, lse = A.attention(q, k, v, np.arange(L), window)
    for p in range(L):
        att = [j for j in range(L) if p - window < j <= p]
        want = np.zeros(16)
        want[att] = 1.0 / len(att)
        np.testing.assert_allclose(f(o[p, 0]), want, rtol=4e-3)
        assert lse[p, 0] == pytest.approx(math.log(len(att)), abs=1e-6)
    assert A.allowed(5, 10, 0).sum() == 6 and A.allowed(5, 10, 2).tolist()[4:6] == [True, True]


def test_sink_equals_extra_softmax_logit():
    rng = np.random.default_rng(4)
    L, d = 7, 8
    s = rng.standard_normal(L)
    vals = rng.standard_normal((L, d))
    sink = 0.7
    e = np.exp(s)
    want = (e / (e.sum() + math.exp(sink))) @ vals        # the sink as a logit with zero value
    o = bf(((e / e.sum()) @ vals)[None, None, :])
    lse = np.array([[math.log(e.sum())]], dtype=np.float32)
    got = f(A.sink_scale(o, lse, bf([sink])))[0, 0]
    np.testing.assert_allclose(got, want, rtol=1.2e-2, atol=1e-3)


def _serial_sampler(logits, temperature, top_p, u):
    """Literal loop of the sampler in Python floats (fp64), the argument of
    exp in fp32 as written and exp rounded to fp32."""
    idx = sorted(range(len(logits)), key=lambda i: (-float(logits[i]), i))
    if temperature < 1e-6:
        return idx[0]
    mx = np.float32(logits[idx[0]])
    scale = np.float32(1.0 / temperature)
    ex = [float(np.float32(math.exp(float(np.float32((np.float32(logits[i]) - mx) * scale)))))
          for i in idx]
    total = math.fsum(ex)
    probs = [v / total for v in ex]
    u, top_p = float(np.float32(u)), float(np.float32(top_p))
    if u < probs[0] / top_p:            # SampleTopPFromProb's short cut
        return idx[0]
    cum, top, cums = 0.0, 0.0, []
    for p in probs:
        if cum < top_p:
            top += p
        else:
            break
        cum += p
        cums.append(cum)
    for i, c in zip(idx, cums):
        if u < c / top:
            return i
    return idx[0]


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("temperature,top_p,u", [(0.7, 0.9, 0.5), (1.0, 1.0, 0.99), (0.3, 0.5, 0.1)])
def test_sampler_matches_serial_loop(seed, temperature, top_p, u):
    rng = np.random.default_rng(seed)
    logits = f(bf(rng.standard_normal(500) * 3)).astype(np.float32)   # bf16 values: ties occur
    assert A.sample_top_p_from_logits(logits, temperature, top_p, u) == \
        _serial_sampler(logits, temperature, top_p, u)


def test_sampler_closed_cases():
    logits = np.array([0.0, 3.0, 3.0, 1.0], dtype=np.float32)
    assert A.sample_top_p_from_logits(logits, 0.0, 0.9, 0.5) == 1          # argmax, lower index
    assert A.sample_top_p_from_logits(logits, 1.0, 0.9, 0.0) == 1          # first of the ties
    # two tied leaders hold most of the mass: u just past the first's share picks the second
    e = np.exp(logits - 3.0)
    p = e / e.sum()
    top = p[1] + p[2]
    assert p[1] < 0.9 <= top          # the running sum reaches top_p at the second leader
    # past both the first leader's share of the top-p mass and p_max / top_p
    cut = max(float(p[1] / top), float(p[1] / 0.9))
    assert A.sample_top_p_from_logits(logits, 1.0, 0.9, cut + 1e-3) == 2
    assert A.sample_top_p_from_logits(logits, 1.0, 0.9, float(p[1] / top) - 1e-3) == 1


def test_sampler_short_cut_to_argmax():
    """TVM's SampleTopPFromProb returns the argmax when uniform < p_max /
    top_p, before it forms the top-p mass.  Here p_max is about 0.47 and the
    top-p mass is the whole mass: at the engine's u = 0.5 and top_p = 0.9,
    u < 0.47 / 0.9 = 0.52 picks the leader, although u exceeds the leader's
    share of the top-p mass (0.47), where the crossing alone would pick the
    second element."""
    logits = np.array([2.0, 1.875, 0.5625], dtype=np.float32)   # bf16 values
    e = np.exp(logits.astype(np.float64) - 2.0)
    p = e / e.sum()
    cums = np.cumsum(p)
    top = cums[np.nonzero(np.concatenate([[0.0], cums[:-1]]) < 0.9)[0][-1]]
    assert 0.45 < p[0] < 0.5 and p[0] / top < 0.5 < p[0] / 0.9
    assert A.sample_top_p_from_logits(logits, 1.0, 0.9, 0.5) == 0
    assert _serial_sampler(logits, 1.0, 0.9, 0.5) == 0
    # above p_max / top_p the crossing decides: the second element
    assert A.sample_top_p_from_logits(logits, 1.0, 0.9, float(p[0] / 0.9) + 1e-3) == 1


def _small_params(seed, H=64):
    return A.make_attn_params(seed, hidden=H)


def test_block_decode_after_prefill_equals_longer_prefill():
    """Cache consistency: prefill n tokens, then decode one more; the decoded
    token's output equals the last row of a prefill of all n + 1 tokens."""
    H, n = 64, 5
    p = _small_params(5, H)
    x = O.make_input(6, n + 1, hidden=H)
    empty = np.zeros((0, A.N_KV_HEADS, A.HEAD_DIM), dtype=np.uint16)
    for window in (0, 3):
        out_all, _, _ = A.attn_block_forward(x, p, empty, empty, window)
        out_pre, k, v = A.attn_block_forward(x[:n], p, empty, empty, window)
        out_dec, _, _ = A.attn_block_forward(x[n:], p, k, v, window)
        np.testing.assert_array_equal(out_pre, out_all[:n])
        np.testing.assert_array_equal(out_dec, out_all[n:])
