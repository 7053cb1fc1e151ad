"""Pins of the CPU oracle (oracle/moe_oracle.py, oracle/moe_ref.c).

The reference ships no tests, fixtures or golden vectors, and its TVM/mlc-llm
dependencies are absent, so each oracle function is pinned here against an
independent derivation: the e2m1/E8M0 bit definitions, exact rational
arithmetic, brute force on tiny inputs, closed forms at the clamps, and
invariants -- chosen so that a dropped term, a wrong index or a transposed
operand fails at least one test.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import moe_oracle as O


# ---------------------------------------------------------------------------
# A1 / A12 dequantisation
# ---------------------------------------------------------------------------

def _e2m1_from_bits(c: int) -> float:
    """OCP MX e2m1: 1 sign, 2 exponent (bias 1), 1 mantissa bit; exponent 0 is subnormal."""
    sign = -1.0 if c & 8 else 1.0
    e, m = (c >> 1) & 3, c & 1
    mag = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
    return sign * mag


def test_fp4_lut_matches_e2m1_bits():
    for c in range(16):
        v = _e2m1_from_bits(c)
        assert O.FP4_VALUES[c] == v
        assert math.copysign(1.0, O.FP4_VALUES[c]) == math.copysign(1.0, v)  # -0.0 at code 8


def test_e8m0_matches_torch_float8_e8m0fnu():
    torch = pytest.importorskip("torch")
    s = np.arange(255, dtype=np.uint8)
    ref = torch.from_numpy(s).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(O.e8m0_to_f32(s), ref)
    # the reference's exp2(255 - 127) is +inf where OCP/torch give NaN
    assert O.e8m0_to_f32(np.array([255], np.uint8))[0] == np.inf
    assert O.e8m0_to_f32(np.array([0], np.uint8))[0] == np.float32(2.0 ** -127)


def _bf16_exact(v: float) -> int:
    """bf16 bits of a value that bf16 represents exactly (or +-inf / NaN)."""
    if math.isnan(v):
        return 0x7FC0
    f = np.array([v], dtype=np.float32)
    assert math.isinf(v) or float(f[0]) == v
    u = int(f.view(np.uint32)[0])
    assert u & 0xFFFF == 0
    return u >> 16


def dequant_table_exact() -> np.ndarray:
    """[256 scales, 16 codes] bf16 bits of e2m1(c) * 2^(s-127), from exact arithmetic.

    Every product is a value with <= 2 significant bits times a power of two,
    so it is exactly representable in bf16 (subnormals included) unless it
    exceeds the bf16/fp32 range, where fp32 overflows to inf; s = 255 is
    exp2(128) = inf, and 0 * inf is NaN.
    """
    tab = np.zeros((256, 16), dtype=np.uint16)
    for s in range(256):
        for c in range(16):
            lut = _e2m1_from_bits(c)
            if s == 255:
                v = math.nan if lut == 0 else math.copysign(math.inf, lut)
            else:
                exact = Fraction(lut) * Fraction(2) ** (s - 127)
                v = float(exact) if abs(exact) < Fraction(2) ** 128 else math.copysign(math.inf, lut)
                if lut == 0:
                    v = math.copysign(0.0, lut)
            tab[s, c] = _bf16_exact(v)
    return tab


def test_dequant_exhaustive_256x256():
    tab = dequant_table_exact()
    blocks = np.broadcast_to(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 16, 16)).copy()
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)          # [256, 16]
    out = O.dequant_mxfp4(blocks, scales)                                              # [256,16,32]
    byte = blocks.astype(np.int64)
    exp_lo = tab[np.arange(256)[:, None, None], byte & 15]
    exp_hi = tab[np.arange(256)[:, None, None], byte >> 4]
    nan_out = (out & 0x7FFF) > 0x7F80
    nan_lo = (exp_lo & 0x7FFF) > 0x7F80
    nan_hi = (exp_hi & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_out[..., 0::2], nan_lo) and np.array_equal(nan_out[..., 1::2], nan_hi)
    assert np.array_equal(np.where(nan_lo, 0, out[..., 0::2]), np.where(nan_lo, 0, exp_lo))
    assert np.array_equal(np.where(nan_hi, 0, out[..., 1::2]), np.where(nan_hi, 0, exp_hi))


def test_dequant_weight_element_order():
    """in_idx = 32*g + 2*byte + nibble, nibble 0 = low 4 bits (model/mlp.py:289-303)."""
    for g, byte, hi in [(0, 0, 0), (0, 0, 1), (1, 5, 0), (2, 15, 1)]:
        blocks = np.zeros((1, 3, 16), np.uint8)
        blocks[0, g, byte] = (2 << 4) if hi else 2   # code 2 = 1.0
        scales = np.full((1, 3), 127, np.uint8)
        w = O.dequant_weight_f64(blocks, scales)
        nz = np.flatnonzero(w[0])
        assert list(nz) == [32 * g + 2 * byte + hi]
        assert w[0, nz[0]] == 1.0


# ---------------------------------------------------------------------------
# A3-A5 norm, router, top-k, softmax
# ---------------------------------------------------------------------------

def _bf(vals):
    return O.f32_to_bf16(np.asarray(vals, dtype=np.float32))


def test_rmsnorm_against_exact_and_eps():
    # small H so a wrong mean denominator or a dropped eps moves the result by many ulps
    x = np.array([[0.5, -1.25, 2.0, 0.0, 3.0, -0.75, 1.5, 0.25],
                  [1e-3, -1e-3, 2e-3, 0, 0, 1e-3, 0, 0]], dtype=np.float32)
    xb = _bf(x)
    w = _bf([1, 2, 0.5, 1, 1, -1, 1, 3])
    t = O.bf16_to_f32(O.rms_norm(xb, w, 1e-5))
    xf, wf = O.bf16_to_f32(xb).astype(np.float64), O.bf16_to_f32(w).astype(np.float64)
    for i in range(2):
        ms = sum(Fraction(float(v)) ** 2 for v in xf[i]) / 8 + Fraction(float(np.float32(1e-5)))
        r = 1.0 / math.sqrt(float(ms))
        exact = xf[i] * r * wf
        ulp = np.maximum(np.abs(exact), 1e-30) * 2 ** -7
        assert np.all(np.abs(t[i] - exact) <= ulp), (t[i], exact)
    # x = 0 stays 0 (eps keeps the rsqrt finite)
    z = O.rms_norm(np.zeros((1, 8), np.uint16), w, 1e-5)
    assert np.all(O.bf16_to_f32(z) == 0)


def test_router_known_answer_double_rounding():
    # t = one-hot -> dot = W[e, i] exactly; W = 1, b = 2^-8: 1 + 2^-8 ties to 1.0 (even)
    H, E = 16, 3
    t = np.zeros((1, H), np.uint16)
    t[0, 5] = _bf([1.0])[0]
    W = np.zeros((E, H), np.float32)
    W[:, 5] = [1.0, 3.0, -2.0]
    b = np.array([2.0 ** -8, 2.0 ** -6, 0.5], np.float32)
    g = O.bf16_to_f32(O.router_logits(t, _bf(W), _bf(b)))
    assert list(g[0]) == [1.0, 3.0 + 2.0 ** -6, -1.5]  # 3 + 2^-6 is a bf16 (ulp 2^-6 in [2,4))


def test_router_matches_exact_dot():
    rng = np.random.default_rng(3)
    H, E = 64, 8
    t = _bf(rng.standard_normal((4, H)))
    W = _bf(rng.standard_normal((E, H)) * 0.02)
    b = _bf(rng.standard_normal(E) * 0.01)
    g = O.router_logits(t, W, b)
    tf, wf, bf = O.bf16_to_f32(t), O.bf16_to_f32(W), O.bf16_to_f32(b)
    for s in range(4):
        for e in range(E):
            dot = sum(Fraction(float(a)) * Fraction(float(c)) for a, c in zip(tf[s], wf[e]))
            d16 = O.f32_to_bf16(np.float32(float(dot)))        # exact -> fp64 -> fp32 -> bf16
            expect = O.f32_to_bf16(np.float32(O.bf16_to_f32(d16) + bf[e]))
            assert g[s, e] == expect


def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(5)
    for _ in range(200):
        E, k = 6, 4
        g = _bf(rng.integers(-3, 4, size=(1, E)).astype(np.float32) * 0.5)  # many ties
        w, idx = O.topk_softmax(g, k)
        gf = O.bf16_to_f32(g)[0]
        expect = sorted(range(E), key=lambda e: (-gf[e], e))[:k]
        assert list(idx[0]) == expect


def test_softmax_closed_forms():
    g = _bf([[2.0, 2.0, 2.0, 2.0, -5.0]])
    w, idx = O.topk_softmax(g, 4)
    assert list(idx[0]) == [0, 1, 2, 3]
    assert np.all(O.bf16_to_f32(w) == 0.25)
    g = _bf([[0.0, 1.0, 0.0, 0.0, 0.0, -1.0]])
    w, idx = O.topk_softmax(g, 4)
    assert list(idx[0]) == [1, 0, 2, 3]
    e = math.e
    expect = [e / (e + 3), 1 / (e + 3), 1 / (e + 3), 1 / (e + 3)]
    assert np.array_equal(w[0], O.f32_to_bf16(np.float32(expect)))


def test_softmax_invariants_random():
    rng = np.random.default_rng(7)
    g = _bf(rng.standard_normal((500, 32)) * 0.3)
    w, idx = O.topk_softmax(g, 4)
    wf = O.bf16_to_f32(w).astype(np.float64)
    assert np.all(np.abs(wf.sum(1) - 1.0) <= 4 * 2 ** -8)
    assert np.all(np.diff(wf, axis=1) <= 0)
    assert all(len(set(r)) == 4 for r in idx)


# ---------------------------------------------------------------------------
# A6 grouping
# ---------------------------------------------------------------------------

def test_permute_brute_force_and_invariants():
    rng = np.random.default_rng(11)
    for n, k, E in [(1, 4, 32), (37, 4, 8), (200, 2, 5), (0, 4, 4)]:
        rows = [rng.permutation(E)[:k] for _ in range(n)]
        idx = np.array(rows, dtype=np.int32).reshape(n, k)
        P = O.permute(idx, E)
        flat = idx.reshape(-1)
        order = [p for e in range(E) for p in range(n * k) if flat[p] == e]
        assert list(P.sorted_pairs) == order
        assert P.indptr[0] == 0 and P.indptr[-1] == n * k and np.all(np.diff(P.indptr) >= 0)
        for e in range(E):
            seg = P.sorted_pairs[P.indptr[e]:P.indptr[e + 1]]
            assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)
            assert np.all(P.expert_ids[P.indptr[e]:P.indptr[e + 1]] == e)
        assert np.array_equal(P.token_indices, P.sorted_pairs // k)
        assert np.array_equal(P.sorted_pairs[P.pair_pos], np.arange(n * k))


# ---------------------------------------------------------------------------
# A7-A11 expert matmuls, SwiGLU, gating, residual
# ---------------------------------------------------------------------------

def _tiny_weights(rng, E, N, K):
    blocks = rng.integers(0, 256, (E, N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(118, 123, (E, N, K // 32), dtype=np.uint8)
    bias = _bf(rng.standard_normal((E, N)) * 0.01)
    return blocks, scales, bias


def _serial_einsum_py(x, idx, blocks, scales, bias):
    """Pure-Python transcription of the TIR loop nest, model/mlp.py:281-319, in fp32."""
    n, k = idx.shape
    E, N, G, _ = blocks.shape
    out = np.zeros((n, k, N), np.float32)
    lut = O.FP4_VALUES
    for s in range(n):
        for r in range(k):
            e = idx[s, r]
            for c in range(N):
                acc = np.float32(O.bf16_to_f32(bias[e, c]))
                for i in range(G * 32):
                    g, loc = divmod(i, 32)
                    byte, hi = divmod(loc, 2)
                    sc = np.float32(2.0) ** np.float32(int(scales[e, c, g]) - 127)
                    nib = (int(blocks[e, c, g, byte]) >> (4 * hi)) & 15
                    xv = x[s, r, i] if x.ndim == 3 else x[s, i]
                    acc = np.float32(acc + np.float32(np.float32(xv * lut[nib]) * sc))
                out[s, r, c] = acc
    return out


def test_einsum_serial_c_matches_python_loop(oracle_lib):
    rng = np.random.default_rng(13)
    E, N, K, n, k = 3, 4, 64, 2, 2
    blocks, scales, bias = _tiny_weights(rng, E, N, K)
    idx = np.array([[0, 2], [1, 0]], np.int32)
    x2 = O.bf16_to_f32(_bf(rng.standard_normal((n, K))))
    x3 = rng.standard_normal((n, k, K)).astype(np.float32)
    for x in (x2, x3):
        ref = _serial_einsum_py(x, idx, blocks, scales, bias)
        assert np.array_equal(oracle_lib.einsum(x, idx, blocks, scales, bias), ref)
        np.testing.assert_allclose(O.einsum_fused(x, idx, blocks, scales, bias), ref,
                                   rtol=0, atol=1e-5 * np.abs(ref).max())


def test_einsum_one_hot_known_answer():
    rng = np.random.default_rng(17)
    E, N, K = 2, 8, 96
    blocks, scales, bias = _tiny_weights(rng, E, N, K)
    idx = np.array([[1, 0]], np.int32)
    for i in (0, 33, 95):
        x = np.zeros((1, K), np.float32)
        x[0, i] = 1.0
        out = O.einsum_fused(x, idx, blocks, scales, bias)
        for r, e in enumerate(idx[0]):
            deq = O.bf16_to_f32(O.dequant_mxfp4(blocks[e], scales[e]).reshape(N, K))[:, i]
            expect = (O.bf16_to_f32(bias[e]) + deq).astype(np.float32)
            assert np.array_equal(out[0, r], expect)


def test_einsum_linearity():
    rng = np.random.default_rng(19)
    E, N, K = 2, 16, 64
    blocks, scales, bias = _tiny_weights(rng, E, N, K)
    idx = np.array([[0, 1], [1, 0]], np.int32)
    x1 = rng.standard_normal((2, K)).astype(np.float32)
    x2 = rng.standard_normal((2, K)).astype(np.float32)
    zero_b = np.zeros_like(bias)
    lhs = O.einsum_fused(x1 + x2, idx, blocks, scales, zero_b)
    rhs = O.einsum_fused(x1, idx, blocks, scales, zero_b) + O.einsum_fused(x2, idx, blocks, scales, zero_b)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-5, atol=1e-5 * np.abs(lhs).max())


def test_swiglu_closed_forms(oracle_lib):
    a = 1.702
    # z = alpha * glu is formed in fp32 (alpha is an fp32 constant, model/mlp.py:50)
    sig = lambda z: 1 / (1 + math.exp(-float(np.float32(z / a) * np.float32(a))))
    cases = [  # (glu, lin, expected)
        (0.0, 3.0, 0.0),
        (2.0, -1.0, 0.0),                                  # (lin + 1) = 0
        (8.0, 0.0, 7.0 * sig(a * 7.0)),                    # glu clamped above at 7
        (7.0, 10.0, 7.0 * sig(a * 7.0) * 8.0),             # lin clamped at +7
        (1.0, -9.0, 1.0 * sig(a) * -6.0),                  # lin clamped at -7
        (-20.0, 0.0, -20.0 * sig(-a * 20.0)),              # no lower clamp on glu
    ]
    x = np.array([[g, l] for g, l, _ in cases], np.float32).reshape(1, -1)
    out = O.swiglu(x)[0]
    c_out = oracle_lib.swiglu(x)[0]
    for (g, l, e), o, co in zip(cases, out, c_out):
        assert o == pytest.approx(e, rel=4e-7, abs=1e-30)
        assert o == co
    # even features are the gate, odd the linear part
    assert O.swiglu(np.array([[0.0, 5.0]], np.float32))[0, 0] == 0.0


def test_gating_and_residual_closed_forms(oracle_lib):
    y = np.array([[[1.5, -2.0], [3.0, 7.0], [0.25, 1.0], [9.0, 9.0]]], np.float32)  # [1, 4, 2]
    w = _bf([[1.0, 0.0, 0.0, 0.0]])
    assert np.array_equal(O.gating(y, w), _bf([[1.5, -2.0]]))
    w = _bf([[0.5, 0.25, 0.0, 0.125]])
    exp = [1.5 * 0.5 + 3.0 * 0.25 + 9.0 * 0.125, -2.0 * 0.5 + 7.0 * 0.25 + 9.0 * 0.125]
    assert np.array_equal(O.gating(y, w), _bf([exp]))
    assert np.array_equal(oracle_lib.gating(y, w), O.gating(y, w))
    # residual: 1 + 2^-8 ties to 1.0; 1 + 3*2^-8 rounds up to 1 + 2^-6
    x = _bf([[1.0, 1.0]])
    t = _bf([[2.0 ** -8, 3 * 2.0 ** -8]])
    assert list(O.bf16_to_f32(O.residual_add(x, t))[0]) == [1.0, 1.0 + 2.0 ** -6]


# ---------------------------------------------------------------------------
# whole block: numpy oracle vs the serial C restatement
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("E,H,I,n", [(8, 128, 96, 7), (4, 64, 64, 3), (32, 256, 128, 40)])
def test_block_numpy_vs_serial_c(oracle_lib, E, H, I, n):
    p = O.make_params(seed=E + H, num_experts=E, hidden=H, inter=I)
    x = O.make_input(seed=n, n=n, hidden=H)
    tr = O.block_forward(x, p)
    out, t, idx, w = oracle_lib.block_forward(x, p)
    assert np.array_equal(t, tr.t) and np.array_equal(idx, tr.idx) and np.array_equal(w, tr.w)
    m = O.compare_outputs(out, tr.out)
    assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m


def test_block_full_shape_two_tokens(oracle_lib):
    p = O.make_params(seed=0)
    x = O.make_input(seed=1, n=2)
    tr = O.block_forward(x, p)
    out, t, idx, w = oracle_lib.block_forward(x, p)
    assert np.array_equal(t, tr.t) and np.array_equal(idx, tr.idx) and np.array_equal(w, tr.w)
    m = O.compare_outputs(out, tr.out)
    assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m


def test_synthetic_distributions():
    p = O.make_params(seed=0, num_experts=4, hidden=64, inter=64)
    s = np.concatenate([p.mlp1_scales.ravel(), p.mlp2_scales.ravel()])
    assert s.min() >= 118 and s.max() <= 122
    nib = np.concatenate([p.mlp1_blocks.ravel() & 15, p.mlp1_blocks.ravel() >> 4])
    assert set(np.unique(nib)) == set(range(16))
    assert np.all(O.bf16_to_f32(p.norm_w) == 1.0)


def test_zipf_bias_skews_load():
    p = O.make_params(seed=0, num_experts=32, hidden=256, inter=64, zipf_beta=0.5)
    x = O.make_input(seed=2, n=1024, hidden=256)
    t = O.rms_norm(x, p.norm_w)
    g = O.router_logits(t, p.gate_w, p.gate_b)
    _, idx = O.topk_softmax(g, 4)
    counts = np.bincount(idx.ravel(), minlength=32)
    assert counts.max() / counts.mean() > 2.5


def test_algorithmic_bytes_per_expert():
    # 13,236,480 bytes per 20B-shape expert (blocks, scales, biases of mlp1 and mlp2)
    assert O.algorithmic_bytes(0, 1, num_experts=0) - 2 * 2880 == 13_236_480
