"""CPU oracle for the gpt-oss MXFP4 MoE block -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of the reference MoE block
(brekkylab/gpt-oss-tvm ``model/mlp.py``, the block that ``model/transformer.py:10``
wires in) plus the grouping semantics of its unwired optimized variant
(``model/mlp_optimized.py:112-172``).  It is the checker for the HIP library:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and never as the thing that is measured or shipped.

Numbers are carried as numpy arrays; bf16 tensors are carried as their uint16
bit patterns (numpy has no bf16 dtype).

Canonical numerics (each choice is where TVM's lowering could not be observed,
because tvm / mlc-llm are absent; the choice is applied identically by the GPU
kernels):

* RMSNorm     sum of squares in fp64, r = fp32(1 / sqrt(ss/H + eps)) computed
              in fp64 and rounded once, t = bf16(fp32(fp32(x * r) * w)).
* Router      dot product exact-ish in fp64, rounded fp64 -> fp32 -> bf16 (the
              matmul's bf16 output), then fp32 add of the bias and a second
              bf16 rounding (``nn.Linear`` emits matmul and add as two ops).
* Top-k       descending bf16 logit; on equal logits the lower expert index
              wins (a stable descending sort, as TVM's CPU argsort).
* Softmax     over the k selected bf16 logits, in fp64, rounded fp64 -> fp32
              -> bf16 (a correctly rounded fp32 softmax, then the bf16 output).
* Einsum      exact products (bf16 x e2m1 x 2^s are exact in fp32), summed
              from the bias; this module sums in fp64 and rounds once to fp32,
              the C restatement (``moe_ref.c``) sums serially in fp32 exactly
              in the order of ``mlp.py:289-317``.
* SwiGLU      fp32 ops in the written order, sigmoid correctly rounded.
* Gating      fp32, slot order r = 0..k-1, multiply then add (no FMA), then
              bf16; the residual add is bf16(fp32(x) + fp32(moe)).

Pins: every function here is checked in ``tests/test_oracle.py`` against an
independent derivation (closed forms, brute force on tiny inputs, exact rational
arithmetic, invariants); no reference golden vectors exist (the reference ships
no tests or fixtures).
"""
from __future__ import annotations

import dataclasses

import numpy as np

# e2m1 code -> value; low 3 bits = |code|, bit 3 = sign.  Reference:
# model/mlp.py:9-26 (same table at mlp_optimized.py:21-38, weights.py:15-32).
FP4_VALUES = np.array(
    [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)

SWIGLU_ALPHA = 1.702  # model/mlp.py:29 (alpha default)


# ---------------------------------------------------------------------------
# bf16 <-> fp32 bit helpers
# ---------------------------------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    """Round fp32 values to bf16 (round-to-nearest-even); returns uint16 bits.

    NaN inputs map to a quiet NaN with the input's sign and high payload.
    """
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to fp32 values (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f64_to_bf16(x) -> np.ndarray:
    """fp64 -> fp32 (RNE) -> bf16 (RNE): the rounding of an fp32 kernel output."""
    return f32_to_bf16(np.asarray(x, dtype=np.float64).astype(np.float32))


# ---------------------------------------------------------------------------
# A1 / A12: MXFP4 dequantisation
# ---------------------------------------------------------------------------

def e8m0_to_f32(s) -> np.ndarray:
    """E8M0 scale byte -> fp32 2^(s-127).

    Reference: ``T.exp2(T.cast(scale - 127, "float32"))`` at model/mlp.py:297-298
    (and mlp.py:156,200).  s = 255 gives exp2(128) = +inf (not NaN as in OCP);
    s = 0 gives the fp32 subnormal 2^-127.
    """
    s = np.asarray(s, dtype=np.int64)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), (s - 127).astype(np.int32)).astype(np.float32)


def dequant_mxfp4(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Standalone dequantisation, bf16 output (uint16 bits).

    Reference: ``dequant_mxfp4`` prim_func, model/mlp.py:172-234:
    out[r, 2j] = bf16(LUT[lo(b)] * 2^(s-127)), out[r, 2j+1] = bf16(LUT[hi(b)] * 2^(s-127)),
    the product taken in fp32 (bf16 LUT widened, fp32 scale).

    blocks: uint8 [..., 16]; scales: uint8 [...]  ->  uint16 [..., 32].
    """
    blocks = np.asarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    assert blocks.shape[:-1] == scales.shape and blocks.shape[-1] == 16
    lo = blocks & 0x0F
    hi = blocks >> 4
    sc = e8m0_to_f32(scales)[..., None]
    with np.errstate(invalid="ignore", over="ignore"):
        v_lo = FP4_VALUES[lo] * sc
        v_hi = FP4_VALUES[hi] * sc
    out = np.empty(blocks.shape[:-1] + (32,), dtype=np.float32)
    out[..., 0::2] = v_lo
    out[..., 1::2] = v_hi
    return f32_to_bf16(out)


def dequant_weight_f64(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Exact dequantised weight matrix in fp64: [..., G, 16] u8 + [..., G] u8 -> [..., G*32].

    Element order follows model/mlp.py:289-303: in_idx = 32*g + 2*byte + nibble,
    nibble 0 = low 4 bits.
    """
    blocks = np.asarray(blocks, dtype=np.uint8)
    vals = _BYTE_PAIRS[blocks].reshape(blocks.shape[:-1] + (32,))
    sc = np.ldexp(1.0, np.asarray(scales, dtype=np.int64) - 127)[..., None]
    with np.errstate(invalid="ignore", over="ignore"):
        vals = vals * sc
    return vals.reshape(blocks.shape[:-2] + (blocks.shape[-2] * 32,))


# byte -> (value of low nibble, value of high nibble), fp64
_BYTE_PAIRS = np.stack([FP4_VALUES[np.arange(256) & 0x0F], FP4_VALUES[np.arange(256) >> 4]],
                       axis=-1).astype(np.float64)


# ---------------------------------------------------------------------------
# A3-A5: norm, router, top-k, softmax
# ---------------------------------------------------------------------------

def rms_norm(x_bf16: np.ndarray, w_bf16: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """t = x / sqrt(mean(x^2) + eps) * w, bf16 out.  Reference: model/mlp.py:81-87,375."""
    xf = bf16_to_f32(x_bf16)
    x64 = xf.astype(np.float64)
    h = x64.shape[-1]
    ss = np.einsum("...i,...i->...", x64, x64)
    eps64 = float(np.float32(eps))
    r = (1.0 / np.sqrt(ss / h + eps64)).astype(np.float32)
    xr = (xf * r[..., None]).astype(np.float32)
    return f32_to_bf16(xr * bf16_to_f32(w_bf16))


def router_logits(t_bf16: np.ndarray, gate_w_bf16: np.ndarray, gate_b_bf16: np.ndarray) -> np.ndarray:
    """g = bf16(bf16(t @ W^T) + b).  Reference: model/mlp.py:88-92,376 (nn.Linear)."""
    t64 = bf16_to_f32(t_bf16).astype(np.float64)
    w64 = bf16_to_f32(gate_w_bf16).astype(np.float64)
    dot = f64_to_bf16(t64 @ w64.T)
    g = bf16_to_f32(dot) + bf16_to_f32(gate_b_bf16)[None, :]
    return f32_to_bf16(g.astype(np.float32))


def topk_softmax(g_bf16: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Top-k (largest, descending, lower index on ties) then softmax over the k.

    Reference: ``nn.op.topk(g, k, axis=-1, largest=True)`` + ``nn.op.softmax(axis=1)``
    at model/mlp.py:381-382.  Returns (weights bf16 [n,k], indices int32 [n,k]).
    """
    g = bf16_to_f32(g_bf16)
    order = np.argsort(-g, axis=-1, kind="stable")[:, :k]
    idx = order.astype(np.int32)
    v = np.take_along_axis(g, order, axis=-1).astype(np.float64)
    m = v[:, :1]
    e = np.exp(v - m)
    s = e[:, 0].copy()
    for i in range(1, k):
        s = s + e[:, i]
    w = f64_to_bf16(e / s[:, None])
    return w, idx


# ---------------------------------------------------------------------------
# A6: expert grouping (stable counting sort)
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class Permutation:
    indptr: np.ndarray        # [E+1] exclusive scan of per-expert counts
    sorted_pairs: np.ndarray  # [n*k] sorted position -> pair index p = token*k + slot
    token_indices: np.ndarray # [n*k] sorted position -> token
    expert_ids: np.ndarray    # [n*k] sorted position -> expert
    pair_pos: np.ndarray      # [n*k] pair index -> sorted position


def permute(idx: np.ndarray, num_experts: int) -> Permutation:
    """Group the n*k (token, slot) pairs by expert, token-ascending within an expert.

    Reference semantics: mlc-llm ``moe_cumsum`` / ``get_indices`` / ``get_indptr``
    (inclusive=False) and ``moe_expand_indptr``, called at
    model/mlp_optimized.py:119-148; the cumulative sum runs over the expert-major
    mask, so within an expert pairs stay in flattened (token, slot) order.
    """
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    k = idx.shape[-1]
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts)[:num_experts]
    indptr = np.zeros(num_experts + 1, dtype=np.int32)
    indptr[1:] = np.cumsum(counts)
    pair_pos = np.empty_like(order)
    pair_pos[order] = np.arange(order.size)
    return Permutation(
        indptr=indptr,
        sorted_pairs=order.astype(np.int32),
        token_indices=(order // k).astype(np.int32),
        expert_ids=flat[order].astype(np.int32),
        pair_pos=pair_pos.astype(np.int32),
    )


# ---------------------------------------------------------------------------
# A7-A11: expert matmuls, SwiGLU, gating, residual
# ---------------------------------------------------------------------------

def einsum_fused(x: np.ndarray, idx: np.ndarray, blocks: np.ndarray, scales: np.ndarray,
                 bias_bf16: np.ndarray) -> np.ndarray:
    """out[s,r,c] = bias[e,c] + sum_i x[s,(r,)i] * W_e[c,i], e = idx[s,r]; fp32 out.

    Reference: ``moe_einsum_fused``, model/mlp.py:238-326.  x is fp32 values,
    either [n, K] (mlp1: the bf16 norm output widened) or [n, k, K] (mlp2).
    Sums in fp64 per expert (exact products), rounds once to fp32.
    """
    n, k = idx.shape
    nrows = blocks.shape[1]
    out = np.empty((n, k, nrows), dtype=np.float32)
    x64 = np.asarray(x, dtype=np.float64)
    for e in np.unique(idx):
        sel = np.nonzero(idx == e)
        w = dequant_weight_f64(blocks[e], scales[e])          # [N, K]
        xs = x64[sel[0]] if x64.ndim == 2 else x64[sel[0], sel[1]]
        y = xs @ w.T + bf16_to_f32(bias_bf16[e]).astype(np.float64)[None, :]
        out[sel[0], sel[1]] = y.astype(np.float32)
    return out


def swiglu(x: np.ndarray, alpha: float = SWIGLU_ALPHA, limit: float = 7.0) -> np.ndarray:
    """Interleaved clamped SwiGLU, fp32 in/out.  Reference: model/mlp.py:29-60.

    Pairs along the last dim: even = glu, odd = linear; glu clamped above only,
    linear clamped to [-limit, limit]; out = glu * sigmoid(alpha*glu) * (lin + 1).
    """
    x = np.asarray(x, dtype=np.float32)
    glu = x[..., 0::2]
    lin = x[..., 1::2]
    lim = np.float32(limit)
    xg = np.minimum(glu, lim)
    xl = np.clip(lin, -lim, lim)
    z = (np.float32(alpha) * xg).astype(np.float32)
    with np.errstate(over="ignore"):
        sig = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    gating = (xg * sig).astype(np.float32)
    return (gating * (xl + np.float32(1.0))).astype(np.float32)


def gating(y: np.ndarray, w_bf16: np.ndarray) -> np.ndarray:
    """out[s,c] = bf16(sum_r y[s,r,c] * w[s,r]), fp32, r in order, from 0.

    Reference: ``moe_gemv_gating``, model/mlp.py:328-369.
    """
    y = np.asarray(y, dtype=np.float32)
    w = bf16_to_f32(w_bf16)
    acc = np.zeros(y.shape[::2], dtype=np.float32)
    for r in range(y.shape[1]):
        acc = (acc + (y[:, r, :] * w[:, r:r + 1]).astype(np.float32)).astype(np.float32)
    return f32_to_bf16(acc)


def residual_add(x_bf16: np.ndarray, t_bf16: np.ndarray) -> np.ndarray:
    """bf16(x + t).  Reference: model/mlp.py:402."""
    return f32_to_bf16(bf16_to_f32(x_bf16) + bf16_to_f32(t_bf16))


@dataclasses.dataclass
class BlockParams:
    """The nine MLPBlock parameters in checkpoint layout (model/mlp.py:63-144)."""
    norm_w: np.ndarray        # [H] bf16 bits
    gate_w: np.ndarray        # [E, H] bf16 bits
    gate_b: np.ndarray        # [E] bf16 bits
    mlp1_blocks: np.ndarray   # [E, 2I, H/32, 16] u8
    mlp1_scales: np.ndarray   # [E, 2I, H/32] u8
    mlp1_bias: np.ndarray     # [E, 2I] bf16 bits
    mlp2_blocks: np.ndarray   # [E, H, I/32, 16] u8
    mlp2_scales: np.ndarray   # [E, H, I/32] u8
    mlp2_bias: np.ndarray     # [E, H] bf16 bits

    @property
    def num_experts(self) -> int:
        return self.gate_w.shape[0]


@dataclasses.dataclass
class BlockTrace:
    t: np.ndarray
    g: np.ndarray
    w: np.ndarray
    idx: np.ndarray
    h1: np.ndarray
    act: np.ndarray
    y: np.ndarray
    moe: np.ndarray
    out: np.ndarray


def block_forward(x_bf16: np.ndarray, p: BlockParams, k: int = 4, eps: float = 1e-5,
                  limit: float = 7.0, alpha: float = SWIGLU_ALPHA) -> BlockTrace:
    """MLPBlock.forward, model/mlp.py:371-402, on x [n, H] bf16 bits."""
    t = rms_norm(x_bf16, p.norm_w, eps)
    g = router_logits(t, p.gate_w, p.gate_b)
    w, idx = topk_softmax(g, k)
    h1 = einsum_fused(bf16_to_f32(t), idx, p.mlp1_blocks, p.mlp1_scales, p.mlp1_bias)
    act = swiglu(h1, alpha, limit)
    y = einsum_fused(act, idx, p.mlp2_blocks, p.mlp2_scales, p.mlp2_bias)
    moe = gating(y, w)
    out = residual_add(x_bf16, moe)
    return BlockTrace(t=t, g=g, w=w, idx=idx, h1=h1, act=act, y=y, moe=moe, out=out)


def tie_tokens(g_bf16: np.ndarray, k: int) -> np.ndarray:
    """Tokens whose k-th and (k+1)-th largest logits are equal (top-k set depends on the tie rule)."""
    g = np.sort(bf16_to_f32(g_bf16), axis=-1)[:, ::-1]
    if g.shape[1] <= k:
        return np.zeros(g.shape[0], dtype=bool)
    return g[:, k - 1] == g[:, k]


def compare_outputs(out_bf16: np.ndarray, ref_bf16: np.ndarray) -> dict:
    """Block-output error metrics: norm-relative max error and mean absolute error."""
    a = bf16_to_f32(out_bf16).astype(np.float64)
    b = bf16_to_f32(ref_bf16).astype(np.float64)
    d = np.abs(a - b)
    return {
        "max_rel": float(d.max() / max(np.abs(b).max(), 1e-30)),
        "mae": float(d.mean()),
        "max_abs": float(d.max()),
        "frac_diff": float((d > 0).mean()),
    }


# ---------------------------------------------------------------------------
# Seeded synthetic inputs
# ---------------------------------------------------------------------------

def _bf16_normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def make_params(seed: int, num_experts: int = 32, hidden: int = 2880, inter: int = 2880,
                scale_lo: int = 118, scale_hi: int = 122, zipf_beta: float = 0.0) -> BlockParams:
    """Synthetic block parameters drawn from numpy PCG64(seed).

    Draw order: gate.W, gate.b, mlp1 blocks/scales/bias, mlp2 blocks/scales/bias.
    blocks uniform u8 (nibbles uniform 0..15), scales uniform in [scale_lo, scale_hi],
    biases N(0, 0.01), gate.W N(0, 0.02), gate.b N(0, 0.01), unit norm weight.
    ``zipf_beta`` > 0 adds beta*ln(p_rank), p ~ rank^-1.1, to the router bias.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    E, H, I = num_experts, hidden, inter
    gate_w = _bf16_normal(rng, (E, H), 0.02)
    gb = rng.standard_normal(E, dtype=np.float32) * np.float32(0.01)
    if zipf_beta:
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
        p /= p.sum()
        gb = (gb + zipf_beta * np.log(p)).astype(np.float32)
    gate_b = f32_to_bf16(gb)
    m1b = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    m1s = rng.integers(scale_lo, scale_hi + 1, (E, 2 * I, H // 32), dtype=np.uint8)
    m1bias = _bf16_normal(rng, (E, 2 * I), 0.01)
    m2b = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    m2s = rng.integers(scale_lo, scale_hi + 1, (E, H, I // 32), dtype=np.uint8)
    m2bias = _bf16_normal(rng, (E, H), 0.01)
    norm_w = f32_to_bf16(np.ones(H, dtype=np.float32))
    return BlockParams(norm_w, gate_w, gate_b, m1b, m1s, m1bias, m2b, m2s, m2bias)


def make_input(seed: int, n: int, hidden: int = 2880) -> np.ndarray:
    """x ~ N(0,1) bf16 [n, hidden] from PCG64(seed)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return _bf16_normal(rng, (n, hidden), 1.0)


def algorithmic_bytes(n: int, touched_experts: int, num_experts: int = 32,
                      hidden: int = 2880, inter: int = 2880) -> int:
    """Compulsory HBM bytes of one block call: touched experts' weights, router and
    norm weights, x in and out.  Intermediates excluded."""
    g1, g2 = hidden // 32, inter // 32
    per_expert = (2 * inter * g1 * 17 + 2 * inter * 2) + (hidden * g2 * 17 + hidden * 2)
    return touched_experts * per_expert + num_experts * hidden * 2 + 2 * num_experts + 2 * hidden + n * hidden * 4


def flops(n: int, k: int = 4, num_experts: int = 32, hidden: int = 2880, inter: int = 2880) -> int:
    """Algorithmic flops of one block call (2 per multiply-add)."""
    return n * (2 * k * (2 * inter * hidden + hidden * inter) + 2 * hidden * num_experts)
