"""numpy specification of the fp8 "pieces" operand encoding (test infrastructure).

The GPU expert matmuls multiply MXFP4 weights by activations carried as a sum
of fp8 e4m3 rows with one E8M0 scale per 32 elements (the operand format of
gfx950's block-scaled MFMA).  This module states that encoding in numpy so
tests can compare the device's packed buffer byte for byte, and so the
encoding's error bounds can be checked on the CPU.  It is not part of the
reference: the reference multiplies bf16 activations by dequantised weights
(model/mlp_optimized.py:324-331) and the block-output tolerance covers the
difference.

Packed layout for rows x K, NC = ceil(K / 128), Kp = 128 NC:
  q  [rows, P, Kp]      e4m3 codes (zero past K)
  qs [rows, P, 4, 28]   qs[r, p, g, c] = E8M0 of 32-block 4c + g (zero past NC)
with qs starting at the first 256-byte boundary after q.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3_decode(codes) -> np.ndarray:
    """e4m3 (OCP: bias 7, no infinities, 0x7F/0xFF NaN) -> float64, from the bits."""
    c = np.asarray(codes, dtype=np.int64)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, np.ldexp(1.0 + m / 8.0, (e - 7).astype(np.int32)))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return np.where(c & 0x80, -mag, mag)


def e4m3_encode(v) -> np.ndarray:
    """Round |v| < 256 to the nearest e4m3 value (ties to even) -> uint8 codes."""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    assert np.all(a < 256.0)
    sign = (np.signbit(v)).astype(np.int64) << 7
    _, ex = np.frexp(np.where(a > 0, a, 1.0))   # a = f * 2^ex, f in [0.5, 1)
    e = ex.astype(np.int64) - 1                  # a in [2^e, 2^(e+1))
    sub = (a < 2.0 ** -6)
    code_sub = np.rint(a * 512.0).astype(np.int64)
    mq = np.rint(a * np.ldexp(1.0, (3 - e).astype(np.int32))).astype(np.int64)  # [8, 16]
    carry = mq == 16
    mq = np.where(carry, 8, mq)
    e = e + carry
    code_norm = ((e + 7) << 3) | (mq - 8)
    return (np.where(sub, code_sub, code_norm) | sign).astype(np.uint8)


def e8m0_for_amax(amax) -> np.ndarray:
    """Smallest E8M0 s with amax / 2^(s-127) < 256: floor(log2 amax) - 7 (+127), >= 0."""
    a = np.asarray(amax, dtype=np.float32)
    eb = (a.view(np.uint32) >> 23).astype(np.int64) & 0xFF
    return np.maximum(eb - 7, 0)


def quantize_pieces(x, pieces: int):
    """x [rows, K] (float32 values) -> (q [rows, P, Kp] u8, qs [rows, P, 4, 28] u8)."""
    x = np.asarray(x, dtype=np.float32)
    rows, K = x.shape
    nc = (K + 127) // 128
    kp = nc * 128
    r = np.zeros((rows, kp), dtype=np.float64)
    r[:, :K] = x
    r = r.reshape(rows, 4 * nc, 32)
    q = np.zeros((rows, pieces, 4 * nc, 32), dtype=np.uint8)
    qs = np.zeros((rows, pieces, 4, 28), dtype=np.uint8)
    for p in range(pieces):
        amax = np.abs(r).max(axis=-1)
        s = e8m0_for_amax(amax)
        scale = np.ldexp(1.0, (s - 127).astype(np.int32))[..., None]
        codes = e4m3_encode(r / scale)
        r = r - e4m3_decode(codes) * scale
        q[:, p] = codes
        blk = np.arange(4 * nc)
        qs[:, p, blk % 4, blk // 4] = s.astype(np.uint8)
    return q.reshape(rows, pieces, kp), qs


def reconstruct(q, qs, K: int) -> np.ndarray:
    """Sum of the pieces, float64 [rows, K]."""
    rows, pieces, kp = q.shape
    nc = kp // 128
    blk = np.arange(4 * nc)
    s = qs[:, :, blk % 4, blk // 4].astype(np.int64)            # [rows, P, 4nc]
    scale = np.ldexp(1.0, (s - 127).astype(np.int32))
    v = e4m3_decode(q.reshape(rows, pieces, 4 * nc, 32)) * scale[..., None]
    return v.sum(axis=1).reshape(rows, kp)[:, :K]


def unpack(packed: np.ndarray, rows: int, K: int, pieces: int):
    """Split a packed device buffer (u8) into (q, qs)."""
    kp = (K + 127) // 128 * 128
    qb = (rows * pieces * kp + 255) // 256 * 256
    q = packed[: rows * pieces * kp].reshape(rows, pieces, kp)
    qs = packed[qb: qb + rows * pieces * 112].reshape(rows, pieces, 4, 28)
    return q, qs
