"""CPU checks of the fp8 pieces encoding (tests/pieces_model.py).

Pinned by: the e4m3 value table against known answers and an independent
construction; exhaustive round trips and tie-to-even at every midpoint; the
scale rule against brute force; and reconstruction bounds that a dropped
piece, a wrong scale or an off-by-one block index would break.
"""
import numpy as np
import pytest

import pieces_model as PM
from oracle import moe_oracle as O


def test_e4m3_known_values():
    d = PM.e4m3_decode(np.arange(256))
    assert d[0x00] == 0.0 and d[0x80] == 0.0 and np.signbit(d[0x80])
    assert d[0x01] == 2.0 ** -9          # smallest subnormal
    assert d[0x07] == 7 * 2.0 ** -9      # largest subnormal
    assert d[0x08] == 2.0 ** -6          # smallest normal
    assert d[0x38] == 1.0
    assert d[0x3C] == 1.5
    assert d[0x7E] == 448.0              # largest finite
    assert d[0xB8] == -1.0
    assert np.isnan(d[0x7F]) and np.isnan(d[0xFF])
    # independent construction: all finite positive values in increasing order
    vals = sorted({m * 2.0 ** -9 for m in range(8)} |
                  {(1 + m / 8) * 2.0 ** (e - 7) for e in range(1, 16) for m in range(8)
                   if not (e == 15 and m == 7)})
    assert np.array_equal(d[:0x7F], np.array(vals))


def test_e4m3_round_trip_and_ties():
    finite = np.array([c for c in range(256)
                       if (c & 0x7F) != 0x7F and abs(PM.e4m3_decode(c)) < 256])
    assert np.array_equal(PM.e4m3_encode(PM.e4m3_decode(finite)), finite.astype(np.uint8))
    pos = np.array([PM.e4m3_decode(c) for c in range(0, 0x78)])   # 0 .. 240
    mids = (pos[:-1] + pos[1:]) / 2
    enc = PM.e4m3_encode(mids).astype(np.int64)
    # a midpoint rounds to the neighbour with the even code
    lo = np.arange(0, 0x77)
    assert np.array_equal(enc, np.where(lo % 2 == 0, lo, lo + 1))
    # just above / below a midpoint round away from the tie
    assert np.array_equal(PM.e4m3_encode(np.nextafter(mids, np.inf)).astype(np.int64), lo + 1)
    assert np.array_equal(PM.e4m3_encode(np.nextafter(mids, -np.inf)).astype(np.int64), lo)
    # 240..256 rounds to 240 or 256 (code 0x78)
    assert PM.e4m3_encode(np.array([250.0]))[0] == 0x78
    assert PM.e4m3_encode(np.array([-0.75]))[0] == 0xB4


def test_scale_rule_brute_force():
    """s is the smallest E8M0 exponent with amax / 2^(s-127) < 256 (0 for tiny amax)."""
    rng = np.random.default_rng(3)
    amax = np.concatenate([
        (rng.standard_normal(500) ** 2 * 10.0 ** rng.integers(-30, 30, 500)).astype(np.float32),
        np.array([0.0, 1.0, 255.99, 256.0, 1e-40, 3e38], np.float32)])
    s = PM.e8m0_for_amax(amax)
    for a, si in zip(amax.astype(np.float64), s):
        best = min(t for t in range(255) if a / 2.0 ** (t - 127) < 256)
        assert si == best, (a, si, best)
        if si > 0:  # and the block maximum then lands in [128, 256)
            assert 128 <= a / 2.0 ** (si - 127) < 256


@pytest.mark.parametrize("K", [2880, 96, 160])
def test_bf16_two_pieces(K):
    rng = np.random.default_rng(K)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((16, K)).astype(np.float32)))
    q, qs = PM.quantize_pieces(x, 2)
    assert q.shape == (16, 2, (K + 127) // 128 * 128)
    rec = PM.reconstruct(q, qs, K)
    blocks = np.abs(x.astype(np.float64)).reshape(16, -1, 32).max(-1)
    err = np.abs(rec - x).reshape(16, -1, 32).max(-1)
    assert np.all(err <= 2.0 ** -14 * blocks)
    # first-piece codes stay below 256 and the block max lands in [128, 256)
    v0 = np.abs(PM.e4m3_decode(q[:, 0]))
    assert np.all(v0 <= 256)
    assert np.all(np.isin(q[:, :, K:], [0]))
    # one dropped piece is far outside the bound
    rec1 = PM.reconstruct(q[:, :1], qs[:, :1], K)
    assert np.abs(rec1 - x).max() > 2.0 ** -10 * blocks.max()


def test_bf16_narrow_blocks_exact():
    """A block whose values span at most 6 binades is reproduced exactly by 2 pieces."""
    rng = np.random.default_rng(5)
    mant = rng.integers(128, 256, (8, 256)).astype(np.float32) / 128.0
    exps = rng.integers(-3, 3, (8, 256)).astype(np.float32)
    sign = rng.choice([-1.0, 1.0], (8, 256)).astype(np.float32)
    x = O.bf16_to_f32(O.f32_to_bf16(sign * mant * 2.0 ** exps))
    q, qs = PM.quantize_pieces(x, 2)
    assert np.array_equal(PM.reconstruct(q, qs, 256), x.astype(np.float64))


def test_fp32_four_pieces():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((8, 2880)) * np.exp(rng.standard_normal((8, 2880)))).astype(np.float32)
    x[0, :64] = 0.0                                  # all-zero blocks
    x[1, 32:64] = np.float32(1e-30)                  # tiny block
    q, qs = PM.quantize_pieces(x, 4)
    rec = PM.reconstruct(q, qs, 2880)
    blocks = np.abs(x.astype(np.float64)).reshape(8, -1, 32).max(-1)
    err = np.abs(rec - x).reshape(8, -1, 32).max(-1)
    # each piece leaves at most half an e4m3 step of the block maximum: <= 2^-4 of it
    assert np.all(err <= 2.0 ** -16 * blocks + 1e-45)
    err3 = np.abs(PM.reconstruct(q[:, :3], qs[:, :3], 2880) - x).max()
    assert err3 > 8 * err.max()
    assert np.all(rec[0, :64] == 0) and np.all(qs[0, :, :2, 0] == 0)
    # scale runs: byte c of run g is block 4c + g; bytes past NC are zero
    assert np.all(qs[:, :, :, 23:] == 0)
    s0 = PM.e8m0_for_amax(np.abs(x[2, 32 * 5: 32 * 6]).max())
    assert qs[2, 0, 5 % 4, 5 // 4] == s0
