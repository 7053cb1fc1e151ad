"""GPU parity of the HIP MoE path against the CPU oracle.

Bars (north star): MXFP4 dequantisation and routing (indices, weights, the
normalised tokens) bit-exact; the grouping bit-exact against a stable sort;
block outputs within max norm-relative error 1e-2 and mean absolute error
1e-3 in bf16.  Intermediate fp32 results are held to tighter bars stated at
each test.  Every call goes through the C ABI (libmoe_gfx950.so via moe_native).
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import moe_oracle as O  # noqa: E402
from gpu_util import (bf16_dev, f32_dev, host, host_bf16, i32_dev, make_block, norm_rel,  # noqa: E402
                      params_from_npz, u8_dev)
import pieces_model as PM  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MAX_REL, MAE = 1e-2, 1e-3
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.fixture(scope="module")
def native():
    import moe_native
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return moe_native


def _nan_aware_equal(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    na = (a & 0x7FFF) > 0x7F80
    nb = (b & 0x7FFF) > 0x7F80
    return np.where(na | nb, na == nb, a == b)


# ---------------------------------------------------------------------------
# dequantisation
# ---------------------------------------------------------------------------

def _all_pairs():
    blocks = np.broadcast_to(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 16, 16)).copy()
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    return blocks, scales


def test_dequant_reference_kernel_exhaustive(native):
    blocks, scales = _all_pairs()
    out = host_bf16(native.dequant_mxfp4(u8_dev(blocks), u8_dev(scales)))
    ref = O.dequant_mxfp4(blocks, scales)
    ok = _nan_aware_equal(out, ref)
    assert ok.all(), f"{(~ok).sum()} mismatches, first at {np.argwhere(~ok)[:4]}"


def test_dequant_fused_path_exact_in_range(native):
    """The matmuls' hardware conversion equals the reference dequant for 2 <= s <= 252."""
    blocks, scales = _all_pairs()
    out = host_bf16(native.dequant_mxfp4(u8_dev(blocks), u8_dev(scales), fast=True))
    ref = O.dequant_mxfp4(blocks, scales)
    ok = _nan_aware_equal(out, ref)
    in_range = (scales >= 2) & (scales <= 252)
    bad = ~ok & in_range[..., None]
    assert not bad.any(), f"{bad.sum()} mismatches in range, first at {np.argwhere(bad)[:4]}"
    edge = sorted(set(int(s) for s in np.argwhere(~ok)[:, 0]))
    print(f"fused-path dequant differs from the reference only at scales {edge}")


# ---------------------------------------------------------------------------
# router and grouping
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("E,H,n,seed", [(32, 2880, 64, 1), (32, 2880, 1, 2), (32, 2880, 1000, 3),
                                        (128, 2880, 300, 4), (8, 128, 7, 5), (256, 64, 33, 6),
                                        (32, 2880, 257, 9), (128, 4096, 5, 10)])
def test_router_bit_exact(native, E, H, n, seed):
    p = O.make_params(seed, num_experts=E, hidden=H, inter=64)
    x = O.make_input(seed + 100, n, hidden=H)
    t_ref = O.rms_norm(x, p.norm_w)
    g_ref = O.router_logits(t_ref, p.gate_w, p.gate_b)
    w_ref, idx_ref = O.topk_softmax(g_ref, 4)
    t, idx, w = native.router_topk(bf16_dev(x), bf16_dev(p.norm_w), bf16_dev(p.gate_w),
                                   bf16_dev(p.gate_b), 4, 1e-5)
    assert np.array_equal(host_bf16(t), t_ref)
    ties = O.tie_tokens(g_ref, 4)
    assert np.array_equal(host(idx), idx_ref), f"ties at tokens {np.flatnonzero(ties)}"
    assert np.array_equal(host_bf16(w), w_ref)
    print(f"E={E} n={n}: {int(ties.sum())} tokens with a 4th/5th tie, all routed identically")


def test_router_dot_on_bf16_tie(native):
    """Token 101 of this input has a gate dot whose fp32 value is exactly a bf16
    tie (low half 0x8000) while the exact dot lies above it: the two roundings
    fp64 -> fp32 -> bf16 give the even neighbour, one fp64 -> bf16 rounding the
    upper one.  Both router paths must keep the two roundings."""
    p = O.make_params(0, num_experts=32, hidden=2880, inter=64)
    x = O.make_input(16, 520)
    t_ref = O.rms_norm(x, p.norm_w)
    d = (O.bf16_to_f32(t_ref).astype(np.float64) @ O.bf16_to_f32(p.gate_w).astype(np.float64).T)
    assert (d.astype(np.float32).view(np.uint32)[101, 6] & 0xFFFF) == 0x8000
    w_ref, idx_ref = O.topk_softmax(O.router_logits(t_ref, p.gate_w, p.gate_b), 4)
    _, idx, w = native.router_topk(bf16_dev(x), bf16_dev(p.norm_w), bf16_dev(p.gate_w),
                                   bf16_dev(p.gate_b), 4, 1e-5)
    assert np.array_equal(host(idx), idx_ref) and np.array_equal(host_bf16(w), w_ref)
    blk = make_block(p)
    blk(bf16_dev(x).view(1, 520, 2880))
    torch.cuda.synchronize()
    ws = blk._workspace(520, torch.device("cuda:0"))
    offs = native.workspace_layout(520, 32, 4, 2880, 64)
    wb = host(ws[offs[2]: offs[2] + 520 * 8].view(torch.int16)).view(np.uint16).reshape(520, 4)
    assert np.array_equal(wb, w_ref), np.argwhere(wb != w_ref)


def test_router_tie_rule(native):
    """Exactly tied logits: the lower expert index wins (as the oracle's stable sort)."""
    E, H, n = 32, 64, 8
    p = O.make_params(7, num_experts=E, hidden=H, inter=64)
    p.gate_w[:] = 0
    rng = np.random.default_rng(0)
    p.gate_b[:] = O.f32_to_bf16(rng.integers(-2, 3, E).astype(np.float32) * 0.25)
    x = O.make_input(8, n, hidden=H)
    w_ref, idx_ref = O.topk_softmax(O.router_logits(O.rms_norm(x, p.norm_w), p.gate_w, p.gate_b), 4)
    t, idx, w = native.router_topk(bf16_dev(x), bf16_dev(p.norm_w), bf16_dev(p.gate_w),
                                   bf16_dev(p.gate_b), 4, 1e-5)
    assert np.array_equal(host(idx), idx_ref) and np.array_equal(host_bf16(w), w_ref)


@pytest.mark.parametrize("n,k,E", [(1, 4, 32), (64, 4, 32), (4096, 4, 32), (8192, 4, 32),
                                   (2048, 4, 128), (300, 2, 256), (5, 4, 4)])
def test_permute_bit_exact(native, n, k, E):
    rng = np.random.default_rng(n + E)
    idx = np.array([rng.permutation(E)[:k] for _ in range(n)], dtype=np.int32).reshape(n, k)
    ref = O.permute(idx, E)
    res = native.permute(i32_dev(idx), E)
    for key in ("indptr", "sorted_pairs", "token_indices", "expert_ids", "pair_pos"):
        assert np.array_equal(host(res[key]), getattr(ref, key)), key


def test_permute_skewed_and_out_of_range(native):
    n, k, E = 777, 4, 16
    rng = np.random.default_rng(9)
    idx = np.stack([np.array([0, 1, 2, 3])[rng.permutation(4)] for _ in range(n)]).astype(np.int32)
    idx[5, 2] = 99     # out of range: not placed
    idx[6, 0] = -1
    res = native.permute(i32_dev(idx), E)
    flat = idx.reshape(-1)
    order = [p for e in range(E) for p in range(n * k) if flat[p] == e]
    counts = [int((flat == e).sum()) for e in range(E)]
    assert list(host(res["indptr"])) == [0] + list(np.cumsum(counts))
    assert list(host(res["sorted_pairs"])[:len(order)]) == order
    pp = host(res["pair_pos"])
    keep = (flat >= 0) & (flat < E)
    assert np.all(pp[~keep] == -1)
    assert np.array_equal(np.array(order)[pp[keep]], np.flatnonzero(keep))


# ---------------------------------------------------------------------------
# expert matmuls
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("E,N,K,n,three_d", [(4, 128, 64, 5, False), (4, 128, 64, 5, True),
                                             (32, 5760, 2880, 64, False), (32, 2880, 2880, 64, True),
                                             (8, 192, 96, 200, False), (8, 192, 96, 200, True)])
def test_einsum_fused(native, E, N, K, n, three_d):
    rng = np.random.default_rng(E * N + n)
    blocks = rng.integers(0, 256, (E, N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(118, 123, (E, N, K // 32), dtype=np.uint8)
    bias = O.f32_to_bf16(rng.standard_normal((E, N)).astype(np.float32) * 0.01)
    idx = np.array([rng.permutation(E)[:4] for _ in range(n)], dtype=np.int32)
    if three_d:
        x = (rng.standard_normal((n, 4, K)) * 0.5).astype(np.float32)
        xd = f32_dev(x)
    else:
        xb = O.f32_to_bf16(rng.standard_normal((n, K)).astype(np.float32))
        x = O.bf16_to_f32(xb)
        xd = bf16_dev(xb)
    ref = O.einsum_fused(x, idx, blocks, scales, bias)
    out = host(native.einsum_fused(xd, i32_dev(idx), u8_dev(blocks), u8_dev(scales), bf16_dev(bias)))
    # x enters the MFMA as fp8 pieces: 2 for bf16 x (exact to 2^-14 of each
    # 32-block's maximum), 4 for fp32 x (to 2^-16 of it); sums in fp32.  A
    # dropped piece or a wrong block scale is off by 4e-3 or more.
    assert norm_rel(out, ref) <= 5e-5, norm_rel(out, ref)


def test_many_tokens_per_expert(native):
    """All tokens on the same 4 experts: > 32 pairs per expert takes several passes."""
    E, H, I, n = 8, 128, 64, 150
    p = O.make_params(21, num_experts=E, hidden=H, inter=I)
    p.gate_b[:] = O.f32_to_bf16(np.array([10, 9, 8, 7, -10, -10, -10, -10], np.float32))
    x = O.make_input(22, n, hidden=H)
    tr = O.block_forward(x, p)
    assert np.all(np.sort(tr.idx, axis=1) == [0, 1, 2, 3])
    blk = make_block(p)
    out = host_bf16(blk(bf16_dev(x).view(1, n, H)).view(n, H))
    m = O.compare_outputs(out, tr.out)
    assert m["max_rel"] <= MAX_REL and m["mae"] <= MAE, m


@pytest.mark.parametrize("E,H,I,n,seed", [(8, 128, 64, 2000, 31), (32, 256, 64, 1030, 32),
                                          (128, 128, 64, 700, 33), (32, 2880, 64, 64, 34),
                                          (32, 2880, 64, 1, 35), (12, 192, 64, 257, 36),
                                          (32, 2880, 2880, 1, 37), (32, 2880, 2880, 64, 38),
                                          (32, 2880, 2880, 128, 39), (32, 2880, 64, 4096, 40),
                                          (128, 2880, 64, 1100, 41), (128, 256, 64, 4100, 42),
                                          (40, 192, 64, 1500, 43), (32, 2880, 2880, 2, 44),
                                          (128, 2880, 64, 2, 45), (128, 256, 64, 1, 46),
                                          (12, 192, 64, 1, 47), (40, 192, 64, 1, 48)])
def test_block_internal_routing(native, E, H, I, n, seed):
    """The block's own router and grouping (logits kernel — VALU fp64 dots up
    to 1024 tokens, fp64 MFMA dots above — then top-k + grouping: at the 20B
    shape by the one-token mlp1 / mlp2 launches at n = 1, by the logits
    launch's last workgroup at n = 2 (the decode launch then runs the
    experts), by the decode launch's own prologue at n = 64 and 128; one
    workgroup of top-k + grouping for other shapes with n k <= 4096, the
    chunked two-pass grouping above): t, indices, weights and every grouping
    array bit-exact, output in tolerance."""
    p = O.make_params(seed, num_experts=E, hidden=H, inter=I)
    x = O.make_input(seed + 100, n, hidden=H)
    tr = O.block_forward(x, p)
    blk = make_block(p)
    out = host_bf16(blk(bf16_dev(x).view(1, n, H)).view(n, H))
    torch.cuda.synchronize()
    ws = blk._workspace(n, torch.device("cuda:0"))
    offs = native.workspace_layout(n, E, 4, H, I)
    nk = n * 4

    def region(i, dtype, count):
        return ws[offs[i]: offs[i] + count * torch.tensor([], dtype=dtype).element_size()].view(dtype)

    assert np.array_equal(host_bf16(region(0, torch.bfloat16, n * H)).reshape(n, H), tr.t)
    assert np.array_equal(host(region(1, torch.int32, nk)).reshape(n, 4), tr.idx), \
        f"ties at tokens {np.flatnonzero(O.tie_tokens(tr.g, 4))}"
    assert np.array_equal(host_bf16(region(2, torch.bfloat16, nk)).reshape(n, 4), tr.w)
    perm = O.permute(tr.idx, E)
    assert np.array_equal(host(region(3, torch.int32, E + 1)), perm.indptr)
    for i, ref in ((4, perm.sorted_pairs), (5, perm.token_indices), (6, perm.expert_ids),
                   (7, perm.pair_pos)):
        assert np.array_equal(host(region(i, torch.int32, nk)), ref), i
    m = O.compare_outputs(out, tr.out)
    assert m["max_rel"] <= MAX_REL and m["mae"] <= MAE, m
    # the workspace's counters (its first 256 bytes) are back at zero
    assert int(torch.count_nonzero(ws[:256])) == 0


def test_block_workspace_reused_across_sizes(native, oracle_lib):
    """One zero-filled workspace serves calls of different sizes in turn (the
    router's arrival count sits at the workspace's start for every n and each
    call leaves it at zero): decode sizes (one router launch whose last
    workgroup selects and groups), a 300-token call (two router launches, the
    GEMV path) and decode again.  Routing bit-exact and outputs in tolerance
    every time; the counters zero after every call."""
    p = O.make_params(50, num_experts=32, hidden=2880, inter=2880)
    blk = make_block(p)
    ws = torch.zeros(blk.workspace_bytes(300), dtype=torch.uint8, device="cuda")
    offs_for = {}
    for i, n in enumerate((64, 1, 300, 64, 100, 2, 64)):
        print(f"reused workspace: call {i}, n={n}", flush=True)
        x = O.make_input(60 + i, n)
        out = torch.empty((n, 2880), dtype=torch.bfloat16, device="cuda")
        blk.forward_into(bf16_dev(x), out, ws)
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ws[:256])) == 0, i
        offs = offs_for.setdefault(n, native.workspace_layout(n, 32, 4, 2880, 2880))
        _, idx_ref = O.topk_softmax(O.router_logits(O.rms_norm(x, p.norm_w), p.gate_w, p.gate_b), 4)
        idx = host(ws[offs[1]: offs[1] + n * 16].view(torch.int32)).reshape(n, 4)
        assert np.array_equal(idx, idx_ref), i
        sel = np.arange(n) if n <= 16 else np.sort(np.random.default_rng(i).choice(n, 16, replace=False))
        ref, _, _, _ = oracle_lib.block_forward(np.ascontiguousarray(x[sel]), p, nthreads=THREADS)
        m = O.compare_outputs(host_bf16(out)[sel], ref)
        assert m["max_rel"] <= MAX_REL and m["mae"] <= MAE, (i, m)


@pytest.mark.parametrize("E,H,I,n,seed,skew", [(8, 192, 192, 200, 41, False),
                                               (8, 192, 96, 300, 42, True),
                                               (12, 384, 96, 157, 43, False)])
def test_block_gemm_path(native, E, H, I, n, seed, skew):
    """Experts averaging 48 or more tokens take the tiled GEMM (token tiles of
    128 for mlp1, 64 for mlp2); skewed routing puts 300 tokens on 4 experts
    (several token tiles each).  Act and output against the oracle."""
    p = O.make_params(seed, num_experts=E, hidden=H, inter=I)
    if skew:
        p.gate_b[:] = O.f32_to_bf16(np.array([10, 9, 8, 7] + [-10] * (E - 4), np.float32))
    x = O.make_input(seed + 100, n, hidden=H)
    tr = O.block_forward(x, p)
    assert n * 4 >= 48 * E
    blk = make_block(p)
    _check_block(blk, x, tr)


# ---------------------------------------------------------------------------
# fp8 pieces of the activations (the scaled-MFMA operand), bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,K,pieces,f32", [(64, 2880, 2, False), (256, 2880, 4, True),
                                               (5, 96, 2, False), (7, 160, 4, True),
                                               (3, 3072, 4, False), (1, 32, 2, True),
                                               (256, 2880, 3, True), (9, 160, 3, True)])
def test_quantize_pieces_bit_exact(native, rows, K, pieces, f32):
    rng = np.random.default_rng(rows * K + pieces)
    x = (rng.standard_normal((rows, K)) * np.exp(2 * rng.standard_normal((rows, K)))).astype(np.float32)
    x[0, :32] = 0.0                         # all-zero block
    if K >= 96:
        x[0, 32:64] = np.float32(3e-39)     # fp32 subnormals
        x[-1, 64:96] *= np.float32(1e20)    # large block
    if f32:
        xd = f32_dev(x)
    else:
        xb = O.f32_to_bf16(x)
        x = O.bf16_to_f32(xb)
        xd = bf16_dev(xb)
    packed = host(native.quantize_pieces(xd, pieces))
    q, qs = PM.unpack(packed, rows, K, pieces)
    rq, rqs = PM.quantize_pieces(x, pieces)
    assert np.array_equal(qs, rqs), np.argwhere(qs != rqs)[:4]
    assert np.array_equal(q, rq), np.argwhere(q != rq)[:4]


# ---------------------------------------------------------------------------
# whole block
# ---------------------------------------------------------------------------

def _check_block(blk, x, tr, staged=True):
    n, H = x.shape
    xd = bf16_dev(x).view(1, n, H)
    out = host_bf16(blk(xd).view(n, H))
    m = O.compare_outputs(out, tr.out)
    assert m["max_rel"] <= MAX_REL and m["mae"] <= MAE, m
    if staged:
        st = blk.forward_staged(xd)
        assert np.array_equal(host_bf16(st["out"]).reshape(n, H), out)
        assert np.array_equal(host_bf16(st["t"]), tr.t)
        assert np.array_equal(host(st["idx"]), tr.idx)
        assert np.array_equal(host_bf16(st["w"]), tr.w)
        sp = host(st["perm"]["sorted_pairs"])
        k = tr.idx.shape[1]
        act_ref = tr.act.reshape(n * k, -1)[sp]
        act = host(st["act"])
        assert norm_rel(act, act_ref) <= 2e-5
        y_ref = tr.y.reshape(n * k, -1)
        assert norm_rel(host(st["y"]), y_ref) <= 1e-4
    return m


GOLDEN_CASES = sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_block_golden_fixture(native, name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    p = params_from_npz(z)
    tr = O.BlockTrace(t=z["t"], g=None, w=z["w"], idx=z["idx"], h1=None, act=z["act"], y=z["y"],
                      moe=None, out=z["out"])
    m = _check_block(make_block(p), z["x"], tr)
    print(name, m)


@pytest.fixture(scope="module")
def block20b():
    p = O.make_params(seed=0)
    return p, make_block(p)


@pytest.mark.parametrize("n,seed", [(1, 10), (64, 11), (2, 9), (3, 8), (5, 12), (32, 13), (33, 14),
                                    (520, 16)])
def test_block_20b_shape(native, block20b, n, seed):
    """BASELINE configs 0 (n = 1) and 1 (n = 64) at full 20B shape, small
    decode batches (2, 3 tokens), a ragged n,
    both sides of the decode launch's fused-combine limit (32 tokens: the
    launch sums the k rows itself; 33: the gating kernel does; the staged
    check compares the block with the gating kernel bit for bit), and 520
    tokens (the tiled GEMM path)."""
    p, blk = block20b
    x = O.make_input(seed, n)
    tr = O.block_forward(x, p)
    m = _check_block(blk, x, tr)
    print(f"20B n={n}: {m}")


@pytest.mark.parametrize("n", [64, 301])
def test_block_router_pieces_fused(native, block20b, n):
    """The block's fused router writes the same t pieces as moe_quantize_pieces(t)."""
    p, blk = block20b
    H = 2880
    x = bf16_dev(O.make_input(15, n)).view(1, n, H)
    blk(x)
    torch.cuda.synchronize()
    ws = blk._workspace(n, x.device)
    offs = native.workspace_layout(n, p.num_experts, 4, H, 2880)
    t = ws[offs[0]: offs[0] + n * H * 2].view(torch.bfloat16).view(n, H)
    assert np.array_equal(host_bf16(t), O.rms_norm(O.make_input(15, n), p.norm_w))
    nb = native.pieces_bytes(n, H, 2)
    fused = PM.unpack(host(ws[offs[8]: offs[8] + nb]), n, H, 2)
    ref = PM.unpack(host(native.quantize_pieces(t.contiguous(), 2)), n, H, 2)
    for a, b in zip(fused, ref):  # codes, then scale runs (the alignment pad is not written)
        assert np.array_equal(a, b), np.argwhere(a != b)[:4]


@pytest.mark.parametrize("n,seed", [(2, 17), (64, 18), (100, 19)])
def test_block_decode_act_pieces(native, block20b, n, seed):
    """The decode launch encodes act in LDS, block by block, into the same three
    pieces as moe_quantize_pieces of mlp1's fp32 output (rows by sorted pair).
    The block runs that launch from two tokens up (one token: separate launches,
    checked by test_one_token_act_pieces)."""
    p, blk = block20b
    H, k = 2880, 4
    nk = n * k
    x = bf16_dev(O.make_input(seed, n)).view(1, n, H)
    blk(x)
    torch.cuda.synchronize()
    ws = blk._workspace(n, x.device)
    offs = native.workspace_layout(n, p.num_experts, k, H, 2880)
    nb = native.pieces_bytes(nk, 2880, 3)
    fused = PM.unpack(host(ws[offs[10]: offs[10] + nb]), nk, 2880, 3)
    st = blk.forward_staged(x)
    ref = PM.unpack(host(native.quantize_pieces(st["act"].contiguous(), 3)), nk, 2880, 3)
    for a, b in zip(fused, ref):
        assert np.array_equal(a, b), np.argwhere(a != b)[:4]


@pytest.mark.parametrize("seed", [24, 25])
def test_one_token_act_pieces(native, block20b, seed):
    """At one token the mlp1 launch encodes act into mlp2's three pieces itself,
    one 32-column block per workgroup (rows by slot, the zero blocks up to 128 x
    23 written by the last block's workgroup): the same code bytes and scale
    bytes as moe_quantize_pieces of mlp1's fp32 output (rows by sorted pair),
    the rows matched through pair_pos."""
    p, blk = block20b
    n, H, k = 1, 2880, 4
    x = bf16_dev(O.make_input(seed, n)).view(1, n, H)
    blk(x)
    torch.cuda.synchronize()
    ws = blk._workspace(n, x.device)
    offs = native.workspace_layout(n, p.num_experts, k, H, 2880)
    nb = native.pieces_bytes(k, 2880, 3)
    q, qs = PM.unpack(host(ws[offs[10]: offs[10] + nb]), k, 2880, 3)
    st = blk.forward_staged(x)
    rq, rqs = PM.unpack(host(native.quantize_pieces(st["act"].contiguous(), 3)), k, 2880, 3)
    pos = host(st["perm"]["pair_pos"])
    for s in range(k):
        assert np.array_equal(q[s], rq[pos[s]]), s
        # scale slots 0..22 of each run (chunks 0..22); 23..27 are never read
        assert np.array_equal(qs[s, :, :, :23], rqs[pos[s], :, :, :23]), s


@pytest.mark.parametrize("n,seed", [(1, 21), (64, 22), (128, 23)])
def test_mlp_decode_matches_three_calls(native, block20b, n, seed):
    """moe_mlp_decode = mlp1_swiglu -> quantize_pieces(act, 3) -> mlp2, bit for bit,
    on two calls in a row (the second reuses the outputs; its counters are re-zeroed)."""
    p, blk = block20b
    x = bf16_dev(O.make_input(seed, n)).view(1, n, 2880)
    st = blk.forward_staged(x)
    t_pk = native.quantize_pieces(st["t"], 2)
    perm, k = st["perm"], 4
    args = (t_pk, n, perm["indptr"], perm["sorted_pairs"], k, blk.mlp1_weight_blocks,
            blk.mlp1_weight_scales, blk.mlp1_bias, blk.mlp2_weight_blocks,
            blk.mlp2_weight_scales, blk.mlp2_bias, 1.702, blk.swiglu_limit)
    nk = n * k
    ref_pk = PM.unpack(host(native.quantize_pieces(st["act"].contiguous(), 3)), nk, 2880, 3)
    done = torch.zeros(33, dtype=torch.int32, device="cuda")
    y, pk = native.mlp_decode(*args, done=done)
    for _ in range(2):
        torch.cuda.synchronize()
        assert np.array_equal(host(y), host(st["y"]))
        # codes, then scale runs (the 256-byte alignment pads are not written)
        for a, b in zip(PM.unpack(host(pk), nk, 2880, 3), ref_pk):
            assert np.array_equal(a, b), np.argwhere(a != b)[:4]
        done.zero_()
        y, pk = native.mlp_decode(*args, act_pieces=pk, done=done, y=y)
    cnt = host(torch.diff(perm["indptr"]))
    assert np.array_equal(host(done[:32]), 360 * ((cnt + 15) // 16))  # mlp1 tiles per expert
    assert int(done[32]) == 0  # status: no wait gave up


def test_mlp_decode_unsupported(native, block20b):
    p, blk = block20b
    n = 129
    x = bf16_dev(O.make_input(24, n)).view(1, n, 2880)
    st = blk.forward_staged(x)
    with pytest.raises(RuntimeError, match="unsupported"):
        native.mlp_decode(native.quantize_pieces(st["t"], 2), n, st["perm"]["indptr"],
                          st["perm"]["sorted_pairs"], 4, blk.mlp1_weight_blocks,
                          blk.mlp1_weight_scales, blk.mlp1_bias, blk.mlp2_weight_blocks,
                          blk.mlp2_weight_scales, blk.mlp2_bias, 1.702, blk.swiglu_limit)


@pytest.mark.parametrize("n,mode", [(32, "four"), (64, "four"), (128, "four"), (100, "zipf")])
def test_block_decode_skewed_routing(native, n, mode):
    """The one-launch decode chain with heavy experts: every token on experts
    0..3 (64 or 128 tokens each: several mlp1 batches of 16 and mlp2 batches of
    15 per expert, so the completion counts span batches), or Zipf routing."""
    H = 2880
    if mode == "four":
        p = O.make_params(25, num_experts=32)
        gb = np.full(32, -10.0, np.float32)
        gb[:4] = [10, 9, 8, 7]
        p.gate_b[:] = O.f32_to_bf16(gb)
    else:
        p = O.make_params(26, num_experts=32, zipf_beta=1.0)
    x = O.make_input(27, n)
    tr = O.block_forward(x, p)
    if mode == "four":
        assert np.all(np.sort(tr.idx, axis=1) == [0, 1, 2, 3])
    m = _check_block(make_block(p), x, tr)
    print(f"decode {mode} n={n}: {m}")


def test_block_120b_shape(native):
    p = O.make_params(seed=3, num_experts=128)
    x = O.make_input(13, 48)
    tr = O.block_forward(x, p)
    m = _check_block(make_block(p), x, tr)
    print(f"120B n=48: {m}")


def test_block_deterministic_and_empty(native, block20b):
    p, blk = block20b
    x = bf16_dev(O.make_input(14, 64)).view(2, 32, 2880)
    a = host_bf16(blk(x))
    b = host_bf16(blk(x))
    assert np.array_equal(a, b)
    empty = blk(torch.empty((1, 0, 2880), dtype=torch.bfloat16, device="cuda"))
    assert empty.shape == (1, 0, 2880)


# ---------------------------------------------------------------------------
# the decode launch's bounded wait: a give-up is reported, never silent
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [16, 64])
def test_decode_wait_give_up_is_reported(native, block20b, n):
    """With the wait bound set to 0 polls from the host, every phase-2
    workgroup of the decode launch gives up at once (all kernels still run to
    their end): moe_block_status reports MOE_ERR_INCOMPLETE, every output is
    NaN (16 tokens: the launch's own combine; 64: the gating kernel), and the
    standalone launch's status word counts the give-ups.  With the default
    bound restored the same calls are correct again."""
    p, blk = block20b
    H = 2880
    x = O.make_input(28, n)
    xd = bf16_dev(x).view(1, n, H)
    prev = native.set_decode_spin_limit(0)
    try:
        out = blk(xd)
        ws = blk._workspace(n, xd.device)
        assert native.block_status(ws, n, 32, 4, H, 2880) == -7
        assert torch.isnan(out.float()).all()
        st = blk.forward_staged(xd)
        t_pk = native.quantize_pieces(st["t"], 2)
        done = torch.zeros(33, dtype=torch.int32, device="cuda")
        native.mlp_decode(t_pk, n, st["perm"]["indptr"], st["perm"]["sorted_pairs"], 4,
                          blk.mlp1_weight_blocks, blk.mlp1_weight_scales, blk.mlp1_bias,
                          blk.mlp2_weight_blocks, blk.mlp2_weight_scales, blk.mlp2_bias, 1.702,
                          blk.swiglu_limit, done=done)
        torch.cuda.synchronize()
        assert int(done[32]) > 0
    finally:
        native.set_decode_spin_limit(prev)
    assert native.set_decode_spin_limit(-1) == prev
    out = host_bf16(blk(xd).view(n, H))
    assert native.block_status(blk._workspace(n, xd.device), n, 32, 4, H, 2880) == 0
    m = O.compare_outputs(out, O.block_forward(x, p).out)
    assert m["max_rel"] <= MAX_REL and m["mae"] <= MAE, m


# ---------------------------------------------------------------------------
# standalone SwiGLU and gating exports
# ---------------------------------------------------------------------------

def test_swiglu_standalone(native):
    """moe_swiglu against the oracle's closed form (model/mlp.py:29-60): the
    clamps are exact (glu clamped above only, at 7; linear to [-7, 7]), zeros
    of either factor give exact zeros, and elsewhere the result is within 4
    ulp (the kernel's sigmoid is the device expf, the oracle's correctly
    rounded).  A sign or clamp mistake is off by far more."""
    rng = np.random.default_rng(5)
    special = np.array([[0.0, 3.0], [2.0, -1.0], [7.0, 7.0], [7.5, 9.0], [100.0, -100.0],
                        [-100.0, 2.0], [-7.5, 0.5], [np.inf, 1.0], [3.0, np.inf],
                        [3.0, -np.inf], [-0.0, 5.0], [6.9999995, -6.9999995]], np.float32)
    rand = (rng.standard_normal((4096, 2)) * 4).astype(np.float32)
    x = np.concatenate([special, rand]).reshape(-1, 2 * 4)  # rows of d = 4 pairs
    got = host(native.swiglu(f32_dev(x), 1.702, 7.0))
    ref = O.swiglu(x)
    # exact where the sigmoid does not enter: zero factors
    zero = (x[:, 0::2] == 0) | (x[:, 1::2] == -1)
    assert np.array_equal(got[zero], ref[zero])
    # the clamps: glu >= 7 behaves as 7, lin beyond +-7 as +-7
    xc = x.copy()
    xc[:, 0::2] = np.minimum(xc[:, 0::2], 7.0)
    xc[:, 1::2] = np.clip(xc[:, 1::2], -7.0, 7.0)
    assert np.array_equal(host(native.swiglu(f32_dev(xc), 1.702, 7.0)), got)
    np.testing.assert_allclose(got, ref, rtol=4 * 2.0 ** -23, atol=1e-37)


def test_gemv_gating_without_residual(native):
    """moe_gemv_gating with x == NULL (the reference's run_gating alone,
    model/mlp.py:328-369) and with x (+ residual, mlp.py:402): bit-exact
    against the oracle's in-order fp32 sum, k = 4 and k = 2."""
    rng = np.random.default_rng(6)
    for n, k, N in ((7, 4, 2880), (33, 2, 64)):
        y = (rng.standard_normal((n, k, N)) * 5).astype(np.float32)
        w = O.f32_to_bf16(rng.random((n, k)).astype(np.float32))
        x = O.make_input(9, n, hidden=N)
        got = host_bf16(native.gemv_gating(f32_dev(y), bf16_dev(w)))
        assert np.array_equal(got, O.gating(y, w))
        got = host_bf16(native.gemv_gating(f32_dev(y), bf16_dev(w), bf16_dev(x)))
        assert np.array_equal(got, O.residual_add(x, O.gating(y, w)))


@pytest.mark.parametrize("n,seed", [(520, 29), (64, 30)])
def test_mlp1_swiglu_pieces(native, block20b, n, seed):
    """moe_mlp1_swiglu_pieces (the block's prefill mlp1: the tiled GEMM's
    epilogue encodes act, n = 520; below 48 pairs per expert the GEMV and the
    encoding pass, n = 64) = quantize_pieces(mlp1_swiglu(...), 3), bit for bit."""
    p, blk = block20b
    x = bf16_dev(O.make_input(seed, n)).view(1, n, 2880)
    st = blk.forward_staged(x)
    t_pk = native.quantize_pieces(st["t"], 2)
    perm, k, nk = st["perm"], 4, n * 4
    pk, _ = native.mlp1_swiglu_pieces(t_pk, n, 2880, perm["indptr"], perm["sorted_pairs"], k,
                                      blk.mlp1_weight_blocks, blk.mlp1_weight_scales,
                                      blk.mlp1_bias, 1.702, blk.swiglu_limit)
    ref = PM.unpack(host(native.quantize_pieces(st["act"].contiguous(), 3)), nk, 2880, 3)
    for a, b in zip(PM.unpack(host(pk), nk, 2880, 3), ref):
        assert np.array_equal(a, b), np.argwhere(a != b)[:4]
    st2 = blk.forward_staged(x, pieces_epilogue=True)
    assert np.array_equal(host_bf16(st2["out"]), host_bf16(st["out"]))
