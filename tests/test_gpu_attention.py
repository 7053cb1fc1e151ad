"""GPU parity of the attention-block kernels (include/attn_gfx950.h) against
the oracle (oracle/attn_oracle.py), through the C ABI.

Bit-exact: RMSNorm, the QKV bias + YaRN RoPE (q and the cached k) and the
appended v, bias + residual, the embedding gather.  Within tolerance (fp32
softmax, probabilities as two bf16 pieces on the MFMA, against the oracle's
fp64): decode and prefill / extend attention with the sink scaling, on
scattered page tables, ragged batches, sliding windows, 4096-query prefills
checked on sampled rows (a sharp softmax; row maxima that creep up block by
block under the lazy rescale's headroom), and the whole AttentionBlock at
gpt-oss-20b shape.  Attention outputs are held to a
norm-relative max error of 1e-2 and a mean absolute error of 1e-3 relative to
the mean magnitude (the block bar of the MoE path).
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import attn_oracle as AO  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host_bf16, i32_dev, f32_dev  # noqa: E402

pytestmark = pytest.mark.gpu

D, HQ, HKV, PAGE = 64, 64, 8, 16
SCALE = 1.0 / math.sqrt(D)


@pytest.fixture(scope="module")
def A():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import attn_native
    return attn_native


def bf(x):
    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def close(got, ref, rel=1e-2, mae=1e-3):
    m = O.compare_outputs(got, ref)
    scale = np.abs(O.bf16_to_f32(ref)).mean()
    assert m["max_rel"] <= rel and m["mae"] <= mae * max(scale, 1e-30), m
    assert np.isfinite(O.bf16_to_f32(got)).all()


def test_rms_norm_bit_exact(A):
    x = O.make_input(11, 7)
    w = bf(np.random.default_rng(12).uniform(0.5, 1.5, 2880))
    got = host_bf16(A.rms_norm(bf16_dev(x), bf16_dev(w), 1e-5))
    np.testing.assert_array_equal(got, O.rms_norm(x, w, 1e-5))


def test_bias_residual_and_embedding_bit_exact(A):
    rng = np.random.default_rng(13)
    x, y = O.make_input(14, 5), O.make_input(15, 5)
    b = bf(rng.standard_normal(2880) * 0.1)
    got = host_bf16(A.bias_residual(bf16_dev(x), bf16_dev(y), bf16_dev(b)))
    want = O.f32_to_bf16(O.bf16_to_f32(x) + O.bf16_to_f32(AO.bias_add(y, b)))
    np.testing.assert_array_equal(got, want)
    table = bf(rng.standard_normal((100, 2880)))
    ids = np.array([3, 99, 0, -1, 100, 3], dtype=np.int32)
    got = host_bf16(A.embedding(i32_dev(ids), bf16_dev(table)))
    want = np.where(((ids >= 0) & (ids < 100))[:, None], table[np.clip(ids, 0, 99)], 0)
    np.testing.assert_array_equal(got, want.astype(np.uint16))


def _inv_freq_dev():
    from model.attention import yarn_rope_tables
    from model.config import GPTOssConfig
    inv, conc = yarn_rope_tables(GPTOssConfig())
    np.testing.assert_array_equal(inv, AO.yarn_inv_freq())     # host table == oracle's
    assert np.float32(conc) == AO.yarn_concentration()
    return f32_dev(inv), conc


def test_qkv_rope_append_bit_exact(A):
    rng = np.random.default_rng(21)
    n, pages = 9, 12
    qkv = bf(rng.standard_normal((n, (HQ + 2 * HKV) * D)))
    bias = bf(rng.standard_normal((HQ + 2 * HKV) * D) * 0.1)
    pos = np.array([0, 1, 2, 15, 16, 4095, 4096, 70000, 131071], dtype=np.int32)
    slots = rng.choice(pages * PAGE, n, replace=False).astype(np.int32)
    slots[-1] = pages * PAGE + 5          # outside the pool: not written
    cache = torch.zeros((pages, 2, HKV, PAGE, D), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((n, HQ, D), dtype=torch.bfloat16, device="cuda")
    inv, conc = _inv_freq_dev()
    A.qkv_rope_append(bf16_dev(qkv), bf16_dev(bias), i32_dev(pos), i32_dev(slots), inv, conc,
                      cache, q)
    ref = AO.bias_add(qkv, bias)
    rq, rk, rv = AO.split_qkv(ref)
    np.testing.assert_array_equal(host_bf16(q), AO.rope(rq, pos))
    rk = AO.rope(rk, pos)
    c = host_bf16(cache)
    want = np.zeros_like(c)
    for i in range(n - 1):
        pg, sl = divmod(int(slots[i]), PAGE)
        want[pg, 0, :, sl] = rk[i]
        want[pg, 1, :, sl] = rv[i]
    np.testing.assert_array_equal(c, want)


class PagedSeqs:
    """Random keys / values of a few sequences laid out in a scattered page pool."""

    def __init__(self, seed, lengths, pages=None, kv=None):
        rng = np.random.default_rng(seed)
        need = [-(-L // PAGE) for L in lengths]
        pool = pages or sum(need) + 3
        perm = rng.permutation(pool)
        if kv is None:
            self.k = [bf(rng.standard_normal((L, HKV, D))) for L in lengths]
            self.v = [bf(rng.standard_normal((L, HKV, D))) for L in lengths]
        else:   # given keys and values (bf16 bits) per sequence
            self.k = [k for k, _ in kv]
            self.v = [v for _, v in kv]
        cache = bf(rng.standard_normal((pool, 2, HKV, PAGE, D)))   # unused slots: garbage
        indptr, ids, off = [0], [], 0
        for L, k, v, npg in zip(lengths, self.k, self.v, need):
            mine = perm[off:off + npg]
            off += npg
            for p in range(L):
                cache[mine[p // PAGE], 0, :, p % PAGE] = k[p]
                cache[mine[p // PAGE], 1, :, p % PAGE] = v[p]
            ids.extend(mine.tolist())
            indptr.append(len(ids))
        self.cache = bf16_dev(cache)
        self.page_indptr = i32_dev(np.array(indptr))
        self.page_indices = i32_dev(np.array(ids))
        self.kv_len = i32_dev(np.array(lengths))
        self.lengths = lengths


@pytest.mark.parametrize("window", [0, 128])
def test_decode_attention(A, window):
    lengths = [1, 130, 1000, 4100]
    seqs = PagedSeqs(31, lengths)
    rng = np.random.default_rng(32)
    q = bf(rng.standard_normal((len(lengths), HQ, D)))
    sinks = bf(rng.standard_normal(HQ))
    span = max(min(L, window) if window else L for L in lengths)
    ws = A.decode_workspace(len(lengths), span)
    out = torch.empty((len(lengths), HQ, D), dtype=torch.bfloat16, device="cuda")
    A.decode(bf16_dev(q), seqs.cache, seqs.page_indptr, seqs.page_indices, seqs.kv_len, span,
             window, SCALE, bf16_dev(sinks), out, ws)
    got = host_bf16(out)
    for b, L in enumerate(lengths):
        o, lse = AO.attention(q[b:b + 1], seqs.k[b], seqs.v[b], np.array([L - 1]), window)
        close(got[b:b + 1], AO.sink_scale(o, lse, sinks))


@pytest.mark.parametrize("L", [129, 200, 256, 257, 600])
def test_decode_attention_one_sequence(A, L):
    """One sequence: a span of at most two 128-key chunks is one split (both
    chunks in one workgroup, no merge), longer spans split by chunk and
    merge; the span bound is far above the length."""
    seqs = PagedSeqs(37 + L, [L])
    rng = np.random.default_rng(38 + L)
    q = bf(rng.standard_normal((1, HQ, D)))
    sinks = bf(rng.standard_normal(HQ))
    ws = A.decode_workspace(1, 4096)
    out = torch.empty((1, HQ, D), dtype=torch.bfloat16, device="cuda")
    A.decode(bf16_dev(q), seqs.cache, seqs.page_indptr, seqs.page_indices, seqs.kv_len, 4096, 0,
             SCALE, bf16_dev(sinks), out, ws)
    o, lse = AO.attention(q, seqs.k[0], seqs.v[0], np.array([L - 1]), 0)
    close(host_bf16(out), AO.sink_scale(o, lse, sinks))


def test_decode_attention_reused_workspace_and_large_bound(A):
    """The last split of each (sequence, kv head) to finish merges the
    group; its arrival counts live in the workspace and are left zero, so
    calls in a row on one workspace agree bit for bit, also with a span bound
    far above the lengths (the split count a captured graph fixes: splits past
    a sequence's keys do nothing)."""
    lengths = [1, 130, 1000, 4100]
    seqs = PagedSeqs(35, lengths)
    rng = np.random.default_rng(36)
    q = bf16_dev(bf(rng.standard_normal((len(lengths), HQ, D))))
    sinks = bf16_dev(bf(rng.standard_normal(HQ)))
    outs = []
    ws = A.decode_workspace(len(lengths), 40960)
    for span in (4100, 40960, 4100):
        for _ in range(2):
            out = torch.empty((len(lengths), HQ, D), dtype=torch.bfloat16, device="cuda")
            A.decode(q, seqs.cache, seqs.page_indptr, seqs.page_indices, seqs.kv_len, span, 0,
                     SCALE, sinks, out, ws)
            outs.append(host_bf16(out))
        assert int(ws[:32 * len(lengths)].count_nonzero()) == 0   # arrival counts left zero
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("L,bound", [(300, 200), (200, 100)])
def test_decode_span_too_small_is_nan(A, L, bound):
    """A span bound below the length gives NaN, also where the span would fit
    one split of two chunks (the bound fixes the splits' reach)."""
    seqs = PagedSeqs(33, [L])
    q = bf(np.random.default_rng(34).standard_normal((1, HQ, D)))
    ws = A.decode_workspace(1, L)
    out = torch.empty((1, HQ, D), dtype=torch.bfloat16, device="cuda")
    A.decode(bf16_dev(q), seqs.cache, seqs.page_indptr, seqs.page_indices, seqs.kv_len, bound, 0,
             SCALE, bf16_dev(bf(np.zeros(HQ))), out, ws)
    assert np.isnan(O.bf16_to_f32(host_bf16(out))).all()


@pytest.mark.parametrize("window", [0, 128])
@pytest.mark.parametrize("qlens", [[300], [1, 64, 65, 200]])
def test_prefill_attention(A, window, qlens):
    # the last q_len tokens of each sequence are the queries: with a cached
    # prefix (extend) for all but the first sequence
    prefix = [0, 5, 100, 37][:len(qlens)]
    lengths = [p + q for p, q in zip(prefix, qlens)]
    seqs = PagedSeqs(41 + len(qlens), lengths)
    rng = np.random.default_rng(42)
    n = sum(qlens)
    q = bf(rng.standard_normal((n, HQ, D)))
    sinks = bf(rng.standard_normal(HQ))
    q_indptr = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    out = torch.empty((n, HQ, D), dtype=torch.bfloat16, device="cuda")
    A.prefill(bf16_dev(q), i32_dev(q_indptr), max(qlens), seqs.cache, seqs.page_indptr,
              seqs.page_indices, seqs.kv_len, window, SCALE, bf16_dev(sinks), out)
    got = host_bf16(out)
    for b, (L, ql) in enumerate(zip(lengths, qlens)):
        rows = slice(q_indptr[b], q_indptr[b + 1])
        o, lse = AO.attention(q[rows], seqs.k[b], seqs.v[b], np.arange(L - ql, L), window)
        close(got[rows], AO.sink_scale(o, lse, sinks))


def _prefill_sampled(A, seqs, prefix, q, sinks, window, rows):
    """One sequence's prefill (its last q.shape[0] positions are the queries)
    checked on the sampled query rows: attention is per query, so the
    oracle's output for those rows alone is their reference."""
    n = q.shape[0]
    L = prefix + n
    out = torch.empty((n, HQ, D), dtype=torch.bfloat16, device="cuda")
    A.prefill(bf16_dev(q), i32_dev(np.array([0, n], dtype=np.int32)), n, seqs.cache,
              seqs.page_indptr, seqs.page_indices, seqs.kv_len, window, SCALE, bf16_dev(sinks),
              out)
    got = host_bf16(out)
    o, lse = AO.attention(q[rows], seqs.k[0], seqs.v[0], np.arange(prefix, L)[rows], window)
    close(got[rows], AO.sink_scale(o, lse, sinks))
    assert np.isfinite(O.bf16_to_f32(got)).all()


def _sample_rows(n, seed):
    """Rows at both ends, on both sides of every 64-row tile edge, and at random."""
    rng = np.random.default_rng(seed)
    edges = [e + d for e in range(64, n, 64 * 7) for d in (-1, 0)]
    rows = set(range(16)) | set(range(n - 16, n)) | set(edges)
    rows |= set(rng.choice(n, 64, replace=False).tolist())
    return np.array(sorted(r for r in rows if 0 <= r < n))


@pytest.mark.parametrize("window", [0, 128])
def test_prefill_attention_long_sharp(A, window):
    """4096 queries after an unaligned 300-token prefix (64 query tiles, up to
    69 key blocks each, the last block of every tile past its diagonal), with
    q scaled by 4 so that the softmax is sharp and row maxima jump between
    blocks (the lazy rescale's reference moves often)."""
    prefix, n = 300, 4096
    seqs = PagedSeqs(51, [prefix + n])
    rng = np.random.default_rng(52)
    q = bf(4.0 * rng.standard_normal((n, HQ, D)))
    sinks = bf(rng.standard_normal(HQ))
    _prefill_sampled(A, seqs, prefix, q, sinks, window, _sample_rows(n, 53))


def test_prefill_attention_creeping_maximum(A):
    """Keys with a component along a fixed direction u that grows with the
    position, queries along u: every row's maximum score rises a little with
    each 64-key block, by less than the 2^8 headroom of the lazy rescale, so
    the reference point stays behind and p reaches about 2^8 before it
    moves.  Scores span about 60 in log2 units along a row."""
    n = 2048
    rng = np.random.default_rng(54)
    u = rng.standard_normal(D)
    u /= np.linalg.norm(u)
    pos = np.arange(n, dtype=np.float64)
    k = 0.5 * rng.standard_normal((n, HKV, D)) + (pos * (40.0 / n))[:, None, None] * u
    v = rng.standard_normal((n, HKV, D))
    q = 0.5 * rng.standard_normal((n, HQ, D)) + 8.0 * u
    seqs = PagedSeqs(55, [n], kv=[(bf(k), bf(v))])
    sinks = bf(rng.standard_normal(HQ))
    _prefill_sampled(A, seqs, 0, bf(q), sinks, 0, _sample_rows(n, 56))


def _block(A, p, layer_idx):
    from model.attention import AttentionBlock
    from model.config import GPTOssConfig
    blk = AttentionBlock(GPTOssConfig(), layer_idx=layer_idx, device="cuda")
    with torch.no_grad():
        blk.sinks.copy_(bf16_dev(p.sinks))
        blk.norm.weight.copy_(bf16_dev(p.norm_w))
        blk.qkv.weight.copy_(bf16_dev(p.qkv_w))
        blk.qkv.bias.copy_(bf16_dev(p.qkv_b))
        blk.out.weight.copy_(bf16_dev(p.out_w))
        blk.out.bias.copy_(bf16_dev(p.out_b))
    return blk


@pytest.mark.parametrize("layer_idx", [0, 1])  # sliding window 128, full attention
def test_attention_block_prefill_then_decode(A, layer_idx):
    """AttentionBlock at 20B shape: a 150-token prefill then three decode
    steps through the paged cache, each against the oracle's block."""
    from model.kv_cache import PagedKVCache
    p = AO.make_attn_params(51 + layer_idx)
    blk = _block(A, p, layer_idx)
    cache = PagedKVCache(num_layers=2, num_pages=64, max_batch=2, max_tokens=256)
    cache.add_sequence(0)
    cache.enable_sliding_window(0, 128)
    window = 128 if layer_idx % 2 == 0 else 0
    n0 = 150
    x = O.make_input(52, n0 + 3)
    kc = np.zeros((0, HKV, D), dtype=np.uint16)
    vc = kc.copy()
    steps = [(0, n0), (n0, n0 + 1), (n0 + 1, n0 + 2), (n0 + 2, n0 + 3)]
    for a, b in steps:
        cache.begin_forward([0], [b - a])
        got = host_bf16(blk(bf16_dev(x[a:b]).view(1, b - a, 2880), cache).view(b - a, 2880))
        cache.end_forward()
        ref, k_new, v_new = AO.attn_block_forward(x[a:b], p, kc, vc, window)
        kc, vc = np.concatenate([kc, k_new]), np.concatenate([vc, v_new])
        m = O.compare_outputs(got, ref)
        assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, (a, b, m)
    assert cache.seq_len(0) == n0 + 3


def _ulp_close(got, ref, what, frac=0.01):
    """Equal but for fp32 summation order: at most `frac` of the elements
    differ, each by one bf16 ulp of its value, or -- for results near zero
    after cancellation -- by at most 2^-16 of the largest magnitude (far above
    fp32 accumulation error, far below one bf16 ulp of typical values)."""
    g, r = O.bf16_to_f32(got).astype(np.float64), O.bf16_to_f32(ref).astype(np.float64)
    ulp = np.spacing(np.abs(r).astype(np.float32)).astype(np.float64) * 2 ** 16
    floor = np.abs(r).max() * 2.0 ** -16
    diff = np.abs(g - r)
    assert (diff > 0).mean() <= frac and np.all(diff <= np.maximum(ulp, floor)), \
        (what, (diff > 0).mean(), (diff / np.maximum(ulp, floor)).max())


@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemv_kernels(A, M):
    """The decode-sized projections: unembedding-shaped GEMV, the output
    projection with bias + residual, and the QKV projection with bias, RoPE
    and the cache append, against the oracle's nn.Linear and RoPE."""
    rng = np.random.default_rng(60 + M)
    K, N = 2880, 4096 + 40          # N not a multiple of the row block
    x = bf(rng.standard_normal((M, K)))
    W = bf(rng.standard_normal((N, K)) * 0.02)
    _ulp_close(host_bf16(A.gemv(bf16_dev(x), bf16_dev(W))), AO.linear(x, W, None), "gemv")
    nw = bf(rng.uniform(0.5, 1.5, K))
    xr = O.make_input(62, M)
    got = host_bf16(A.gemv(bf16_dev(xr), bf16_dev(W), norm_w=bf16_dev(nw), eps=1e-5))
    _ulp_close(got, AO.linear(O.rms_norm(xr, nw, 1e-5), W, None), "norm + gemv")
    Ko, No = 4096, 2880
    o = bf(rng.standard_normal((M, Ko)) * 0.3)
    Wo = bf(rng.standard_normal((No, Ko)) * 0.02)
    bo = bf(rng.standard_normal(No) * 0.01)
    res = O.make_input(61, M)
    got = host_bf16(A.gemv_bias_residual(bf16_dev(o), bf16_dev(Wo), bf16_dev(bo), bf16_dev(res)))
    want = O.f32_to_bf16(O.bf16_to_f32(res) + O.bf16_to_f32(AO.linear(o, Wo, bo)))
    _ulp_close(got, want, "out projection", frac=0.02)
    Wq = bf(rng.standard_normal(((HQ + 2 * HKV) * D, K)) * 0.02)
    bq = bf(rng.standard_normal((HQ + 2 * HKV) * D) * 0.01)
    pos = np.arange(100, 100 + M, dtype=np.int32) * 37
    pages = 4
    slots = rng.choice(pages * PAGE, M, replace=False).astype(np.int32)
    cache = torch.zeros((pages, 2, HKV, PAGE, D), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((M, HQ, D), dtype=torch.bfloat16, device="cuda")
    inv, conc = _inv_freq_dev()
    xq = O.make_input(63, M)
    A.qkv_gemv_rope_append(bf16_dev(xq), bf16_dev(Wq), bf16_dev(bq), i32_dev(pos), i32_dev(slots),
                           inv, conc, cache, q, norm_w=bf16_dev(nw), eps=1e-5)
    rq, rk, rv = AO.split_qkv(AO.linear(O.rms_norm(xq, nw, 1e-5), Wq, bq))
    _ulp_close(host_bf16(q), AO.rope(rq, pos), "q", frac=0.03)
    c = host_bf16(cache)
    rk = AO.rope(rk, pos)
    for i in range(M):
        pg, sl = divmod(int(slots[i]), PAGE)
        _ulp_close(c[pg, 0, :, sl], rk[i], "k", frac=0.03)
        _ulp_close(c[pg, 1, :, sl], rv[i], "v", frac=0.03)
