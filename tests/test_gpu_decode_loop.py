"""The decode loop on the GPU: embedding -> 2 x (AttentionBlock, MLPBlock) ->
final norm -> unembedding -> top-p sampling, driven through the Engine as
the reference's chat loop drives its own (engine.py:133-174, chat.py:62-101),
against the oracle (oracle/attn_oracle.py: OracleModel, the restated TVM
sampler).

* The sampler at the full gpt-oss vocabulary (201088) against the oracle's
  restatement (exact masses): the same token, on flat and peaked logits, at
  the engine's parameters and at the edges (argmax, top_p 1, u near 1 and 0).
* The loop: the GPU samples each next token and runs the next step; at every
  step the oracle replays each sub-block on the GPU's own input to that
  sub-block (the attention block with a cache built from the GPU's earlier
  inputs), because MoE routing turns a last-bit difference in a block's input
  into a different expert for tokens near a top-k tie, so two implementations
  drift apart across layers on random weights (measured: 21% of one layer's
  outputs differ after such flips).  On the same input, each attention block
  and each MoE block meets the block bar (norm-relative max error 1e-2, MAE
  1e-3; MoE routing bit-exact), the logits equal the oracle's final norm and
  unembedding of the GPU's last block output to within one bf16 ulp on at
  most 1% of the vocabulary (at decode the norm runs inside the unembedding
  GEMV), and each sampled token equals the oracle sampler's on the GPU's
  logits.
* popn / extend: rolling the cache back and extending it replays the same way.
* The decode step captured in one HIP graph (Engine.capture_decode) and
  replayed gives the eager steps' tokens and logits bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import attn_oracle as AO  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host_bf16, u8_dev  # noqa: E402

pytestmark = pytest.mark.gpu

VOCAB_FULL = 201088


@pytest.fixture(scope="module")
def A():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import attn_native
    return attn_native


def _sample_ok(logits_f32, temperature, top_p, u, got):
    return got == AO.sample_top_p_from_logits(logits_f32, temperature, top_p, u)


@pytest.mark.parametrize("sigma", [0.5, 2.0, 8.0])
def test_sampler_full_vocab(A, sigma):
    rng = np.random.default_rng(int(sigma * 10))
    B = 3
    logits = O.f32_to_bf16(rng.standard_normal((B, VOCAB_FULL), dtype=np.float32) * sigma)
    lf = O.bf16_to_f32(logits)
    ws = A.sample_workspace(B)
    dev = bf16_dev(logits)
    for temperature, top_p, u in [(0.7, 0.9, 0.5), (0.0, 0.9, 0.5), (1.0, 1.0, 0.999),
                                  (0.3, 0.5, 0.1), (0.7, 0.9, 0.0)]:
        ids = A.sample_top_p(dev, temperature, top_p, u, ws).cpu().numpy()
        again = A.sample_top_p(dev, temperature, top_p, u, ws).cpu().numpy()
        np.testing.assert_array_equal(ids, again)      # the histogram is left zeroed
        for b in range(B):
            assert _sample_ok(lf[b], temperature, top_p, u, int(ids[b])), (temperature, top_p, u, b)
    per_seq = ws.view(torch.int32).view(B, -1)
    assert int(per_seq[:, :65537].abs().sum().item()) == 0     # counts and maximum


def test_sampler_ties_take_index_order(A):
    logits = np.zeros((1, 1000), dtype=np.float32)
    logits[0, [10, 500, 900]] = 5.0                # three tied leaders, the rest flat
    ws = A.sample_workspace(1)
    for u in (0.1, 0.4, 0.7, 0.95):
        got = int(A.sample_top_p(bf16_dev(O.f32_to_bf16(logits)), 1.0, 0.9, u, ws).item())
        assert got == AO.sample_top_p_from_logits(logits[0], 1.0, 0.9, u)


def test_sampler_short_cut_to_argmax(A):
    """TVM's SampleTopPFromProb returns the argmax when uniform < p_max /
    top_p.  Three leaders with p_max about 0.47 over a flat tail (-30: no
    mass to speak of): at u = 0.5, top_p = 0.9 the leader; just above
    p_max / top_p the second one (the crossing)."""
    logits = np.full((1, 4096), -30.0, dtype=np.float32)
    logits[0, [700, 20, 3000]] = [2.0, 1.875, 0.5625]
    ws = A.sample_workspace(1)
    dev = bf16_dev(O.f32_to_bf16(logits))
    for u, want in ((0.5, 700), (0.45, 700), (0.53, 20), (0.95, 3000)):
        got = int(A.sample_top_p(dev, 1.0, 0.9, u, ws).item())
        assert got == want == AO.sample_top_p_from_logits(logits[0], 1.0, 0.9, u), (u, got)


def _model_from_oracle(mp: AO.ModelParams, config):
    from engine import Engine
    eng = Engine(config=config, max_total_seq_len=1024)
    m = eng.model
    with torch.no_grad():
        m.model.embedding.weight.copy_(bf16_dev(mp.embedding))
        m.unembedding.weight.copy_(bf16_dev(mp.unembedding))
        m.model.norm.weight.copy_(bf16_dev(mp.norm_w))
        for blk, (ap, bp) in zip(m.model.block, mp.layers):
            a = blk.attn
            a.sinks.copy_(bf16_dev(ap.sinks))
            a.norm.weight.copy_(bf16_dev(ap.norm_w))
            a.qkv.weight.copy_(bf16_dev(ap.qkv_w))
            a.qkv.bias.copy_(bf16_dev(ap.qkv_b))
            a.out.weight.copy_(bf16_dev(ap.out_w))
            a.out.bias.copy_(bf16_dev(ap.out_b))
            g = blk.mlp
            g.norm.weight.copy_(bf16_dev(bp.norm_w))
            g.gate.weight.copy_(bf16_dev(bp.gate_w))
            g.gate.bias.copy_(bf16_dev(bp.gate_b))
            g.mlp1_weight_blocks.copy_(u8_dev(bp.mlp1_blocks))
            g.mlp1_weight_scales.copy_(u8_dev(bp.mlp1_scales))
            g.mlp1_bias.copy_(bf16_dev(bp.mlp1_bias))
            g.mlp2_weight_blocks.copy_(u8_dev(bp.mlp2_blocks))
            g.mlp2_weight_scales.copy_(u8_dev(bp.mlp2_scales))
            g.mlp2_bias.copy_(bf16_dev(bp.mlp2_bias))
    return eng


class _Replay:
    """Hooks on every sub-block of the GPU model: after each step, the oracle
    replays each sub-block on the GPU's input to it and compares outputs."""

    def __init__(self, eng, mp: AO.ModelParams):
        self.mp = mp
        self.io = {}
        self.seen = {}      # (layer, kind) -> (GPU rows, oracle rows) of the run so far
        blocks = eng.model.model.block
        for i, blk in enumerate(blocks):
            for kind in ("attn", "mlp"):
                getattr(blk, kind).register_forward_hook(self._hook(i, kind))
        empty = np.zeros((0, AO.N_KV_HEADS, AO.HEAD_DIM), dtype=np.uint16)
        self.kc = [empty.copy() for _ in blocks]
        self.vc = [empty.copy() for _ in blocks]

    def _hook(self, i, kind):
        def f(mod, args, out):
            H = out.shape[-1]
            self.io[(i, kind)] = (host_bf16(args[0].reshape(-1, H)), host_bf16(out.reshape(-1, H)))
        return f

    def _bar(self, i, kind, got, ref, what):
        """The block bar (max relative error 1e-2, MAE 1e-3) over the rows of
        the run so far.  A decode step adds one row, too few values for a
        max-normalised error on its own: two bf16 ulps in the row's largest
        binade (0.25 against a maximum of 23.25) already exceed 1e-2, and the
        chain of bf16 roundings (expert output, weighted sum, residual) gives
        that from fp32 sums that differ in their last bits.  The block tests
        apply the same bar over a sample of tokens."""
        g0, r0 = self.seen.get((i, kind), (got[:0], ref[:0]))
        g, r = np.concatenate([g0, got]), np.concatenate([r0, ref])
        self.seen[(i, kind)] = (g, r)
        m = O.compare_outputs(g, r)
        assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, (what, i, kind, m)
        m = O.compare_outputs(got, ref)                   # this step's rows alone
        assert m["mae"] <= 1e-3, (what, i, kind, m)

    def check(self, logits_f32, what):
        for i, (ap, bp) in enumerate(self.mp.layers):
            x_in, got = self.io[(i, "attn")]
            ref, k, v = AO.attn_block_forward(x_in, ap, self.kc[i], self.vc[i],
                                              AO.SLIDING_WINDOW if i % 2 == 0 else 0)
            self.kc[i] = np.concatenate([self.kc[i], k])
            self.vc[i] = np.concatenate([self.vc[i], v])
            self._bar(i, "attn", got, ref, what)
            x_in, got = self.io[(i, "mlp")]
            self._bar(i, "mlp", got, O.block_forward(x_in, bp).out, what)
        last_out = self.io[(len(self.mp.layers) - 1, "mlp")][1]
        h = O.rms_norm(last_out[-1:], self.mp.norm_w)   # the final norm (bit-exact kernels)
        own = AO.bf16_to_f32(AO.linear(h, self.mp.unembedding, None))[-1]
        d = O.compare_outputs(O.f32_to_bf16(logits_f32), O.f32_to_bf16(own))
        # one bf16 ulp of each logit, or for a logit near zero after
        # cancellation 2^-16 of the largest (fp32 summation order alone moves
        # such a logit by several of its own ulps)
        ulp = np.spacing(np.abs(own).astype(np.float32)) * 2 ** 16
        floor = np.abs(own).max() * 2.0 ** -16
        assert d["frac_diff"] <= 0.01 and np.all(np.abs(logits_f32 - own) <= np.maximum(ulp, floor)), \
            (what, d)


@pytest.fixture(scope="module")
def small_model():
    from model.config import GPTOssConfig
    cfg = GPTOssConfig(num_hidden_layers=2, num_experts=32, vocab_size=4096,
                       context_window_size=1024, prefill_chunk_size=512)
    mp = AO.make_model_params(900, layers=2, vocab=4096)
    return cfg, mp


def test_decode_loop(A, small_model):
    cfg, mp = small_model
    eng = _model_from_oracle(mp, cfg)
    rep = _Replay(eng, mp)
    rng = np.random.default_rng(901)
    prompt = rng.integers(0, cfg.vocab_size, 150).astype(np.int32)   # past the 128 window
    seq = eng.begin_sequence()
    logits = eng.prefill(prompt, seq)
    got = logits.view(-1).cpu().numpy()
    rep.check(got, "prefill")
    p = eng.sample_parameters
    for step in range(5):
        tok = eng.sample(logits)
        assert _sample_ok(got, p["temperature"], p["top_p"], p["random_seed"], tok), step
        logits = eng.decode(np.array([tok], dtype=np.int32), seq)
        got = logits.view(-1).cpu().numpy()
        rep.check(got, f"decode step {step}")
    assert eng.get_kv_total_seq_len() == 155


def test_popn_then_extend(A, small_model):
    cfg, mp = small_model
    eng = _model_from_oracle(mp, cfg)
    rep = _Replay(eng, mp)
    rng = np.random.default_rng(902)
    toks = rng.integers(0, cfg.vocab_size, 40).astype(np.int32)
    seq = eng.begin_sequence()
    rep.check(eng.prefill(toks[:30], seq).view(-1).cpu().numpy(), "prefill")
    for t in toks[30:33]:
        eng.decode(np.array([t]), seq)
    eng.popn(seq, 3)
    assert eng.get_kv_total_seq_len() == 30
    logits = eng.extend(toks[30:40], seq)
    rep.check(logits.view(-1).cpu().numpy(), "extend after popn")


def test_graphed_decode_equals_eager(A, small_model):
    cfg, mp = small_model
    eng = _model_from_oracle(mp, cfg)
    rng = np.random.default_rng(903)
    seq = eng.begin_sequence()
    tok0 = eng.sample_device(eng.prefill(rng.integers(0, cfg.vocab_size, 140).astype(np.int32),
                                         seq)).clone()
    steps = 6
    eng._token.copy_(tok0)
    toks, ref_logits = [], []
    for _ in range(steps):                        # eager steps
        lg = eng.decode(eng._token, seq)
        ref_logits.append(lg.view(-1).cpu().numpy().copy())
        toks.append(int(eng.sample_device(lg).item()))
    eng.popn(seq, steps)
    eng._token.copy_(tok0)
    eng.capture_decode(seq)
    assert int(eng._token.item()) == int(tok0.item())
    for k in range(steps):
        t = eng.decode_sample(seq)
        got = eng.graph_logits.view(-1).cpu().numpy()
        np.testing.assert_array_equal(got, ref_logits[k])
        assert int(t.item()) == toks[k], k
    assert eng.get_kv_total_seq_len() == 140 + steps


def test_captured_step_survives_a_longer_extend(A, small_model):
    """The captured decode step holds the raw addresses of every MoE block's
    workspace.  A later turn that extends the sequence by more tokens than any
    call before the capture (the reference's chat loop, chat.py:157-162) grows
    the eager workspaces; the captured ones must stay alive and untouched by
    eager work.  Sentinel buffers of the captured workspaces' sizes are
    allocated after the extend (torch's allocator would hand a freed workspace
    to them) and must be intact after the replays, and the replayed steps must
    equal eager steps bit for bit."""
    cfg, mp = small_model
    eng = _model_from_oracle(mp, cfg)
    rng = np.random.default_rng(904)
    seq = eng.begin_sequence()
    eng._token.copy_(eng.sample_device(
        eng.prefill(rng.integers(0, cfg.vocab_size, 12).astype(np.int32), seq)))
    eng.capture_decode(seq)
    blocks = [blk.mlp for blk in eng.model.model.block]
    captured = [m._ws.data_ptr() for m in blocks]
    sizes = [m._ws.numel() for m in blocks]
    logits = eng.extend(rng.integers(0, cfg.vocab_size, 200).astype(np.int32), seq)
    assert all(m._ws.data_ptr() != p for m, p in zip(blocks, captured))   # grown
    assert all(any(h.data_ptr() == p for h in m._ws_held) for m, p in zip(blocks, captured))
    sentinels = [torch.full((sz,), 0x5A, dtype=torch.uint8, device="cuda") for sz in sizes]
    tok0 = eng.sample_device(logits).clone()
    eng._token.copy_(tok0)
    steps = 3
    graph_logits, toks = [], []
    for _ in range(steps):
        t = eng.decode_sample(seq)
        graph_logits.append(eng.graph_logits.view(-1).cpu().numpy().copy())
        toks.append(int(t.item()))
    torch.cuda.synchronize()
    for s in sentinels:
        assert bool((s == 0x5A).all().item())
    eng.popn(seq, steps)
    eng._token.copy_(tok0)
    for k in range(steps):
        lg = eng.decode(eng._token, seq)
        np.testing.assert_array_equal(lg.view(-1).cpu().numpy(), graph_logits[k])
        assert int(eng.sample_device(lg).item()) == toks[k], k
    assert eng.get_kv_total_seq_len() == 12 + 200 + steps
