"""Config 4's mixed step captured in one HIP graph.

Chained 20B-shape MoE blocks (RMSNorm -> MoE -> residual add, the MoE half
of the reference's layer loop, model/transformer.py:59-60 -> mlp.py:371-402)
with independent seeded weights per layer, over one mixed step: 32 decode
tokens routed with the layer's own router bias (near uniform) and a
2048-token prefill chunk routed with that bias plus the Zipf(1.1) profile at
beta 0.5 (the two token groups use views of the same layer weights,
MLPBlock.with_gate_bias).  The step (MoEStack.forward: every call of every
layer, nothing allocated) is captured with torch.cuda.CUDAGraph and replayed:

* every replay equals the eager step bit for bit, with eager work and host
  synchronisations between the replays, and with new inputs copied into the
  captured input buffers;
* layer 0 of each token group matches the oracle (all 32 decode tokens; a
  32-token prefill sample with half its tokens on the hottest expert).
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host_bf16, make_block  # noqa: E402

pytestmark = pytest.mark.gpu

LAYERS, N_DEC, N_PRE, H = 3, 32, 2048, 2880
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def zipf_bias(E: int, beta: float) -> np.ndarray:
    p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
    return beta * np.log(p / p.sum())


@pytest.fixture(scope="module")
def mixed():
    from model.stack import MoEStack
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    params, layers = [], []
    for layer in range(LAYERS):
        p = O.make_params(seed=600 + layer)
        dec = make_block(p)
        gb = O.bf16_to_f32(p.gate_b).astype(np.float64) + zipf_bias(32, 0.5)
        pre_bias = O.f32_to_bf16(gb.astype(np.float32))
        pre = dec.with_gate_bias(bf16_dev(pre_bias))
        params.append((p, pre_bias))
        layers.append((dec, pre))
    stack = MoEStack(layers)
    stack.reserve(N_DEC, N_PRE)
    return params, stack


def _inputs(seed):
    return O.make_input(seed, N_DEC), O.make_input(seed + 1, N_PRE)


def test_layer0_matches_oracle(mixed, oracle_lib):
    params, stack = mixed
    (p, pre_bias) = params[0]
    dec, pre = stack.layers[0]
    xd, xp = _inputs(610)
    out_d = host_bf16(dec(bf16_dev(xd).view(1, N_DEC, H)).view(N_DEC, H))
    m = O.compare_outputs(out_d, O.block_forward(xd, p).out)
    assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m
    out_p = host_bf16(pre(bf16_dev(xp).view(1, N_PRE, H)).view(N_PRE, H))
    pz = O.BlockParams(p.norm_w, p.gate_w, pre_bias, p.mlp1_blocks, p.mlp1_scales, p.mlp1_bias,
                       p.mlp2_blocks, p.mlp2_scales, p.mlp2_bias)
    _, idx = O.topk_softmax(O.router_logits(O.rms_norm(xp, p.norm_w), p.gate_w, pre_bias), 4)
    counts = np.bincount(idx.reshape(-1), minlength=32)
    assert counts.max() > 3 * counts.mean()  # the prefill group is Zipf-skewed
    hot = np.flatnonzero((idx == counts.argmax()).any(axis=1))
    rng = np.random.default_rng(611)
    sel = np.unique(np.concatenate([rng.choice(hot, 16, replace=False),
                                    rng.choice(N_PRE, 16, replace=False)]))
    ref, _, ref_idx, _ = oracle_lib.block_forward(np.ascontiguousarray(xp[sel]), pz,
                                                  nthreads=THREADS)
    assert np.array_equal(ref_idx, idx[sel])
    m = O.compare_outputs(out_p[sel], ref)
    assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m


def test_graph_replay_equals_eager(mixed):
    params, stack = mixed
    xd0, xp0 = _inputs(620)
    xd_s = bf16_dev(xd0).view(1, N_DEC, H)     # captured input buffers
    xp_s = bf16_dev(xp0).view(1, N_PRE, H)

    def eager(xd, xp):
        od, op = stack(bf16_dev(xd).view(1, N_DEC, H), bf16_dev(xp).view(1, N_PRE, H))
        return host_bf16(od), host_bf16(op)

    ref0 = eager(xd0, xp0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack(xd_s, xp_s)                       # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        od_s, op_s = stack(xd_s, xp_s)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host_bf16(od_s), ref0[0]), f"replay {rep}: decode group"
        assert np.array_equal(host_bf16(op_s), ref0[1]), f"replay {rep}: prefill group"
        other = eager(*_inputs(630 + rep))      # eager work between replays
        torch.cuda.synchronize()
        assert np.isfinite(O.bf16_to_f32(other[0])).all()
    # new inputs through the captured buffers
    xd1, xp1 = _inputs(640)
    ref1 = eager(xd1, xp1)
    xd_s.copy_(bf16_dev(xd1).view(1, N_DEC, H))
    xp_s.copy_(bf16_dev(xp1).view(1, N_PRE, H))
    graph.replay()
    torch.cuda.synchronize()
    assert np.array_equal(host_bf16(od_s), ref1[0])
    assert np.array_equal(host_bf16(op_s), ref1[1])
    assert not np.array_equal(ref1[1], ref0[1])
