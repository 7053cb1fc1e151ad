"""Config 4's mixed step at its stated depth, captured in one HIP graph.

24 chained 20B-shape MoE blocks (RMSNorm -> MoE -> residual add, the MoE half
of the reference's layer loop, model/transformer.py:59-60 -> mlp.py:371-402)
with independent seeded weights per layer, over one mixed step: 32 decode
tokens routed with the layer's own router bias (near uniform) and a
2048-token prefill chunk routed with that bias plus the Zipf(1.1) profile at
beta 0.5 (the two token groups use views of the same layer weights,
MLPBlock.with_gate_bias).  The stack is bench.py's own (``mixed_stack``: the
same seeds and distributions), so the step the bench times is the step
checked here.  The step (MoEStack.forward: every call of every layer,
nothing allocated) is captured with torch.cuda.CUDAGraph and replayed:

* the eager step equals the layers run one call at a time (every layer's
  output of both groups kept), bit for bit;
* every replay equals the eager step bit for bit, with eager work and host
  synchronisations between the replays, and with new inputs copied into the
  captured input buffers;
* layers 0, 12 and 23 of each token group match the oracle on the GPU's own
  input to that layer (all 32 decode tokens; a 32-token prefill sample with
  half its tokens on the layer's hottest expert), routing bit-exact.
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host, host_bf16  # noqa: E402

pytestmark = pytest.mark.gpu

LAYERS, N_DEC, N_PRE, H = 24, 32, 2048, 2880
CHECKED = (0, 12, 23)
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.fixture(scope="module")
def stack():
    import bench
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    print(f"config 4: building {LAYERS} layers", flush=True)
    s = bench.mixed_stack(torch.device("cuda:0"), LAYERS, N_DEC, N_PRE)
    torch.cuda.synchronize()
    return s


def _inputs(seed):
    return O.make_input(seed, N_DEC), O.make_input(seed + 1, N_PRE)


def _params_host(blk) -> O.BlockParams:
    """A block's nine parameters copied back in the oracle's format."""
    return O.BlockParams(host_bf16(blk.norm.weight), host_bf16(blk.gate.weight),
                         host_bf16(blk.gate.bias), host(blk.mlp1_weight_blocks),
                         host(blk.mlp1_weight_scales), host_bf16(blk.mlp1_bias),
                         host(blk.mlp2_weight_blocks), host(blk.mlp2_weight_scales),
                         host_bf16(blk.mlp2_bias))


def _chain(stack, xd, xp):
    """Every layer's input and output per group, one forward_into call at a
    time through the stack's workspace: ins[g][l], outs[g][l] (device)."""
    ins, outs = ([], []), ([], [])
    cur = [bf16_dev(xd), bf16_dev(xp)]
    for layer in stack.layers:
        for g, blk in enumerate(layer):
            nxt = torch.empty_like(cur[g])
            blk.forward_into(cur[g], nxt, stack._ws)
            ins[g].append(cur[g])
            outs[g].append(nxt)
            cur[g] = nxt
    return ins, outs


def test_deep_layers_match_oracle(stack, oracle_lib):
    xd, xp = _inputs(610)
    ins, outs = _chain(stack, xd, xp)
    rng = np.random.default_rng(611)
    for layer in CHECKED:
        dec, pre = stack.layers[layer]
        p = _params_host(dec)
        pre_bias = host_bf16(pre.gate.bias)
        for g, (n, bias) in enumerate(((N_DEC, p.gate_b), (N_PRE, pre_bias))):
            print(f"config 4: layer {layer} group {g} vs oracle", flush=True)
            x_in = host_bf16(ins[g][layer])
            out = host_bf16(outs[g][layer])
            pg = O.BlockParams(p.norm_w, p.gate_w, bias, p.mlp1_blocks, p.mlp1_scales,
                               p.mlp1_bias, p.mlp2_blocks, p.mlp2_scales, p.mlp2_bias)
            if g == 0:
                sel = np.arange(n)
            else:
                _, idx = O.topk_softmax(O.router_logits(O.rms_norm(x_in, p.norm_w), p.gate_w,
                                                        bias), 4)
                counts = np.bincount(idx.reshape(-1), minlength=32)
                assert counts.max() > 3 * counts.mean(), counts   # Zipf-skewed
                hot = np.flatnonzero((idx == counts.argmax()).any(axis=1))
                sel = np.unique(np.concatenate([rng.choice(hot, 16, replace=False),
                                                rng.choice(n, 16, replace=False)]))
            ref, _, ref_idx, _ = oracle_lib.block_forward(np.ascontiguousarray(x_in[sel]), pg,
                                                          nthreads=THREADS)
            _, idx_sel = O.topk_softmax(O.router_logits(O.rms_norm(x_in[sel], p.norm_w),
                                                        p.gate_w, bias), 4)
            assert np.array_equal(ref_idx, idx_sel)
            m = O.compare_outputs(out[sel], ref)
            assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, (layer, g, m)


def test_graph_replay_equals_eager(stack):
    xd0, xp0 = _inputs(620)
    xd_s = bf16_dev(xd0).view(1, N_DEC, H)     # captured input buffers
    xp_s = bf16_dev(xp0).view(1, N_PRE, H)

    def eager(xd, xp):
        od, op = stack(bf16_dev(xd).view(1, N_DEC, H), bf16_dev(xp).view(1, N_PRE, H))
        return host_bf16(od), host_bf16(op)

    ref0 = eager(xd0, xp0)
    _, outs = _chain(stack, xd0, xp0)            # the same layers one call at a time
    assert np.array_equal(host_bf16(outs[0][-1]), ref0[0].reshape(N_DEC, H))
    assert np.array_equal(host_bf16(outs[1][-1]), ref0[1].reshape(N_PRE, H))
    # the chain's layers differ from one another (every layer ran)
    assert not np.array_equal(host_bf16(outs[1][-2]), host_bf16(outs[1][-1]))
    del outs
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
        print(f"config 4: replay {rep}", flush=True)
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
