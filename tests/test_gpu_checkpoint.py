"""Checkpoint path on the GPU: a safetensors file with the gpt-oss checkpoint's
tensor names (block.N.mlp.*, weights.py:102-113 naming) is loaded by
TorchCheckpoint straight onto the device (weights.py:76-96: safetensors ->
device tensors, MXFP4 kept packed as uint8), each layer's MLPBlock runs its
forward, and the output is held to the block bar against the oracle run on
the parameters that were written."""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from safetensors.torch import save_file  # noqa: E402

from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host_bf16  # noqa: E402

pytestmark = pytest.mark.gpu


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("E,H,inter,n", [(8, 128, 96, 9), (32, 2880, 2880, 16)])
def test_checkpoint_forward(tmp_path, E, H, inter, n):
    import weights as W
    from model.config import GPTOssConfig
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    layers = 2
    params = [O.make_params(70 + i, num_experts=E, hidden=H, inter=inter) for i in range(layers)]
    tensors = {}
    for i, p in enumerate(params):
        pre = f"block.{i}.mlp."
        tensors.update({
            pre + "norm.scale": _bf16(p.norm_w), pre + "gate.weight": _bf16(p.gate_w),
            pre + "gate.bias": _bf16(p.gate_b),
            pre + "mlp1_weight.blocks": torch.from_numpy(p.mlp1_blocks),
            pre + "mlp1_weight.scales": torch.from_numpy(p.mlp1_scales),
            pre + "mlp1_bias": _bf16(p.mlp1_bias),
            pre + "mlp2_weight.blocks": torch.from_numpy(p.mlp2_blocks),
            pre + "mlp2_weight.scales": torch.from_numpy(p.mlp2_scales),
            pre + "mlp2_bias": _bf16(p.mlp2_bias),
        })
    save_file(tensors, os.path.join(tmp_path, "model.safetensors"))
    del tensors
    cfg = GPTOssConfig(num_experts=E, hidden_size=H, intermediate_size=inter,
                       num_hidden_layers=layers)
    ck = W.TorchCheckpoint(tmp_path, "cuda")
    assert ck.get_tensor("block.1.mlp.mlp1_weight.blocks").device.type == "cuda"
    blocks = W.load_mlp_blocks(ck, cfg)
    x = O.make_input(80, n, hidden=H)
    for p, blk in zip(params, blocks):
        out = host_bf16(blk(bf16_dev(x).view(1, n, H)).view(n, H))
        m = O.compare_outputs(out, O.block_forward(x, p).out)
        assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m


@pytest.mark.parametrize("n", [16, 520])
def test_checkpoint_scale_bytes_0_and_1(tmp_path, oracle_lib, n):
    """Scale bytes 0 and 1 (weights 2^-128 ... 6 x 2^-126: fp32 subnormals and
    the smallest normals in the reference, model/mlp.py:297-298) on 3% of the
    blocks of a 20B-shape layer: loaded with a warning, and the block output
    stays within the bar through the decode launch (16 tokens) and the
    prefill GEMMs (520 tokens, 65 pairs per expert); the oracle runs on a
    32-token sample there (each token's output depends on that token only)."""
    import weights as W
    from model.config import GPTOssConfig
    E, H = 32, 2880
    p = O.make_params(75, num_experts=E, hidden=H, inter=H)
    rng = np.random.default_rng(76)
    for sc in (p.mlp1_scales, p.mlp2_scales):
        hit = rng.random(sc.shape) < 0.03
        sc[hit] = rng.integers(0, 2, int(hit.sum()))
    pre = "block.0.mlp."
    save_file({
        pre + "norm.scale": _bf16(p.norm_w), pre + "gate.weight": _bf16(p.gate_w),
        pre + "gate.bias": _bf16(p.gate_b),
        pre + "mlp1_weight.blocks": torch.from_numpy(p.mlp1_blocks),
        pre + "mlp1_weight.scales": torch.from_numpy(p.mlp1_scales),
        pre + "mlp1_bias": _bf16(p.mlp1_bias),
        pre + "mlp2_weight.blocks": torch.from_numpy(p.mlp2_blocks),
        pre + "mlp2_weight.scales": torch.from_numpy(p.mlp2_scales),
        pre + "mlp2_bias": _bf16(p.mlp2_bias),
    }, os.path.join(tmp_path, "model.safetensors"))
    cfg = GPTOssConfig(num_experts=E, hidden_size=H, intermediate_size=H, num_hidden_layers=1)
    with pytest.warns(RuntimeWarning, match="outside"):
        (blk,) = W.load_mlp_blocks(W.TorchCheckpoint(tmp_path, "cuda"), cfg)
    assert W.scale_range(blk)[0] == 0
    x = O.make_input(77, n, hidden=H)
    out = host_bf16(blk(bf16_dev(x).view(1, n, H)).view(n, H))
    sel = np.arange(n) if n <= 32 else np.sort(rng.choice(n, 32, replace=False))
    ref, _, _, _ = oracle_lib.block_forward(np.ascontiguousarray(x[sel]), p,
                                            nthreads=max(1, min(16, len(os.sched_getaffinity(0)))))
    m = O.compare_outputs(out[sel], ref)
    assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m


def test_engine_loads_whole_model_checkpoint(tmp_path):
    """Engine(model_path) (engine.py:17-28 -> weights.py:70-122): a whole
    gpt-oss checkpoint with the real tensor names (embedding.weight,
    block.N.attn.{sinks, norm.scale, qkv.*, out.*}, block.N.mlp.*,
    norm.scale, unembedding.weight) and a config.json with gpt-oss's own
    spelling of a field (experts_per_token).  Every parameter holds exactly
    the written tensor; then a prefill and two decode steps, each sub-block
    replayed by the oracle on the GPU's own input (as the decode-loop tests
    do) and each sampled token checked against the oracle sampler."""
    import json

    import weights as W
    from engine import Engine
    from oracle import attn_oracle as AO
    from test_gpu_decode_loop import _Replay, _sample_ok
    mp = AO.make_model_params(950, layers=2, vocab=4096)
    tensors = {"embedding.weight": _bf16(mp.embedding), "norm.scale": _bf16(mp.norm_w),
               "unembedding.weight": _bf16(mp.unembedding)}
    for i, (ap, bp) in enumerate(mp.layers):
        a, m = f"block.{i}.attn.", f"block.{i}.mlp."
        tensors.update({
            a + "sinks": _bf16(ap.sinks), a + "norm.scale": _bf16(ap.norm_w),
            a + "qkv.weight": _bf16(ap.qkv_w), a + "qkv.bias": _bf16(ap.qkv_b),
            a + "out.weight": _bf16(ap.out_w), a + "out.bias": _bf16(ap.out_b),
            m + "norm.scale": _bf16(bp.norm_w), m + "gate.weight": _bf16(bp.gate_w),
            m + "gate.bias": _bf16(bp.gate_b),
            m + "mlp1_weight.blocks": torch.from_numpy(bp.mlp1_blocks),
            m + "mlp1_weight.scales": torch.from_numpy(bp.mlp1_scales),
            m + "mlp1_bias": _bf16(bp.mlp1_bias),
            m + "mlp2_weight.blocks": torch.from_numpy(bp.mlp2_blocks),
            m + "mlp2_weight.scales": torch.from_numpy(bp.mlp2_scales),
            m + "mlp2_bias": _bf16(bp.mlp2_bias),
        })
    save_file(tensors, os.path.join(tmp_path, "model.safetensors"))
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump({"num_hidden_layers": 2, "num_experts": 32, "experts_per_token": 4,
                   "vocab_size": 4096, "hidden_size": 2880, "intermediate_size": 2880,
                   "context_window_size": 1024, "prefill_chunk_size": 512}, f)
    eng = Engine(tmp_path, max_total_seq_len=1024)
    assert eng.config.num_experts_per_tok == 4 and eng.config.num_hidden_layers == 2
    names = [n for n, _ in eng.model.named_parameters()]
    assert sorted(W.convert_key(n) for n in names) == sorted(tensors)
    for name, prm in eng.model.named_parameters():
        src = tensors[W.convert_key(name)]
        assert torch.equal(prm.detach().cpu().view(torch.uint8), src.view(torch.uint8)), name
    rep = _Replay(eng, mp)
    rng = np.random.default_rng(951)
    seq = eng.begin_sequence()
    logits = eng.prefill(rng.integers(0, 4096, 140).astype(np.int32), seq)
    got = logits.view(-1).cpu().numpy()
    rep.check(got, "prefill")
    p = eng.sample_parameters
    for step in range(2):
        tok = eng.sample(logits)
        assert _sample_ok(got, p["temperature"], p["top_p"], p["random_seed"], tok), step
        logits = eng.decode(np.array([tok], dtype=np.int32), seq)
        got = logits.view(-1).cpu().numpy()
        rep.check(got, f"decode step {step}")
