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
