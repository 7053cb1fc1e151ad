"""Write the committed golden fixtures under tests/golden/.

The reference ships no golden vectors (no tests, no fixtures) and cannot be
imported here (tvm / mlc-llm are absent), so these fixtures come from the
pinned CPU oracle (oracle/moe_oracle.py, itself checked in tests/test_oracle.py)
and exist to freeze its outputs: a regression pin for the oracle and a
ready-made expected output for the GPU tests.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import moe_oracle as O  # noqa: E402

# (name, experts, hidden, intermediate, tokens, param seed, input seed, zipf beta)
CASES = [
    ("moe_tiny_e8_h128_i96_n7", 8, 128, 96, 7, 101, 102, 0.0),
    ("moe_small_e32_h256_i128_n64", 32, 256, 128, 64, 201, 202, 0.0),
    ("moe_small_zipf_e16_h192_i64_n96", 16, 192, 64, 96, 301, 302, 0.5),
]


def make(case) -> dict:
    name, E, H, I, n, ps, xs, beta = case
    p = O.make_params(ps, num_experts=E, hidden=H, inter=I, zipf_beta=beta)
    x = O.make_input(xs, n, hidden=H)
    tr = O.block_forward(x, p)
    return {
        "x": x, "norm_w": p.norm_w, "gate_w": p.gate_w, "gate_b": p.gate_b,
        "mlp1_blocks": p.mlp1_blocks, "mlp1_scales": p.mlp1_scales, "mlp1_bias": p.mlp1_bias,
        "mlp2_blocks": p.mlp2_blocks, "mlp2_scales": p.mlp2_scales, "mlp2_bias": p.mlp2_bias,
        "t": tr.t, "idx": tr.idx, "w": tr.w, "act": tr.act, "y": tr.y, "out": tr.out,
    }


def main() -> None:
    manifest = {}
    for case in CASES:
        arrays = make(case)
        path = os.path.join(HERE, case[0] + ".npz")
        np.savez_compressed(path, **arrays)
        with open(path, "rb") as f:
            manifest[case[0]] = hashlib.sha256(f.read()).hexdigest()
        print(f"wrote {path}")
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump({"cases": [list(c) for c in CASES], "sha256": manifest}, f, indent=1)


if __name__ == "__main__":
    main()
