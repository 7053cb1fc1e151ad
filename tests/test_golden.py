"""The committed fixtures under tests/golden/ still match the oracle bit for bit."""
import json
import os

import numpy as np
import pytest

from oracle import moe_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = json.load(open(os.path.join(GOLDEN, "MANIFEST.json")))["cases"]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_oracle_reproduces_fixture(case):
    name, E, H, I, n, ps, xs, beta = case
    ref = np.load(os.path.join(GOLDEN, name + ".npz"))
    p = O.make_params(ps, num_experts=E, hidden=H, inter=I, zipf_beta=beta)
    x = O.make_input(xs, n, hidden=H)
    assert np.array_equal(ref["x"], x)
    assert np.array_equal(ref["mlp1_blocks"], p.mlp1_blocks)
    tr = O.block_forward(x, p)
    for key in ("t", "idx", "w", "act", "y", "out"):
        assert np.array_equal(ref[key], getattr(tr, key)), key
