"""The no-allocation entry point (moe_block_forward_noalloc) against the
workspace entry point (moe_block_forward) it varies.

Both run the same kernels, so the outputs must agree bit for bit; they are
also held to the oracle's block bar.  Two calls in a row, the second with
fewer tokens (the static scratch then holds the first call's contents), and
one call past the scratch limit, which must be refused before any launch.
Neither torch's allocator nor the device (its free bytes, which a hipMalloc
inside the library would lower) may see an allocation after the first call.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import moe_oracle as O  # noqa: E402
from gpu_util import bf16_dev, host_bf16, make_block  # noqa: E402

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_entry_point():
    import moe_native as native
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    p = O.make_params(seed=400)
    blk = make_block(p)
    params = blk.packed_params()
    H = 2880
    for i, (n, seed) in enumerate(((200, 401), (64, 402), (5, 403))):
        print(f"noalloc n={n}", flush=True)
        x = O.make_input(seed, n)
        xd = bf16_dev(x)
        ref = blk(xd.view(1, n, H)).view(n, H)
        out = torch.full((n, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        free_before = torch.cuda.mem_get_info()[0]   # the device's free bytes (hipMemGetInfo)
        native.block_forward_noalloc(xd, params, 4, 1e-5, 1.702, 7.0, out)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        if i:   # after the first call (runtime set-up): no device allocation at all
            assert torch.cuda.mem_get_info()[0] == free_before
        got = host_bf16(out)
        assert np.array_equal(got, host_bf16(ref))
        m = O.compare_outputs(got, O.block_forward(x, p).out)
        assert m["max_rel"] <= 1e-2 and m["mae"] <= 1e-3, m
    # beyond the 48 MiB scratch: refused with MOE_ERR_TOO_LARGE, nothing launched
    n = 531
    x = torch.zeros((n, H), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((n, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match=r"\(-8\)"):
        native.block_forward_noalloc(x, params, 4, 1e-5, 1.702, 7.0, out)
    assert int(torch.count_nonzero(out)) == 0
