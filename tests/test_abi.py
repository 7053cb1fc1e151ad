"""The C-ABI library loads, exports every entry point of include/moe_gfx950.h, and
rejects bad arguments with the documented status codes before touching the GPU.

No kernel is launched here (this suite runs without a GPU): every call below
fails host-side validation.
"""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_gfx950.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"MOE_API\s+[\w\s\*]+?\b(moe_\w+)\s*\(", text)))


def header_codes():
    return {m[0]: int(m[1]) for m in re.findall(r"#define (MOE_\w+) \(?(-?\d+)\)?", open(HEADER).read())}


@pytest.fixture(scope="module")
def native():
    import moe_native
    return moe_native


def test_header_declares_entry_points():
    syms = header_symbols()
    for name in ("moe_block_forward", "moe_router_topk", "moe_permute", "moe_einsum_fused",
                 "moe_mlp1_swiglu", "moe_mlp2", "moe_gemv_gating", "moe_dequant_mxfp4"):
        assert name in syms


def test_library_exports_every_header_symbol(native):
    lib = native.lib()
    for name in header_symbols():
        assert hasattr(lib, name), name
        assert name in native.EXPORTED, f"{name} has no ctypes signature in moe_native"


ATTN_HEADER = os.path.join(REPO, "include", "attn_gfx950.h")


def test_library_exports_every_attention_symbol(native):
    import attn_native
    syms = sorted(set(re.findall(r"MOE_API\s+[\w\s\*]+?\b(attn_\w+)\s*\(",
                                 open(ATTN_HEADER).read())))
    assert {"attn_decode", "attn_prefill", "attn_qkv_rope_append", "attn_rms_norm"} <= set(syms)
    for name in syms:
        assert hasattr(native.lib(), name), name
        assert name in attn_native.EXPORTED, f"{name} has no ctypes signature in attn_native"
    with pytest.raises(AttributeError):
        getattr(native.lib(), "attn_launch_decode")


def test_attention_validation(native):
    """Bad arguments are refused on the host (no launch, no GPU needed)."""
    lib = native.lib()
    import attn_native  # noqa: F401  (registers the signatures)
    p = ctypes.c_void_p(16)
    codes = header_codes()
    assert lib.attn_rms_norm(None, 1, 2880, p, 1e-5, p, None) == codes["MOE_ERR_NULL"]
    assert lib.attn_rms_norm(p, 1, 2881, p, 1e-5, p, None) == codes["MOE_ERR_SHAPE"]
    assert lib.attn_rms_norm(ctypes.c_void_p(18), 1, 2880, p, 1e-5, p, None) == codes["MOE_ERR_ALIGN"]
    assert lib.attn_decode(p, 1, p, 0, p, p, p, 128, 0, 0.125, p, p, p, 1 << 20, None) == \
        codes["MOE_ERR_SHAPE"]                                       # no pages
    # partials of (sequence, query head, split): a batch of 2 takes two
    # 128-key chunks per split, so 300 keys need two splits
    need = lib.attn_decode_workspace_bytes(2, 300)
    assert need >= 2 * 64 * 2 * 66 * 4
    assert lib.attn_decode(p, 2, p, 8, p, p, p, 300, 0, 0.125, p, p, p, need - 1, None) == \
        codes["MOE_ERR_WORKSPACE"]
    assert lib.attn_prefill(p, p, 1, 10, p, 8, p, p, p, 0, 0.125, None, p, None) == \
        codes["MOE_ERR_NULL"]
    assert lib.attn_prefill(p, p, 1, 0, p, 8, p, p, p, 0, 0.125, p, p, None) == codes["MOE_OK"]
    assert lib.attn_embedding(p, 3, p, 0, 2880, p, None) == codes["MOE_ERR_SHAPE"]
    assert lib.attn_bias_residual(p, p, p, 2, 2882, p, None) == codes["MOE_ERR_SHAPE"]


def test_internal_launchers_are_hidden(native):
    with pytest.raises(AttributeError):
        getattr(native.lib(), "moe_launch_mx_gemv")


def test_status_codes_match_header(native):
    codes = header_codes()
    assert codes["MOE_OK"] == 0
    for name in ("MOE_ERR_NULL", "MOE_ERR_SHAPE", "MOE_ERR_ALIGN", "MOE_ERR_UNSUPPORTED",
                 "MOE_ERR_LAUNCH", "MOE_ERR_WORKSPACE", "MOE_ERR_INCOMPLETE"):
        assert codes[name] < 0
        assert native.status_string(codes[name]) not in ("unknown status", "ok")
    assert native.lib().moe_version() >= 100


def test_validation_rejects_bad_arguments(native):
    L = native.lib()
    codes = header_codes()
    P = ctypes.c_void_p
    fake = P(0x1000)        # aligned, never dereferenced: validation fails first
    odd = P(0x1008)
    # unsupported k / E
    assert L.moe_router_topk(fake, fake, fake, fake, 4, 2880, 32, 9, 1e-5, fake, fake, fake, None) \
        == codes["MOE_ERR_UNSUPPORTED"]
    assert L.moe_router_topk(fake, fake, fake, fake, 4, 2880, 300, 4, 1e-5, fake, fake, fake, None) \
        == codes["MOE_ERR_UNSUPPORTED"]
    # H not a multiple of 8
    assert L.moe_router_topk(fake, fake, fake, fake, 4, 2882, 32, 4, 1e-5, fake, fake, fake, None) \
        == codes["MOE_ERR_SHAPE"]
    # null / misaligned pointers
    assert L.moe_router_topk(None, fake, fake, fake, 4, 2880, 32, 4, 1e-5, fake, fake, fake, None) \
        == codes["MOE_ERR_NULL"]
    assert L.moe_router_topk(odd, fake, fake, fake, 4, 2880, 32, 4, 1e-5, fake, fake, fake, None) \
        == codes["MOE_ERR_ALIGN"]
    # block: hidden not a multiple of 64, intermediate not a multiple of 32
    args = [fake] * 9
    assert L.moe_block_forward(fake, 4, 32, 4, 2880 + 32, 2880, *args, 1e-5, 1.702, 7.0, fake,
                               fake, 1 << 30, None) == codes["MOE_ERR_SHAPE"]
    assert L.moe_block_forward(fake, 4, 32, 4, 2880, 2880 + 16, *args, 1e-5, 1.702, 7.0, fake,
                               fake, 1 << 30, None) == codes["MOE_ERR_SHAPE"]
    # workspace too small
    assert L.moe_block_forward(fake, 4, 32, 4, 2880, 2880, *args, 1e-5, 1.702, 7.0, fake, fake,
                               16, None) == codes["MOE_ERR_WORKSPACE"]
    # workspace not 256-byte aligned
    assert L.moe_block_forward(fake, 4, 32, 4, 2880, 2880, *args, 1e-5, 1.702, 7.0, fake,
                               P(0x1010), 1 << 30, None) == codes["MOE_ERR_ALIGN"]
    # einsum: N not a multiple of 64, K beyond the supported maximum
    assert L.moe_einsum_fused(fake, 0, fake, 4, 4, 32, 100, 2880, fake, fake, fake, fake, fake,
                              1 << 20, None) == codes["MOE_ERR_SHAPE"]
    assert L.moe_einsum_fused(fake, 0, fake, 4, 4, 32, 128, 4096, fake, fake, fake, fake, fake,
                              1 << 20, None) == codes["MOE_ERR_SHAPE"]
    assert L.moe_einsum_fused(fake, 0, fake, 4, 4, 32, 128, 2880, fake, fake, fake, fake, fake,
                              8, None) == codes["MOE_ERR_WORKSPACE"]
    # permute: E out of range
    assert L.moe_permute(fake, 4, 4, 0, fake, fake, fake, fake, fake, None) == codes["MOE_ERR_UNSUPPORTED"]
    # gating: N not a multiple of 4
    assert L.moe_gemv_gating(fake, fake, None, 4, 4, 2882, fake, None) == codes["MOE_ERR_SHAPE"]
    # dequant: negative rows, null
    assert L.moe_dequant_mxfp4(fake, fake, fake, -1, None) == codes["MOE_ERR_SHAPE"]
    assert L.moe_dequant_mxfp4(None, fake, fake, 16, None) == codes["MOE_ERR_NULL"]
    # empty inputs are a successful no-op without any launch
    assert L.moe_block_forward(fake, 0, 32, 4, 2880, 2880, *args, 1e-5, 1.702, 7.0, fake, fake, 0,
                               None) == codes["MOE_OK"]
    assert L.moe_dequant_mxfp4(None, None, None, 0, None) == codes["MOE_OK"]


def test_workspace_layout(native):
    E, k, H, I = 32, 4, 2880, 2880
    for n in (64, 16, 8, 1):
        total = native.workspace_bytes(n, E, k, H, I)
        offs = native.workspace_layout(n, E, k, H, I)
        nk = n * k
        assert len(offs) == 15 and all(o % 256 == 0 for o in offs)
        if nk > 2 * E:   # act shares y's bytes (read by the pieces kernel before mlp2)
            assert offs[9] == offs[11]
            rest = offs[:9] + offs[10:]
        else:            # mlp2's GEMV reads act while writing y: a region of its own
            assert offs[9] + nk * I * 4 <= offs[10]
            rest = offs
        assert rest == sorted(rest)
        assert offs[11] + nk * max(H, I) * 4 <= offs[12]     # y before logits
        counts = max((n + 15) // 16 * E, n * (H // 16) if n <= 32 else 0)
        assert offs[13] + counts * 4 <= offs[14]            # counts, then sync
        assert offs[14] + (E + 1) * 4 <= total              # sync last: E counts + status
    assert native.workspace_bytes(64, E, k, H + 1, I) == 0


def test_noalloc_limits_documented(native):
    """The header's token limits of moe_block_forward_noalloc (48 MiB of
    static scratch): 530 tokens at gpt-oss-20b's shape, 528 at 120b's."""
    lim = 48 << 20
    for E, n_max in ((32, 530), (128, 528)):
        assert native.workspace_bytes(n_max, E, 4, 2880, 2880) <= lim
        assert native.workspace_bytes(n_max + 1, E, 4, 2880, 2880) > lim


def test_decode_spin_limit_hook(native):
    """Host-side only: the bound is swapped and restored (negative = default)."""
    prev = native.set_decode_spin_limit(5)
    assert native.set_decode_spin_limit(-1) == 5
    assert native.set_decode_spin_limit(prev) == 1 << 20
    assert native.set_decode_spin_limit(prev) == prev


def test_block_status_validates(native):
    L = native.lib()
    codes = header_codes()
    assert L.moe_block_status(None, 4, 32, 4, 2880, 2880, None) == codes["MOE_ERR_NULL"]
    assert L.moe_block_status(ctypes.c_void_p(0x1000), 4, 32, 4, 2882, 2880, None) \
        == codes["MOE_ERR_SHAPE"]
    assert L.moe_block_status(None, 0, 32, 4, 2880, 2880, None) == codes["MOE_OK"]
