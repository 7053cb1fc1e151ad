"""Benchmark of the MI355X MXFP4 MoE block (the path BASELINE.json names).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode64]

A step is one MLPBlock.forward over one batch of synthetic tokens at the
gpt-oss-20b shape (hidden 2880, 32 experts, top-4, intermediate 2880, MXFP4
weights packed in HBM).  The default workload is BASELINE config 1, decode
batch 64; ``value`` is tokens per second with inputs and weights resident in
HBM.  Three independent weight sets (3 x 424 MB, beyond the 256 MB MALL) are
rotated so that every step streams its experts from HBM.

Besides the JSON contract fields the line carries
  roofline      for the dominant kernel of the workload (at decode the
                one-launch chain moe_mx_decode_kernel; at prefill the mlp1
                GEMM): algorithmic bytes (or flops) per launch / its average
                duration from HIP events recorded on the launch stream around
                that kernel in a second timed pass, against 8 TB/s (or the
                2.5 PFLOP/s dense bf16 peak); traffic from rocprofv3
                FETCH_SIZE + WRITE_SIZE when a measured summary is committed
                under profiles/;
  secondary     the other BASELINE workloads, each timed the same way with
                fewer steps: configs 0 (decode 1), 2 (prefill 4096, Zipf
                routing), 3a/3b (120B decode 256 / prefill 2048) and 4 (24
                chained layers, a mixed decode + prefill step captured in one
                HIP graph and replayed); the attention kernels (decode over
                64 x 4096 cached tokens, prefill of 4096) and the whole
                gpt-oss-20b decode loop (tokens per second);
  cpu_baseline  the serial C restatement of the reference block (the CPU
                oracle) timed on this host's cores on a bounded sample of the
                same tokens and weights, one thread (the reference's llvm
                build is serial) and, under "all_cores", OpenMP over every
                core this process may use; its outputs double as a parity
                check.
Only one GPU is used; --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "gpt-oss-tvm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE-layer tok/s at 20B shape; decode HBM GB/s %peak; prefill MFMA util"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
# Arithmetic of the path: MXFP4 weights (e2m1 + E8M0) times the activations
# as fp8 e4m3 pieces (2 for t, 3 for act) on the block-scaled MFMA, fp32
# accumulation; router dots fp64; bf16 in and out.
DTYPE = "mxfp4 x fp8-pieces MFMA, fp32 accumulate (bf16 in/out)"
PIECES_T, PIECES_ACT = 2, 3

# name -> (experts, tokens, zipf beta, BASELINE config label)
CONFIGS = {
    "decode64": (32, 64, 0.0, "config 1: gpt-oss-20b MoE block, decode batch 64"),
    "decode1": (32, 1, 0.0, "config 0: gpt-oss-20b MoE block, decode 1 token"),
    "prefill4096": (32, 4096, 0.5, "config 2: gpt-oss-20b MoE block, 4096-token prefill, Zipf routing"),
    "decode256_120b": (128, 256, 0.0, "config 3a: gpt-oss-120b MoE block, decode batch 256"),
    "prefill2048_120b": (128, 2048, 0.0, "config 3b: gpt-oss-120b MoE block, 2048-token prefill"),
}
MIXED = ("mixed24", "config 4: 24 chained gpt-oss-20b MoE blocks, one mixed step of 32 decode "
         "tokens (uniform routing) + a 2048-token prefill chunk (Zipf routing), one HIP graph")
H = I = 2880
K_TOP = 4
PER_EXPERT_BYTES = (2 * I * (H // 32) * 17 + 2 * I * 2) + (H * (I // 32) * 17 + H * 2)  # 13,236,480


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def zipf_bias(E: int, beta: float, device):
    import torch
    pr = torch.arange(1, E + 1, device=device, dtype=torch.float64) ** -1.1
    return (beta * torch.log(pr / pr.sum())).float()


def make_block(E: int, seed: int, zipf_beta: float, device):
    """Random-init MLPBlock of the gpt-oss architecture (BASELINE distributions), on the GPU."""
    import torch

    from model.config import GPTOssConfig
    from model.mlp import MLPBlock

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    blk = MLPBlock(GPTOssConfig(num_experts=E, num_experts_per_tok=K_TOP, hidden_size=H,
                                intermediate_size=I), device=device)
    with torch.no_grad():
        for name in ("mlp1_weight_blocks", "mlp2_weight_blocks"):
            p = blk.get_parameter(name)
            p.copy_(torch.randint(0, 256, p.shape, generator=g, device=device, dtype=torch.uint8))
        for name in ("mlp1_weight_scales", "mlp2_weight_scales"):
            p = blk.get_parameter(name)
            p.copy_(torch.randint(118, 123, p.shape, generator=g, device=device, dtype=torch.uint8))
        for name, std in (("mlp1_bias", 0.01), ("mlp2_bias", 0.01), ("gate.weight", 0.02)):
            p = blk.get_parameter(name)
            p.copy_(torch.randn(p.shape, generator=g, device=device) * std)
        b = torch.randn(E, generator=g, device=device) * 0.01
        if zipf_beta:
            b = b + zipf_bias(E, zipf_beta, device)
        blk.gate.bias.copy_(b)
        blk.norm.weight.fill_(1.0)
    return blk


def hbm_ceiling():
    """The achievable HBM read bandwidth measured on these boxes (GB/s), from the
    committed `bench.py --hbm-calibration` summary, or None."""
    path = os.path.join(REPO, "profiles", "hbm_calibration.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("best_gbs")


def with_ceiling(roof: dict) -> dict:
    """Adds the HBM-bound roofline's fraction of the calibrated ceiling."""
    c = hbm_ceiling()
    if c:
        roof["ceiling_gbs"] = c
        roof["frac_of_ceiling"] = round(roof["achieved"] / c, 4)
    return roof


def read_traffic(workload: str, kernel: str):
    """Measured HBM bytes per launch of `kernel` (a name prefix) from a committed
    rocprofv3 PMC summary of this workload, if any."""
    path = os.path.join(REPO, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        kernels = json.load(f).get("kernels", {})
    for name, v in kernels.items():
        if name.startswith(kernel):
            return v.get("traffic_bytes")
    return None


def block_bytes(n: int, touched: float, E: int) -> float:
    """Compulsory HBM bytes of one block call: touched experts' weights,
    router and norm weights, x in and out."""
    return touched * PER_EXPERT_BYTES + E * H * 2 + 2 * E + 2 * H + n * H * 4


def block_flops(n: int, E: int) -> float:
    return n * (2 * K_TOP * (2 * I * H + H * I) + 2 * H * E)


def timed_steps(fn, steps: int, warmup: int) -> float:
    """Seconds per call over `steps` calls after `warmup` (synchronised on both sides)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def marked_pass(blocks, xs, steps: int) -> dict:
    """Per-stage times of the block's own launches (MLPBlock.forward_marked:
    HIP events recorded on the launch stream between them).  A spin kernel is
    queued first so that the host runs ahead of the GPU and the events time
    the kernels, not gaps left by Python between calls."""
    import torch
    recs = []
    nw = len(blocks)
    torch.cuda._sleep(int(2.4e9 * 0.4e-3 * steps))
    for i in range(steps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(8)]
        _, names = blocks[i % nw].forward_marked(xs[i % nw], ev)
        recs.append((ev, names))
    torch.cuda.synchronize()
    out: dict = {}
    for ev, names in recs:
        for j, name in enumerate(names):
            out[name] = out.get(name, 0.0) + ev[j].elapsed_time(ev[j + 1]) * 1e3
    return {k: v / len(recs) for k, v in out.items()}


def run_block_config(name: str, steps: int, warmup: int, weight_sets: int, dev) -> tuple:
    """Time one single-block workload; returns (result dict, blocks, xs)."""
    import torch
    E, n, beta, label = CONFIGS[name]
    log(f"workload {name}: E={E} n={n} zipf_beta={beta}")
    blocks = [make_block(E, 1000 + i, beta, dev) for i in range(weight_sets)]
    gx = torch.Generator(device=dev)
    gx.manual_seed(7)
    xs = [torch.randn((1, n, H), generator=gx, device=dev).to(torch.bfloat16)
          for _ in range(weight_sets)]
    for blk in blocks:
        blk.reserve(n)
    torch.cuda.synchronize()

    touched, loads = [], []
    for blk, x in zip(blocks, xs):
        st = blk.forward_staged(x)
        cnt = torch.diff(st["perm"]["indptr"])
        touched.append(int((cnt > 0).sum()))
        loads.append(float((cnt.max().float() / cnt.float().mean()).item()))
    avg_touched = sum(touched) / len(touched)

    nw = len(blocks)
    sec = timed_steps(lambda i: blocks[i % nw](xs[i % nw]), steps, warmup)
    us = sec * 1e6
    log(f"{name}: {us:.1f} us/block, {n / sec:.0f} tok/s")
    # Decode sizes also from one HIP graph holding one call per weight set:
    # at one token the block's three launches take less GPU time than the
    # host needs to issue them one call at a time, so the eager figure above
    # is partly the host's; the graph replays them back to back.
    graph_us = None
    if n <= 128:
        for blk in blocks:
            blk.reserve(n, for_graph=True)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for j in range(nw):
                blocks[j](xs[j])
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for j in range(nw):
                blocks[j](xs[j])
        reps = max(10, steps // nw)
        graph_us = timed_steps(lambda i: graph.replay(), reps, 3) / nw * 1e6
        del graph
        log(f"{name}: {graph_us:.1f} us/block from one HIP graph")

    nk = n * K_TOP
    gemm = nk >= 48 * E
    stage_us = marked_pass(blocks, xs, min(steps, 100))
    fused = "decode" in stage_us
    log(f"{name} stage us: " + ", ".join(f"{s}={v:.1f}" for s, v in stage_us.items()))

    bb = block_bytes(n, avg_touched, E)
    bf = block_flops(n, E)
    res = {
        "workload": label, "tokens": n, "experts": E, "us_per_block": round(us, 2),
        "graph_us_per_block": round(graph_us, 2) if graph_us is not None else None,
        "tok_s": round(n / sec, 1), "touched_experts": avg_touched,
        "max_over_mean_load": round(sum(loads) / len(loads), 2),
        "block_hbm_frac": round(bb / sec / 1e9 / HBM_PEAK_GBS, 4),
        "block_bf16_mfma_frac": round(bf / sec / 1e12 / BF16_PEAK_TFLOPS, 4),
        "stages_us": {s: round(v, 2) for s, v in stage_us.items()},
    }
    if fused:
        # compulsory bytes: the touched experts' weights plus 4 bytes per
        # token element (the token in and out); the act pieces written and read
        # back inside the launch are intermediates, listed apart and not counted
        alg = avg_touched * PER_EXPERT_BYTES + n * H * 4
        t = stage_us["decode"]
        achieved = alg / (t * 1e-6) / 1e9
        roof = {"bound": "hbm",
                "kernel": "moe_mx_decode_kernel ("
                          + ("routing + " if "router_logits" in stage_us else "")
                          + "mlp1 + SwiGLU + act pieces + mlp2"
                          + (" + gated combine)" if "gating" not in stage_us else ")"),
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic(name, "moe::moe_mx_decode_kernel"),
                "algorithmic_bytes": int(alg),
                "intermediate_bytes": int(2 * nk * I * PIECES_ACT + nk * H * 4),
                "avg_us": round(t, 2)}
        with_ceiling(roof)
    elif not gemm:
        alg = avg_touched * (2 * I * (H // 32) * 17 + 2 * I * 2) + n * H * PIECES_T
        t = stage_us["mlp1"]
        achieved = alg / (t * 1e-6) / 1e9
        # one token runs its own mlp1 launch (each wave on one weight tile,
        # act's pieces written by the epilogue); more tokens the persistent GEMV
        kern, trace_name = (("moe_mx_token1_mlp1_kernel (mlp1 + SwiGLU + act pieces)",
                             "moe::moe_mx_token1_mlp1_kernel") if n == 1 else
                            ("moe_mx_gemv_kernel<2,1,23> (mlp1)",
                             "moe::moe_mx_gemv_kernel<2, 1, 23>"))
        roof = {"bound": "hbm", "kernel": kern,
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic(name, trace_name),
                "algorithmic_bytes": int(alg), "avg_us": round(t, 2)}
        with_ceiling(roof)
    else:
        f1 = 2 * nk * 2 * I * H
        t = stage_us["mlp1"]
        tflops = f1 / (t * 1e-6) / 1e12
        # mlp1's compulsory bytes: the touched experts' mlp1 weights, t's pieces
        # in, act's three pieces out
        b1 = (avg_touched * (2 * I * (H // 32) * 17 + 2 * I * 2) + n * H * PIECES_T
              + nk * I * PIECES_ACT * 33 / 32)
        gbs = b1 / (t * 1e-6) / 1e9
        ridge = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)     # flop per byte
        kern = "moe_mx_gemm_kernel<2,2> (mlp1, act pieces epilogue)"
        common = {"kernel": kern, "traffic": read_traffic(name, "moe::moe_mx_gemm_kernel<2, 2>"),
                  "algorithmic_flops": int(f1), "algorithmic_bytes": int(b1),
                  "intensity_flop_per_byte": round(bf / bb, 1), "avg_us": round(t, 2),
                  # the MFMA executes every fp8 piece: algorithmic x pieces,
                  # at the fp8 (fp8 x fp4) dense rate
                  "fp8_hw_frac": round(tflops * PIECES_T / FP8_PEAK_TFLOPS, 4)}
        if bf / bb < ridge:
            # below the ridge (the 120B prefill of 2048 tokens): HBM-bound
            roof = with_ceiling({"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                                 "bf16_mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                                 **common})
        else:
            roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                    "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), **common}
        t2 = stage_us["mlp2"]
        f2 = 2 * nk * H * I
        b2 = avg_touched * (H * (I // 32) * 17 + H * 2) + nk * I * PIECES_ACT * 33 / 32 + nk * H * 4
        res["mlp2"] = {"avg_us": round(t2, 2),
                       "frac": round(f2 / (t2 * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                       "hbm_frac": round(b2 / (t2 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "fp8_hw_frac": round(f2 * PIECES_ACT / (t2 * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4),
                       "traffic": read_traffic(name, "moe::moe_mx_gemm_kernel<3, 0>")}
    res["roofline"] = roof
    res["algorithmic_bytes"] = int(bb)
    res["algorithmic_flops"] = int(bf)
    return res, blocks, xs


def mixed_stack(dev, layers: int = 24, n_dec: int = 32, n_pre: int = 2048):
    """Config 4's layers: per layer one 20B block with its own seeded weights
    (seed 2000 + layer) for the decode group and a view of it under the Zipf
    router bias (beta 0.5) for the prefill group, chained in a MoEStack
    reserved for n_dec and n_pre tokens (tests/test_gpu_graph.py checks this
    same stack)."""
    from model.stack import MoEStack
    zb = zipf_bias(32, 0.5, dev)
    pairs = []
    for layer in range(layers):
        dec = make_block(32, 2000 + layer, 0.0, dev)
        pre = dec.with_gate_bias(dec.gate.bias.float() + zb)
        pairs.append((dec, pre))
    stack = MoEStack(pairs)
    stack.reserve(n_dec, n_pre)
    return stack


def run_mixed(steps: int, warmup: int, dev, layers: int = 24, n_dec: int = 32,
              n_pre: int = 2048) -> dict:
    """Config 4: `layers` chained 20B blocks (independent seeded weights), one
    mixed step = the decode group (layer's own router bias) and the prefill
    group (that bias + the Zipf profile at beta 0.5) layer by layer, captured
    in one HIP graph (MoEStack: nothing allocated inside) and replayed."""
    import torch

    log(f"workload mixed24: {layers} layers, {n_dec} decode + {n_pre} prefill tokens")
    stack = mixed_stack(dev, layers, n_dec, n_pre)
    gx = torch.Generator(device=dev)
    gx.manual_seed(9)
    xd = torch.randn((1, n_dec, H), generator=gx, device=dev).to(torch.bfloat16)
    xp = torch.randn((1, n_pre, H), generator=gx, device=dev).to(torch.bfloat16)
    eager_s = timed_steps(lambda i: stack(xd, xp), max(3, steps // 2), 1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack(xd, xp)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack(xd, xp)
    sec = timed_steps(lambda i: graph.replay(), steps, warmup)
    n = n_dec + n_pre
    log(f"mixed24: graph {sec * 1e3:.3f} ms/step ({n / sec:.0f} tok/s), eager {eager_s * 1e3:.3f} ms")
    flops = layers * (block_flops(n_dec, 32) + block_flops(n_pre, 32))
    # each group's call streams the layer's weights (all 32 experts touched)
    bytes_ = layers * (block_bytes(n_dec, 32, 32) + block_bytes(n_pre, 32, 32))
    res = {"workload": MIXED[1], "layers": layers, "tokens": n, "ms_per_step": round(sec * 1e3, 4),
           "tok_s": round(n / sec, 1), "eager_ms_per_step": round(eager_s * 1e3, 4),
           "bf16_mfma_frac": round(flops / sec / 1e12 / BF16_PEAK_TFLOPS, 4),
           "hbm_frac": round(bytes_ / sec / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_flops": int(flops)}
    del graph, stack
    return res


def kernel_us(fn, steps: int, warmup: int = 3) -> float:
    """Average microseconds per call from HIP events on the launch stream; a
    spin kernel queued first lets the host run ahead of the GPU."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.4e9 * 30e-6 * steps))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / steps


def run_attention(steps: int, dev) -> dict:
    """The attention kernels at gpt-oss shape (64 query heads, 8 KV heads,
    head_dim 64, pages of 16): decode attention over 64 sequences of 4096
    cached tokens (scattered pages; full layer and 128-token sliding layer),
    HBM-bound on the K/V bytes read; prefill attention of one 4096-token
    sequence, MFMA-bound on its causal (windowed) score and value products."""
    import math

    import torch

    import attn_native as A
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    B, L = 64, 4096
    pages = B * L // 16
    log(f"workload attention: decode {B} x {L} cached tokens, prefill {L}")
    cache = torch.randn((pages, 2, 8, 16, 64), generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(pages, generator=g, device=dev).to(torch.int32)
    indptr = (torch.arange(B + 1, device=dev, dtype=torch.int32) * (L // 16)).contiguous()
    kv_len = torch.full((B,), L, dtype=torch.int32, device=dev)
    q = torch.randn((B, 64, 64), generator=g, device=dev).to(torch.bfloat16)
    sinks = torch.randn(64, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(64)
    res = {}
    for window in (0, 128):
        span = L if window == 0 else window
        ws = A.decode_workspace(B, span, dev)
        us = kernel_us(lambda i: A.decode(q, cache, indptr, perm, kv_len, span, window, scale,
                                          sinks, out, ws), steps)
        kv_bytes = B * span * 8 * 64 * 2 * 2
        gbs = kv_bytes / us / 1e3
        res[f"decode_b{B}_ctx{L}_window{window}"] = {
            "us": round(us, 2), "kv_bytes": kv_bytes, "achieved_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "attn decode_partial + decode_merge (split over 128-key chunks)"}
    del cache, perm
    n = L
    cache = torch.randn((n // 16, 2, 8, 16, 64), generator=g, device=dev).to(torch.bfloat16)
    pages1 = torch.arange(n // 16, dtype=torch.int32, device=dev)
    ind1 = torch.tensor([0, n // 16], dtype=torch.int32, device=dev)
    qi = torch.tensor([0, n], dtype=torch.int32, device=dev)
    kl = torch.tensor([n], dtype=torch.int32, device=dev)
    qp = torch.randn((n, 64, 64), generator=g, device=dev).to(torch.bfloat16)
    op = torch.empty_like(qp)
    for window in (0, 128):
        us = kernel_us(lambda i: A.prefill(qp, qi, n, cache, ind1, pages1, kl, window, scale,
                                           sinks, op), max(5, steps // 10))
        pairs = sum(min(i + 1, window) if window else i + 1 for i in range(n))
        flops = pairs * 64 * 2 * 64 * 2          # q.k and p.v per (query, key, head)
        tf = flops / us / 1e6
        res[f"prefill_{n}_window{window}"] = {
            "us": round(us, 2), "algorithmic_flops": flops, "tflops": round(tf, 2),
            "bf16_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
            "kernel": "attn prefill_kernel (bf16 MFMA 16x16x32, probabilities as two bf16 pieces)"}
    for k, v in res.items():
        log(f"attention {k}: {v['us']} us")
    return res


def _random_model(model, seed: int):
    """Random weights of the reference's distributions into a GPTOssForCausalLM:
    MXFP4 bytes uniform, E8M0 scales in 118..122, biases N(0, 0.01), dense
    weights N(0, 0.02), embedding and sinks N(0, 1), norm weights 1."""
    import torch
    g = torch.Generator(device=next(model.parameters()).device)
    g.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dtype == torch.uint8:
                lo, hi = (118, 123) if name.endswith("scales") else (0, 256)
                p.copy_(torch.randint(lo, hi, p.shape, generator=g, device=p.device,
                                      dtype=torch.int32).to(torch.uint8))
            elif name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                std = (1.0 if ("embedding.weight" in name and "unembedding" not in name)
                       or name.endswith("sinks") else 0.01 if "bias" in name else 0.02)
                p.copy_((torch.randn(p.shape, generator=g, device=p.device) * std).to(p.dtype))


def run_decode_loop(dev, prompt_len: int = 128, steps: int = 32) -> dict:
    """The decode loop of the whole gpt-oss-20b model (24 layers, vocab
    201088, random weights): a prompt prefill, then `steps` decode steps, each
    the next-token forward and the GPU top-p sample, the sampled token fed
    back on the device (eager, one host table update per step), then the same
    step captured in one HIP graph and replayed."""
    import torch

    from engine import Engine
    from model.config import gpt_oss_20b
    cfg = gpt_oss_20b()
    cfg.context_window_size = 4096
    cfg.prefill_chunk_size = 4096
    log(f"workload decode_loop20b: {cfg.num_hidden_layers} layers, prompt {prompt_len}, {steps} steps")
    eng = Engine(config=cfg, max_total_seq_len=prompt_len + steps + 64)
    _random_model(eng.model, 11)
    g = torch.Generator()
    g.manual_seed(12)
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), generator=g, dtype=torch.int32)
    seq = eng.begin_sequence()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = eng.sample_device(eng.prefill(prompt, seq))
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    for _ in range(3):
        tok = eng.sample_device(eng.decode(tok, seq))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = eng.sample_device(eng.decode(tok, seq))
    torch.cuda.synchronize()
    t_dec = (time.perf_counter() - t0) / steps
    # the same steps replayed from one captured HIP graph
    eng.capture_decode(seq)
    for _ in range(3):
        eng.decode_sample(seq)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = eng.decode_sample(seq)
    torch.cuda.synchronize()
    t_graph = (time.perf_counter() - t0) / steps
    weight_bytes = sum(p.numel() * p.element_size() for p in eng.model.parameters())
    res = {"workload": "gpt-oss-20b decode loop (24 layers, vocab 201088, random weights), batch 1",
           "prompt_tokens": prompt_len, "decode_steps": steps,
           "prefill_ms": round(t_pre * 1e3, 2), "prefill_tok_s": round(prompt_len / t_pre, 1),
           "ms_per_token": round(t_dec * 1e3, 3), "decode_tok_s": round(1.0 / t_dec, 1),
           "graph_ms_per_token": round(t_graph * 1e3, 3),
           "graph_decode_tok_s": round(1.0 / t_graph, 1),
           "model_bytes": weight_bytes, "last_token": int(tok.item())}
    log(f"decode_loop20b: prefill {res['prefill_ms']} ms, decode {res['ms_per_token']} ms/token "
        f"eager, {res['graph_ms_per_token']} ms/token from one HIP graph")
    del eng
    return res


def hbm_calibration(dev, reps: int = 10) -> dict:
    """Achievable HBM read bandwidth: the library's streaming-read kernel
    (moe_hbm_read) over 2 and 4 GiB buffers (far beyond the 256 MB MALL),
    swept over grid sizes and loads in flight; HIP events around `reps` reads
    each, the best configuration reported with the whole sweep."""
    import torch

    import moe_native
    sink = torch.zeros(1 << 15, dtype=torch.int32, device=dev)
    sweep = []
    for gib in (2, 4):
        buf = torch.empty(gib << 30, dtype=torch.uint8, device=dev)
        buf.fill_(0x5A)
        for grid in (1024, 2048, 4096, 8192, 16384, 32768):
            for unroll in (4, 8, 16):
                moe_native.hbm_read(buf, grid, unroll, sink)
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for _ in range(reps):
                    moe_native.hbm_read(buf, grid, unroll, sink)
                b.record()
                torch.cuda.synchronize()
                us = a.elapsed_time(b) * 1e3 / reps
                sweep.append({"gib": gib, "grid": grid, "unroll": unroll, "us": round(us, 1),
                              "gbs": round(buf.numel() / (us * 1e-6) / 1e9, 1)})
        del buf
    best = max(sweep, key=lambda r: r["gbs"])
    log(f"hbm calibration: best {best['gbs']} GB/s ({best})")
    return {"metric": "achievable HBM read bandwidth (streaming read, moe_hbm_read)",
            "best_gbs": best["gbs"], "best": best, "peak_gbs": HBM_PEAK_GBS,
            "best_frac_of_peak": round(best["gbs"] / HBM_PEAK_GBS, 4), "sweep": sweep}


def mfma_calibration(dev, size: int = 8192, reps: int = 20) -> dict:
    """The matrix cores' achievable rate as the vendor library reaches it:
    torch's bf16 matmul and fp8 scaled_mm (hipBLASLt) on size^3, timed with
    HIP events over `reps` calls after a warmup.  A reference point for the
    expert GEMMs' MFMA fractions, not a kernel of this build."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    a = torch.randn((size, size), generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn((size, size), generator=g, device=dev).to(torch.bfloat16)
    flops = 2.0 * size ** 3
    res = {"size": size}

    def rate(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return flops / (e0.elapsed_time(e1) * 1e-3 / reps) / 1e12

    tf = rate(lambda: torch.matmul(a, b))
    res["bf16_tflops"] = round(tf, 1)
    res["bf16_frac_of_2500"] = round(tf / BF16_PEAK_TFLOPS, 3)
    for name in ("float8_e4m3fn", "float8_e4m3fnuz"):
        dt = getattr(torch, name, None)
        if dt is None:
            continue
        try:
            a8, b8 = a.to(dt), b.t().contiguous().to(dt).t()
            one = torch.ones((), device=dev, dtype=torch.float32)
            tf8 = rate(lambda: torch._scaled_mm(a8, b8, scale_a=one, scale_b=one,
                                                out_dtype=torch.bfloat16))
            res["fp8_dtype"] = name
            res["fp8_tflops"] = round(tf8, 1)
            res["fp8_frac_of_5000"] = round(tf8 / 5000.0, 3)
            break
        except (RuntimeError, TypeError) as exc:
            res[f"fp8_{name}_error"] = str(exc).splitlines()[0][:120]
    # the attention block's prefill projections at 4096 tokens, as
    # model/attention.py runs them (F.linear: x W^T, bf16, hipBLASLt)
    for name, (m, nn, kk) in (("qkv_4096x5120x2880", (4096, 5120, 2880)),
                               ("out_4096x2880x4096", (4096, 2880, 4096))):
        x = torch.randn((m, kk), generator=g, device=dev).to(torch.bfloat16)
        w = torch.randn((nn, kk), generator=g, device=dev).to(torch.bfloat16)
        f = 2.0 * m * nn * kk
        t = rate(lambda: torch.nn.functional.linear(x, w)) * f / flops   # rate() counts size^3
        us = f / (t * 1e12) * 1e6
        res[name] = {"tflops": round(t, 1), "frac_of_2500": round(t / BF16_PEAK_TFLOPS, 3),
                     "us": round(us, 1)}
    return res


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(blocks, xs, n_sample: int):
    """Serial C restatement of model/mlp.py on the first n_sample tokens (weight
    set 0), then the same restatement with OpenMP over (token, slot) on every
    core this process may use, on all tokens of every weight set."""
    import numpy as np
    import torch

    from oracle import moe_oracle as O
    from oracle import moe_ref

    def u16(t):
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def params(blk):
        return O.BlockParams(u16(blk.norm.weight), u16(blk.gate.weight), u16(blk.gate.bias),
                             blk.mlp1_weight_blocks.cpu().numpy(), blk.mlp1_weight_scales.cpu().numpy(),
                             u16(blk.mlp1_bias), blk.mlp2_weight_blocks.cpu().numpy(),
                             blk.mlp2_weight_scales.cpu().numpy(), u16(blk.mlp2_bias))

    ps = [params(b) for b in blocks]
    xh = [u16(x.reshape(-1, H)) for x in xs]
    t0 = time.perf_counter()
    out, _, idx, _ = moe_ref.block_forward(xh[0][:n_sample], ps[0], k=K_TOP, nthreads=1)
    dt = time.perf_counter() - t0
    gpu_out = u16(blocks[0](xs[0]).reshape(-1, H))[:n_sample]
    parity = O.compare_outputs(gpu_out, out)
    gpu_idx = blocks[0].route(xs[0].reshape(-1, H))[1].cpu().numpy()[:n_sample]
    parity["routing_equal"] = bool(np.array_equal(gpu_idx, idx))
    cores = len(os.sched_getaffinity(0))
    tot = 0
    t0 = time.perf_counter()
    for x, p in zip(xh, ps):
        moe_ref.block_forward(x, p, k=K_TOP, nthreads=cores)
        tot += x.shape[0]
    dt_all = time.perf_counter() - t0
    model = cpu_model()
    return {
        "value": round(n_sample / dt, 4), "unit": "tok/s", "cores": 1, "kind": "port",
        "cpu_model": model,
        "sample": (f"first {n_sample} tokens of the workload batch with weight set 0, serial C "
                   f"restatement of model/mlp.py (oracle/moe_ref.c, 1 thread), {dt:.1f} s"),
        "all_cores": {"value": round(tot / dt_all, 3), "unit": "tok/s", "cores": cores,
                      "kind": "port", "cpu_model": model,
                      "sample": (f"all {tot} tokens of the {len(xs)} weight sets, the same "
                                 f"restatement with OpenMP over (token, slot), {dt_all:.1f} s")},
    }, parity


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode64", choices=sorted(CONFIGS))
    ap.add_argument("--weight-sets", type=int, default=3)
    ap.add_argument("--cpu-tokens", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="time only the primary workload")
    ap.add_argument("--secondary",
                    default="decode1,prefill4096,decode256_120b,prefill2048_120b,mixed24,"
                            "attention,decode_loop20b",
                    help="comma-separated secondary workloads")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 device copies of 512 MiB (the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters), then exit")
    ap.add_argument("--hbm-calibration", action="store_true",
                    help="only sweep the streaming-read kernel over 2 and 4 GiB buffers (the "
                         "achievable HBM read bandwidth), print it and exit")
    ap.add_argument("--mfma-calibration", action="store_true",
                    help="only time library GEMMs of 8192^3 through torch (hipBLASLt: bf16 "
                         "matmul, fp8 scaled_mm) as the matrix cores' achievable rate, then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(expert-parallel sharding is a design note, not a measured path)", file=sys.stderr)
        return 2

    import torch

    if args.hbm_calibration:
        print(json.dumps(hbm_calibration(torch.device("cuda:0"))), flush=True)
        return 0
    if args.copy_calibration:
        src = torch.ones(512 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 5 x 512 MiB device copies")
        return 0

    dev = torch.device("cuda:0")
    if args.mfma_calibration:
        print(json.dumps(mfma_calibration(dev)), flush=True)
        return 0
    prim, blocks, xs = run_block_config(args.config, args.steps, args.warmup, args.weight_sets, dev)
    E, n, _, label = CONFIGS[args.config]
    us = prim["us_per_block"]
    line = {
        "metric": METRIC, "value": prim["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(us * 1e-3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DTYPE,
        "data": "synthetic (seeded random MXFP4 weights and bf16 N(0,1) tokens, BASELINE distributions)",
        "config": {"workload": label, "tokens": n, "experts": E, "top_k": K_TOP, "hidden": H,
                   "intermediate": I, "weight_sets": len(blocks),
                   "touched_experts": prim["touched_experts"],
                   "max_over_mean_load": prim["max_over_mean_load"]},
        "block": {"hbm_gbs": round(prim["block_hbm_frac"] * HBM_PEAK_GBS, 1),
                  "hbm_frac": prim["block_hbm_frac"],
                  "tflops": round(prim["block_bf16_mfma_frac"] * BF16_PEAK_TFLOPS, 2),
                  "algorithmic_bytes": prim["algorithmic_bytes"]},
        "stages_us": prim["stages_us"],
        "roofline": prim["roofline"],
    }
    if not args.no_cpu:
        ns = min(args.cpu_tokens, n)
        log(f"cpu baseline on {ns} tokens (+ all cores)")
        cb, parity = cpu_baseline(blocks, xs, ns)
        line["cpu_baseline"] = cb
        line["parity_vs_cpu"] = parity
    else:
        line["cpu_baseline"] = None
    del blocks, xs
    torch.cuda.empty_cache()
    if not args.no_secondary:
        sec = {}
        for name in [s for s in args.secondary.split(",") if s and s != args.config]:
            if name == MIXED[0]:
                sec[name] = run_mixed(10, 2, dev)
            elif name == "attention":
                sec[name] = run_attention(50, dev)
            elif name == "decode_loop20b":
                sec[name] = run_decode_loop(dev)
            else:
                st = 30 if CONFIGS[name][1] >= 2048 else 100
                res, b, x = run_block_config(name, st, 5, args.weight_sets, dev)
                del b, x
                sec[name] = res
            torch.cuda.empty_cache()
        line["secondary"] = sec
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
