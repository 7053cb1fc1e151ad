"""Benchmark of the MI355X MXFP4 MoE block (the path BASELINE.json names).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode64]

A step is one MLPBlock.forward over one batch of synthetic tokens at the
gpt-oss-20b shape (hidden 2880, 32 experts, top-4, intermediate 2880, MXFP4
weights packed in HBM).  The default workload is BASELINE config 1, decode
batch 64; ``value`` is tokens per second with inputs and weights resident in
HBM.  Three independent weight sets (3 x 424 MB, beyond the 256 MB MALL) are
rotated so that every step streams its experts from HBM.

Besides the JSON contract fields the line carries
  roofline      for the dominant kernel (at decode the one-launch chain
                moe_mx_decode_kernel, else mlp1): algorithmic bytes per launch
                / its average duration, from HIP events recorded on the launch
                stream around that kernel in a second timed pass, vs 8 TB/s;
                traffic from rocprofv3 FETCH_SIZE + WRITE_SIZE when a
                measured summary is committed under profiles/;
  cpu_baseline  the serial C restatement of the reference block (the CPU
                oracle) timed on this host's cores on a bounded sample of the
                same tokens and weights; its outputs double as a parity check.
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

# name -> (experts, tokens, zipf beta, BASELINE config label)
CONFIGS = {
    "decode64": (32, 64, 0.0, "config 1: gpt-oss-20b MoE block, decode batch 64"),
    "decode1": (32, 1, 0.0, "config 0: gpt-oss-20b MoE block, decode 1 token"),
    "prefill4096": (32, 4096, 0.5, "config 2: gpt-oss-20b MoE block, 4096-token prefill, Zipf routing"),
    "decode256_120b": (128, 256, 0.0, "config 3a: gpt-oss-120b MoE block, decode batch 256"),
    "prefill2048_120b": (128, 2048, 0.0, "config 3b: gpt-oss-120b MoE block, 2048-token prefill"),
}
H = I = 2880
K_TOP = 4


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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
            pr = torch.arange(1, E + 1, device=device, dtype=torch.float64) ** -1.1
            b = b + zipf_beta * torch.log(pr / pr.sum()).float()
        blk.gate.bias.copy_(b)
        blk.norm.weight.fill_(1.0)
    return blk


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


def cpu_baseline(blk, x, n_sample: int):
    """Serial C restatement of model/mlp.py on the first n_sample tokens (weight set 0)."""
    import numpy as np
    import torch

    from oracle import moe_oracle as O
    from oracle import moe_ref

    def u16(t):
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    p = O.BlockParams(u16(blk.norm.weight), u16(blk.gate.weight), u16(blk.gate.bias),
                      blk.mlp1_weight_blocks.cpu().numpy(), blk.mlp1_weight_scales.cpu().numpy(),
                      u16(blk.mlp1_bias), blk.mlp2_weight_blocks.cpu().numpy(),
                      blk.mlp2_weight_scales.cpu().numpy(), u16(blk.mlp2_bias))
    xs = u16(x.reshape(-1, H))[:n_sample]
    t0 = time.perf_counter()
    out, _, idx, _ = moe_ref.block_forward(xs, p, k=K_TOP, nthreads=1)
    dt = time.perf_counter() - t0
    gpu_out = u16(blk(x.reshape(1, -1, H)).reshape(-1, H))[:n_sample]
    parity = O.compare_outputs(gpu_out, out)
    gpu_idx = blk.route(x.reshape(-1, H))[1].cpu().numpy()[:n_sample]
    parity["routing_equal"] = bool(np.array_equal(gpu_idx, idx))
    return {
        "value": round(n_sample / dt, 4), "unit": "tok/s", "cores": 1, "kind": "port",
        "sample": (f"first {n_sample} tokens of the workload batch with weight set 0, serial C "
                   f"restatement of model/mlp.py (oracle/moe_ref.c, 1 thread), {dt:.1f} s"),
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
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 device copies of 512 MiB (the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(expert-parallel sharding is a design note, not a measured path)", file=sys.stderr)
        return 2

    import torch

    if args.copy_calibration:
        src = torch.ones(512 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 5 x 512 MiB device copies")
        return 0

    from oracle import moe_oracle as O

    dev = torch.device("cuda:0")
    E, n, beta, label = CONFIGS[args.config]
    log(f"workload {args.config}: E={E} n={n} zipf_beta={beta}")
    blocks = [make_block(E, 1000 + i, beta, dev) for i in range(args.weight_sets)]
    gx = torch.Generator(device=dev)
    gx.manual_seed(7)
    xs = [torch.randn((1, n, H), generator=gx, device=dev).to(torch.bfloat16)
          for _ in range(args.weight_sets)]
    torch.cuda.synchronize()
    log("weights ready")

    # routing statistics (touched experts per weight set) for the algorithmic bytes
    touched = []
    for blk, x in zip(blocks, xs):
        st = blk.forward_staged(x)
        cnt = torch.diff(st["perm"]["indptr"])
        touched.append(int((cnt > 0).sum()))
    max_load = float((cnt.max().float() / cnt.float().mean()).item())

    nw = len(blocks)
    for i in range(args.warmup):
        blocks[i % nw](xs[i % nw])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        blocks[i % nw](xs[i % nw])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = n / (dt / args.steps)
    log(f"timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step, {value:.0f} tok/s")

    # both prefill configs average 48 or more pairs per expert: the tiled GEMM
    mfma_bound = args.config.startswith("prefill")
    # At decode the block runs mlp1, the act encoding and mlp2 as one launch
    # (moe_mlp_decode) where the shape allows it: that launch is the one timed.
    fused = False
    if not mfma_bound and n <= 128:
        try:
            blocks[0].forward_staged(xs[0], fused_decode=True)
            fused = True
        except RuntimeError as e:
            log(f"mlp_decode not used: {e}")
    torch.cuda.synchronize()

    # second pass: per-stage HIP events on the launch stream.  A spin kernel is
    # queued first so the host runs ahead of the GPU and the events time the
    # kernels, not gaps left by Python between launches.
    if fused:
        stages = ("router", "permute", "pieces_t", "mlp_decode", "combine")
    else:
        stages = ("router", "permute", "pieces_t", "mlp1", "pieces_act", "mlp2", "combine")
    recs = []
    torch.cuda._sleep(int(2.4e9 * 0.4e-3 * args.steps))
    for i in range(args.steps):
        ev = {s: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for s in stages}
        blocks[i % nw].forward_staged(xs[i % nw], events=ev, fused_decode=fused)
        recs.append(ev)
    torch.cuda.synchronize()
    stage_us = {s: sum(r[s][0].elapsed_time(r[s][1]) for r in recs) / len(recs) * 1e3
                for s in stages}
    log("stage us: " + ", ".join(f"{s}={v:.1f}" for s, v in stage_us.items()))

    g1, g2 = H // 32, I // 32
    mlp1_weight_bytes = 2 * I * g1 * 17 + 2 * I * 2
    mlp2_weight_bytes = H * g2 * 17 + H * 2
    avg_touched = sum(touched) / len(touched)
    nk = n * K_TOP
    flops_per_step = O.flops(n, K_TOP, E, H, I)
    if fused:
        # weights of the touched experts, t in (two 1-byte pieces per element),
        # act's three pieces written and read back, y out (fp32)
        alg = (avg_touched * (mlp1_weight_bytes + mlp2_weight_bytes) + n * H * 2 +
               2 * nk * I * 3 + nk * H * 4)
        achieved = alg / (stage_us["mlp_decode"] * 1e-6) / 1e9
        roof = {"bound": "hbm",
                "kernel": "moe_mx_decode_kernel (mlp1 + SwiGLU + act pieces + mlp2)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic(args.config, "moe::moe_mx_decode_kernel"),
                "algorithmic_bytes": int(alg), "avg_us": round(stage_us["mlp_decode"], 2)}
    elif not mfma_bound:
        alg = avg_touched * mlp1_weight_bytes + n * H * 2 + nk * I * 4
        achieved = alg / (stage_us["mlp1"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "kernel": "moe_mx_gemv_kernel<2,1,23> (mlp1)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic(args.config, "moe::moe_mx_gemv_kernel<2, 1, 23>"),
                "algorithmic_bytes": int(alg), "avg_us": round(stage_us["mlp1"], 2)}
    else:
        f1 = 2 * nk * 2 * I * H
        achieved = f1 / (stage_us["mlp1"] * 1e-6) / 1e12
        roof = {"bound": "mfma", "kernel": "mlp1", "achieved": round(achieved, 2),
                "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                "traffic": read_traffic(args.config, "moe::moe_mx_gemm_kernel<2, 1>"),
                "algorithmic_flops": int(f1),
                "avg_us": round(stage_us["mlp1"], 2)}

    block_bytes = O.algorithmic_bytes(n, round(avg_touched), E, H, I)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random MXFP4 weights and bf16 N(0,1) tokens, BASELINE distributions)",
        "config": {"workload": label, "tokens": n, "experts": E, "top_k": K_TOP, "hidden": H,
                   "intermediate": I, "weight_sets": nw, "touched_experts": avg_touched,
                   "max_over_mean_load": round(max_load, 2)},
        "block": {"hbm_gbs": round(block_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                  "hbm_frac": round(block_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "tflops": round(flops_per_step / (ms_per_step * 1e-3) / 1e12, 2),
                  "algorithmic_bytes": int(block_bytes)},
        "stages_us": {s: round(v, 2) for s, v in stage_us.items()},
        "roofline": roof,
    }
    if not args.no_cpu:
        ns = min(args.cpu_tokens, n)
        log(f"cpu baseline on {ns} tokens")
        cb, parity = cpu_baseline(blocks[0], xs[0], ns)
        line["cpu_baseline"] = cb
        line["parity_vs_cpu"] = parity
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
