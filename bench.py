"""Benchmark of the MI355X Mega-MoE layer (one GPU).

    python bench.py [--config e32|qwen|kimi|skew|toy] [--steps K] [--warmup W] [--gpus 1]

A step is one pass of the layer over one batch of synthetic input resident in
HBM: forward (routing -> FC1+gated act -> FC2 -> combine) and, for configs
that train, the five-stage backward. ``value`` is the layer's algorithmic
throughput in TFLOP/s (6RHI forward, +12RHI backward) over the timed steps;
``ms_per_step`` is the layer latency. ``roofline`` reports the dominant
kernel (FC1 grouped GEMM + fused activation) against the MFMA bf16 dense
peak or, for the weight-streaming Kimi shape, against HBM bandwidth, from
HIP events recorded on the launch stream inside the timed region.
``cpu_baseline`` times the CPU restatement of the reference's Torch path
(oracle/moe_oracle.py) on a bounded token sample of the same configuration.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mega-moe-td_amd"))

MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="e32")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--save-fc1-dtype", default="bf16", choices=("bf16", "fp16", "fp8"),
                    help="saved FC1 format of the training configs (MoEForwardConfig.save_fc1_dtype)")
    ap.add_argument("--cpu-tokens", type=int, default=0, help="token sample for the CPU baseline (0 = auto)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy 5 times (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def fc1_algorithmic(spec, save_fc1: bool):
    """(flops, bytes) of one FC1+activation launch."""
    R, H, I, E = spec.routes, spec.hidden, spec.inter, spec.experts
    flops = 4.0 * R * H * I
    byts = 2.0 * E * H * 2 * I + 2.0 * R * H + 2.0 * R * I + 4.0 * R + (4.0 * R * I if save_fc1 else 0.0)
    return flops, byts


def cpu_inputs(spec, tokens: int, seed: int = 99):
    """CPU inputs for a token sample: the sample's routing over all E experts,
    with weights materialised only for the experts the sample touches
    (renumbered densely), so the per-token CPU work equals the full layer's."""
    import torch

    from mega_moe.bench_configs import CaseSpec, make_routing

    s = CaseSpec(spec.name, tokens, spec.hidden, spec.inter, spec.experts, spec.top_k, spec.routing,
                 spec.backward, spec.dtype, spec.zipf_s)
    gen = torch.Generator().manual_seed(seed)
    sel, rw = make_routing(s, gen)
    used = torch.unique(sel)
    remap = torch.full((spec.experts,), -1, dtype=torch.int32)
    remap[used.long()] = torch.arange(used.numel(), dtype=torch.int32)
    sel = remap[sel.long()]
    U, H, I = used.numel(), spec.hidden, spec.inter
    bf = torch.bfloat16
    x = torch.randn(tokens, H, generator=gen).to(bf)
    dy = torch.randn(tokens, H, generator=gen).to(bf)
    gate_up = (torch.randn(U, H, 2 * I, generator=gen) * 0.02).to(bf)
    down = (torch.randn(U, I, H, generator=gen) * 0.02).to(bf).transpose(1, 2)
    return dict(x=x, selected=sel, rw=rw, gate_up=gate_up, down=down, dy=dy), U


def cpu_baseline(spec, tokens: int):
    """Time the CPU restatement of the reference's Torch layer on a token sample."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import moe_oracle as O

    threads = torch.get_num_threads()
    inp, used = cpu_inputs(spec, tokens)
    times = []
    for _ in range(2):
        t0 = time.perf_counter()
        out, st = O.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"])
        if spec.backward:
            O.backward(st, inp["dy"])
        times.append(time.perf_counter() - t0)
    t = min(times)
    flops = (6.0 + (12.0 if spec.backward else 0.0)) * tokens * spec.top_k * spec.hidden * spec.inter
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{spec.name} layer {'fwd+bwd' if spec.backward else 'fwd'} on {tokens} of {spec.tokens} tokens "
                  f"({used} experts touched, full H={spec.hidden}/I={spec.inter}), per-expert fp32 matmul loop "
                  f"with bf16 rounding, best of 2: {t * 1e3:.0f} ms",
    }


def main():
    args = parse()
    if args.calibrate_copy:
        import torch

        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 1 << 30, "launches": 5}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus > 1 is not supported "
                                   "(expert parallelism across GPUs is out of scope)"}))
        sys.exit(2)
    import torch

    import mega_moe
    from mega_moe.bench_configs import CASES, make_inputs
    from mega_moe.runtime.timing import StageTimer

    spec = CASES[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"[bench] config={spec.name} T={spec.tokens} H={spec.hidden} I={spec.inter} E={spec.experts} "
          f"k={spec.top_k} backward={spec.backward}", file=sys.stderr, flush=True)
    inp = make_inputs(spec, device=dev, seed=1234)
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=spec.tokens, hidden_size=spec.hidden,
                                  top_k=spec.top_k, num_experts=spec.experts,
                                  config=mega_moe.MoEForwardConfig(save_fc1_dtype=args.save_fc1_dtype))

    def step():
        if spec.backward:
            out, saved = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"],
                                    return_saved=True)
            mega_moe.moe_backward_triton(saved, inp["dy"])
        else:
            op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer = StageTimer()
    op.stage_timer = timer
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    op.stage_timer = None
    ms = ev0.elapsed_time(ev1) / args.steps
    stages = timer.summary()

    flops = spec.fwd_flops() + (spec.bwd_flops() if spec.backward else 0.0)
    value = flops / (ms * 1e-3) / 1e12
    f1_flops, f1_bytes = fc1_algorithmic(spec, save_fc1=spec.backward)
    f1_ms = stages.get("fc1_swiglu", float("nan"))
    weight_bound = spec.name == "kimi"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{spec.name}.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("fc1_swiglu_bytes")
    if weight_bound:
        ach = f1_bytes / (f1_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach / HBM_PEAK_GBS,
                "traffic": traffic}
    else:
        ach = f1_flops / (f1_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": ach / MFMA_BF16_PEAK_TFLOPS, "traffic": traffic}
    roof["kernel"] = "fc1_swiglu (grouped_rows_kernel gated) + tile-list build"
    roof["kernel_ms"] = f1_ms

    # HBM-bound row kernels against the 8 TB/s peak (algorithmic bytes / stage time)
    R, T, H, I = spec.routes, spec.tokens, spec.hidden, spec.inter
    bw_bytes = {"combine": 2.0 * R * H + 2.0 * T * H + 4.0 * R}
    if spec.backward:
        bw_bytes["combine_bwd"] = 2.0 * R * H + 2.0 * T * H + 4.0 * R + 2.0 * R + 4.0 * R
        bw_bytes["swiglu_bwd"] = 10.0 * R * I + 6.0 * R
    bandwidth = {}
    for name, nbytes in bw_bytes.items():
        t = stages.get(name)
        if t:
            gbs = nbytes / (t * 1e-3) / 1e9
            bandwidth[name] = {"GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "ms": t}
    bandwidth["route"] = {"ms": stages.get("route"), "note": "latency-bound (<= 2 MB of tables)"}

    cpu = None
    if not args.no_cpu_baseline:
        toks = args.cpu_tokens or {"toy": 512, "e32": 4096, "qwen": 2048, "kimi": 2, "skew": 512}[spec.name]
        print(f"[bench] cpu baseline on {toks} tokens", file=sys.stderr, flush=True)
        try:
            cpu = cpu_baseline(spec, toks)
        except Exception as exc:  # reported, never fatal for the GPU measurement
            cpu = {"value": None, "unit": "TFLOP/s", "cores": None, "kind": "port", "sample": f"failed: {exc}"}

    line = {
        "metric": "MoE layer fwd/bwd ms + grouped-GEMM TFLOP/s (% MFMA peak), 1x MI355X",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "wall_s": wall,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, config routing)",
        "config": {"workload": f"{spec.name}: T={spec.tokens} H={spec.hidden} I={spec.inter} E={spec.experts} "
                               f"top-{spec.top_k} {'fwd+bwd' if spec.backward else 'fwd'}"
                               + (f" save_fc1={args.save_fc1_dtype}" if spec.backward and args.save_fc1_dtype != "bf16"
                                  else ""),
                   "global_batch": spec.tokens, "parallelism": "single GPU, all experts resident"},
        "stages_ms": stages,
        "roofline": roof,
        "bandwidth_kernels": bandwidth,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
