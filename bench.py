"""Benchmark of the MI355X Mega-MoE layer (one GPU).

    python bench.py [--config kimi|qwen|skew|e32|toy] [--steps K] [--warmup W] [--gpus 1]

The default is the headline configuration: the Kimi-scale layer (T=4096,
H=7168, I=2048, E=896, top-16), forward + backward.

A step is one pass of the layer over one batch of synthetic input resident in
HBM: forward (routing -> FC1+gated act -> FC2 -> combine) and, for configs
that train, the five-stage backward. ``value`` is the layer's algorithmic
throughput in TFLOP/s (6RHI forward, +12RHI backward) over the timed steps;
``ms_per_step`` is the layer latency. ``roofline`` reports the dominant
GEMM stage (the longest) against the MFMA bf16 dense peak or, for the
weight-streaming Kimi shape, against HBM bandwidth, from HIP events recorded
on the launch stream inside the timed region, plus the whole step against
its floor. ``cpu_baseline`` times the CPU restatement of the reference's
Torch path (oracle/moe_oracle.py) on a bounded sample of the same
configuration.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
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
    ap.add_argument("--config", default="kimi",
                    help="toy | e32 | qwen | kimi | skew | kimi8k | kimi16k | dsv3 (default: kimi fwd+bwd)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--save-fc1-dtype", default="bf16", choices=("bf16", "fp16", "fp8"),
                    help="saved FC1 format of the training configs (MoEForwardConfig.save_fc1_dtype)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy 5 times (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def stage_work(spec, save_fc1: bool) -> dict:
    """Algorithmic (flops, HBM bytes) of one launch of each GEMM stage.

    Bytes count every operand once: the weight table (2 bytes per element),
    the gathered or expert-major activation rows read, the rows written, and
    the saved FC1 output when the forward keeps it.
    """
    R, H, I, E = spec.routes, spec.hidden, spec.inter, spec.experts
    w1, w2 = 2.0 * E * H * 2 * I, 2.0 * E * H * I
    return {
        "fc1_swiglu": (4.0 * R * H * I, w1 + 2.0 * R * H + 2.0 * R * I + 4.0 * R + (4.0 * R * I if save_fc1 else 0.0)),
        "fc2": (2.0 * R * H * I, w2 + 2.0 * R * I + 2.0 * R * H),
        "fc2_dgrad": (2.0 * R * H * I, w2 + 2.0 * R * H + 2.0 * R * I),
        "fc2_wgrad": (2.0 * R * H * I, w2 + 2.0 * R * H + 2.0 * R * I),
        "fc1_dgrad": (4.0 * R * H * I, w1 + 4.0 * R * I + 2.0 * R * H),
        "fc1_wgrad": (4.0 * R * H * I, w1 + 2.0 * R * H + 4.0 * R * I),
    }


# kernels behind each stage (the stage's HIP-event time also holds the
# tile-list build; the weight gradients gather their rows in place)
STAGE_KERNELS = {
    "fc1_swiglu": "grouped_rows_kernel (gated epilogue)",
    "fc2": "grouped_rows_kernel",
    "fc2_dgrad": "grouped_rows_kernel (gathered dy rows)",
    "fc1_dgrad": "grouped_rows_kernel (K-contiguous gate_up)",
    "fc2_wgrad": "wgrad_persist_kernel (small K) / grouped_wgrad_kernel, wgrad_reg_kernel (deep K)",
    "fc1_wgrad": "wgrad_persist_kernel (small K) / grouped_wgrad_kernel, wgrad_reg_kernel (deep K)",
}

# CPU-baseline sample per config: (tokens, experts). Where the layer's experts
# are spread evenly, the sample is an expert shard with the same rows per
# expert (Kimi: 1/16 of the experts and of the tokens, 73 rows per expert as
# in the full layer); Skew keeps all 32 experts so the Zipf skew is preserved.
CPU_SAMPLE = {"toy": (512, 8), "e32": (1024, 8), "qwen": (1024, 16), "kimi": (256, 56), "skew": (2048, 32),
              "kimi8k": (512, 56), "kimi16k": (1024, 56), "dsv3": (256, 16)}


def cpu_inputs(spec, tokens: int, experts: int, seed: int = 99):
    """Seeded CPU inputs of the sample: same H, I, top-k and routing rule as the
    configuration, over ``experts`` experts and ``tokens`` tokens."""
    import torch

    from mega_moe.bench_configs import CaseSpec, make_routing

    s = CaseSpec(spec.name, tokens, spec.hidden, spec.inter, experts, spec.top_k, spec.routing,
                 spec.backward, spec.dtype, spec.zipf_s)
    gen = torch.Generator().manual_seed(seed)
    sel, rw = make_routing(s, gen)
    H, I = spec.hidden, spec.inter
    dt = torch.float32 if spec.dtype == "fp32" else torch.bfloat16
    x = torch.randn(tokens, H, generator=gen).to(dt)
    dy = torch.randn(tokens, H, generator=gen).to(dt)
    gate_up = torch.empty(experts, H, 2 * I, dtype=dt)
    down = torch.empty(experts, I, H, dtype=dt)
    for e in range(experts):
        gate_up[e] = torch.randn(H, 2 * I, generator=gen) * 0.02
        down[e] = torch.randn(I, H, generator=gen) * 0.02
    return dict(x=x, selected=sel, rw=rw, gate_up=gate_up, down=down.transpose(1, 2), dy=dy)


def _cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def cpu_baseline(spec):
    """Time the CPU restatement of the reference's Torch layer on a sample:
    1 warm-up, then the median of 3 runs (toy: 10), GEMMs in the config's
    dtype (bf16 operands, fp32 accumulation; fp32 for the toy config)."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import moe_oracle as O

    tokens, experts = CPU_SAMPLE[spec.name]
    inp = cpu_inputs(spec, tokens, experts)
    mm = torch.float32 if spec.dtype == "fp32" else torch.bfloat16

    def run():
        t0 = time.perf_counter()
        out, st = O.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], matmul_dtype=mm)
        if spec.backward:
            O.backward(st, inp["dy"])
        return time.perf_counter() - t0

    run()
    t = statistics.median(run() for _ in range(10 if spec.name == "toy" else 3))
    flops_per_route = (6.0 + (12.0 if spec.backward else 0.0)) * spec.hidden * spec.inter
    rate = flops_per_route * tokens * spec.top_k / t
    return {
        "value": rate / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "host_cpus": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "kind": "port",
        "ms_sample": t * 1e3,
        "ms_full_layer_at_this_rate": flops_per_route * spec.routes / rate * 1e3,
        "sample": f"{spec.name} layer {'fwd+bwd' if spec.backward else 'fwd'} on {tokens} tokens x {experts} "
                  f"experts (full: {spec.tokens} x {spec.experts}; same H={spec.hidden}, I={spec.inter}, "
                  f"top-{spec.top_k}, routing rule), oracle per-expert loop with {str(mm).split('.')[-1]} GEMMs, "
                  f"1 warm-up + median of {10 if spec.name == 'toy' else 3}: {t * 1e3:.0f} ms; the full-layer "
                  f"figure scales that rate to the layer's flops, no NPU 256-row M padding",
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
    # dominant GEMM stage (longest HIP-event time) against its roofline:
    # HBM for the weight-streaming Kimi shape, MFMA for the others
    work = stage_work(spec, save_fc1=spec.backward)
    weight_bound = spec.name.startswith("kimi")
    gemm = {}
    for name, (fl, by) in work.items():
        t = stages.get(name)
        if t:
            gemm[name] = {"ms": t, "TFLOP/s": fl / (t * 1e-3) / 1e12, "GB/s": by / (t * 1e-3) / 1e9,
                          "mfma_frac": fl / (t * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                          "hbm_frac": by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS}
    dom = max(gemm, key=lambda n: gemm[n]["ms"])
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{spec.name}.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get(f"{dom}_bytes")
    if weight_bound:
        ach = gemm[dom]["GB/s"]
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach / HBM_PEAK_GBS,
                "traffic": traffic}
    else:
        ach = gemm[dom]["TFLOP/s"]
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": ach / MFMA_BF16_PEAK_TFLOPS, "traffic": traffic}
    roof["stage"] = dom
    roof["kernel"] = STAGE_KERNELS[dom]
    roof["kernel_ms"] = gemm[dom]["ms"]
    roof["algorithmic"] = {"flops": work[dom][0], "bytes": work[dom][1]}
    # whole step against its floor: max(GEMM flops at the MFMA peak, weight
    # bytes at the HBM peak: read once forward; read and written once backward)
    w_bytes = spec.weight_bytes() * (3.0 if spec.backward else 1.0)
    floor_ms = max(flops / (MFMA_BF16_PEAK_TFLOPS * 1e12), w_bytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    roof["step_floor_ms"] = floor_ms
    roof["step_frac"] = floor_ms / ms

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
        print(f"[bench] cpu baseline on {CPU_SAMPLE[spec.name]} (tokens, experts)", file=sys.stderr, flush=True)
        try:
            cpu = cpu_baseline(spec)
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
        "gemm_stages": gemm,
        "bandwidth_kernels": bandwidth,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
