"""Per-stage summary of rocprofv3 runs of ``bench.py`` (kernel time, HBM
traffic, clock), the measurement counterpart of the reference's msprof stage
tables (benchmark/layer/*.py there).

Input: one ``--kernel-trace --stats`` directory of a bench run with K timed
steps, and one ``--pmc`` directory each for FETCH_SIZE, WRITE_SIZE and
GRBM_COUNT of a one-step run of the same configuration, plus the FETCH_SIZE /
WRITE_SIZE directories of ``bench.py --calibrate-copy`` (five 1 GiB device
copies), which give the bytes per counter unit. Kernels are assigned to the
layer's stages from their launch order within each step (a step starts at
the routing kernel); a stage's tile-list build and operand permutes belong
to it.

    python -m mega_moe.runtime.rocprof_summary --trace DIR --fetch DIR --write DIR \
        --clock DIR --cal-fetch DIR --cal-write DIR --bench JSON --md OUT.md --json OUT.json
    python -m mega_moe.runtime.rocprof_summary --mfma DIR --bench JSON --title TITLE
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics

GEMM_ORDER = ("fc1_swiglu", "fc2", "fc2_dgrad", "fc1_dgrad")
WGRAD_ORDER = ("fc2_wgrad", "fc1_wgrad")
STAGE_ORDER = ("route", "fc1_swiglu", "fc2", "combine", "fc2_dgrad", "swiglu_bwd", "act_recompute", "fc2_wgrad",
               "fc1_dgrad", "combine_bwd", "fc1_wgrad")


def short_name(name: str) -> str:
    n = name.replace("(anonymous namespace)::", "")
    return n.split("(")[0]


def _rows(directory: str, pattern: str):
    files = sorted(glob.glob(os.path.join(directory, "**", pattern), recursive=True))
    if not files:
        raise FileNotFoundError(f"no {pattern} under {directory}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def dispatches(directory: str, counter: str | None = None):
    """[(dispatch id, kernel name, start ns, end ns, counter value)] in launch order."""
    if counter is None:
        rows = _rows(directory, "*kernel_trace.csv")
        out = [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]), 0.0)
               for r in rows]
    else:
        acc = {}
        for r in _rows(directory, "*counter_collection.csv"):
            if r["Counter_Name"] != counter:
                continue
            key = int(r["Dispatch_Id"])
            d = acc.setdefault(key, [r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]), 0.0])
            d[3] += float(r["Counter_Value"])
        out = [(k, v[0], v[1], v[2], v[3]) for k, v in acc.items()]
    return sorted(out)


def split_steps(disp):
    """Group the layer's own kernels into steps; each step starts at the
    routing count kernel. Kernels before the first step (input generation)
    are dropped."""
    steps, cur = [], None
    for d in disp:
        n = short_name(d[1])
        if "route_count_kernel" in n:
            cur = []
            steps.append(cur)
        if cur is not None and _is_layer_kernel(n):
            cur.append(d)
    return steps


def _is_layer_kernel(n: str) -> bool:
    return any(s in n for s in ("route_", "build_tiles", "grouped_rows", "combine_items", "gather_route_grad",
                                "swiglu_bwd", "gated_act", "permute_kernel", "wgrad"))


def assign_stages(step):
    """{stage: [dispatch, ...]} for one step, from the launch order."""
    out = {}
    gemm_i = wgrad_i = 0
    combines = 0
    pending = []  # permutes waiting for their weight gradient
    cur_gemm = None
    for d in step:
        n = short_name(d[1])
        if n.startswith("route_"):
            out.setdefault("route", []).append(d)
        elif "build_tiles" in n:
            cur_gemm = GEMM_ORDER[gemm_i]
            gemm_i += 1
            out.setdefault(cur_gemm, []).append(d)
        elif "grouped_rows" in n:
            out.setdefault(cur_gemm, []).append(d)
        elif "combine_items" in n:
            out.setdefault("combine" if combines == 0 else "combine_bwd", []).append(d)
            combines += 1
        elif "gather_route_grad" in n:
            out.setdefault("combine_bwd", []).append(d)
        elif "swiglu_bwd" in n:
            out.setdefault("swiglu_bwd", []).append(d)
        elif "gated_act" in n:
            out.setdefault("act_recompute", []).append(d)
        elif "permute_kernel" in n:
            pending.append(d)
        elif "wgrad" in n:
            st = WGRAD_ORDER[wgrad_i]
            wgrad_i += 1
            out.setdefault(st, []).extend(pending + [d])
            pending = []
    return out


def calibration(directory: str, counter: str) -> float:
    """Bytes per counter unit from the 1 GiB copies of bench.py --calibrate-copy."""
    vals = [d[4] for d in dispatches(directory, counter) if "copyBuffer" in d[1] or "copy" in short_name(d[1])]
    vals = [v for v in vals if v > 0]
    if not vals:
        raise ValueError(f"no copy dispatch in {directory}")
    return float(1 << 30) / statistics.median(vals)


def per_stage(disp_steps, steps: int, value):
    """{stage: mean over the last `steps` steps of sum(value(dispatch))}."""
    use = disp_steps[-steps:]
    acc = {}
    for st in use:
        for stage, ds in assign_stages(st).items():
            acc.setdefault(stage, []).append(sum(value(d) for d in ds))
    return {k: sum(v) / len(v) for k, v in acc.items()}


GEMM_LABELS = {"fc1_swiglu": "FC1 (gate/up + act)", "fc2": "FC2 (down)", "fc2_dgrad": "dAct = dY W2",
               "fc2_wgrad": "dW2", "fc1_dgrad": "dX = dFC1 W1", "fc1_wgrad": "dW1"}
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "GRBM_GUI_ACTIVE")


def mfma_table(pmc_dir: str, bench: dict, title: str) -> str:
    """MFMA utilisation of each GEMM stage's main kernel from one PMC pass of
    SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_BF16 and GRBM_GUI_ACTIVE
    (last step of the run): counted TFLOP = MOPS x 512, clock = GUI_ACTIVE /
    8 XCDs / duration, MFMA busy = BUSY / (GUI_ACTIVE / 8 x 1024 SIMDs),
    TFLOP/s = algorithmic flops (the bench line's) / duration."""
    rows = _rows(pmc_dir, "*counter_collection.csv")
    acc = {}
    for r in rows:
        d = acc.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"], "dur": int(r["End_Timestamp"]) -
                                                    int(r["Start_Timestamp"]), "start": int(r["Start_Timestamp"])})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    disp = sorted((k, v["name"], v["start"], v["start"] + v["dur"], v) for k, v in acc.items())
    step = split_steps(disp)[-1]
    out = [f"## {title}", "",
           "| stage | kernel | us | algorithmic TFLOP | counted TFLOP | clock GHz | MFMA busy | TFLOP/s | "
           "% of 2.5 PF | % of peak at clock |", "|---|---|---|---|---|---|---|---|---|---|"]
    tot_fl = tot_us = 0.0
    for stage, ds in assign_stages(step).items():
        if stage not in GEMM_LABELS:
            continue
        main_k = [d for d in ds if "grouped_rows" in d[1] or "wgrad" in d[1]]
        if not main_k:
            continue
        d = main_k[-1]
        c = d[4]
        us = c["dur"] / 1e3
        g = bench["gemm_stages"][stage]
        fl = g["TFLOP/s"] * 1e12 * g["ms"] * 1e-3
        counted = c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512
        gui = c.get("GRBM_GUI_ACTIVE", 0.0)
        clock = gui / 8 / c["dur"]
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (gui / 8 * 1024) if gui else 0.0
        tf = fl / (us * 1e-6) / 1e12
        tot_fl += fl
        tot_us += us
        out.append(f"| {GEMM_LABELS[stage]} | `{short_name(d[1])}` | {us:.0f} | {fl / 1e12:.3f} | "
                   f"{counted / 1e12:.3f} | {clock:.2f} | {busy * 100:.1f}% | {tf:.0f} | {tf / 2500 * 100:.1f}% | "
                   f"{tf / (2500 * clock / 2.4) * 100:.1f}% |")
    if tot_us:
        tf = tot_fl / (tot_us * 1e-6) / 1e12
        out += ["", f"All GEMMs of the step: {tot_fl / 1e12:.2f} TFLOP in {tot_us / 1e3:.2f} ms = {tf:.0f} TFLOP/s "
                f"({tf / 2500 * 100:.1f}% of 2.5 PF)."]
    return "\n".join(out) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    for k in ("trace", "fetch", "write", "clock", "cal_fetch", "cal_write", "bench", "md", "json"):
        ap.add_argument("--" + k.replace("_", "-"), required=k not in ("md", "json", "clock"))
    ap.add_argument("--title", default="")
    ap.add_argument("--mfma", help="PMC directory of the three MFMA counters: print the MFMA table instead")
    ap.add_argument("--commands", default="", help="text block of the commands that made the inputs")
    if argv is None:
        import sys
        argv = sys.argv[1:]
    if "--mfma" in argv:  # only --mfma, --bench and --title are needed
        mp = argparse.ArgumentParser()
        for k in ("mfma", "bench", "title"):
            mp.add_argument("--" + k, required=k != "title", default="")
        m, _ = mp.parse_known_args(argv)
        print(mfma_table(m.mfma, json.load(open(m.bench)), m.title))
        return
    a = ap.parse_args(argv)

    bench = json.load(open(a.bench))
    steps = int(bench["steps"])
    trace_steps = split_steps(dispatches(a.trace))
    kernel_ms = per_stage(trace_steps, steps, lambda d: (d[3] - d[2]) * 1e-6)
    # per kernel name within each stage: mean ms per step over the timed steps
    names = {}
    for st in trace_steps[-steps:]:
        for stage, ds in assign_stages(st).items():
            per = names.setdefault(stage, {})
            for d in ds:
                per[short_name(d[1])] = per.get(short_name(d[1]), 0.0) + (d[3] - d[2]) * 1e-6 / steps
    fs, ws = calibration(a.cal_fetch, "FETCH_SIZE"), calibration(a.cal_write, "WRITE_SIZE")
    read_b = per_stage(split_steps(dispatches(a.fetch, "FETCH_SIZE")), 1, lambda d: d[4] * fs)
    write_b = per_stage(split_steps(dispatches(a.write, "WRITE_SIZE")), 1, lambda d: d[4] * ws)
    clock = {}
    if a.clock:
        csteps = split_steps(dispatches(a.clock, "GRBM_COUNT"))
        for stage, ds in assign_stages(csteps[-1]).items():
            long_ds = [d for d in ds if d[3] - d[2] >= 100_000]
            if long_ds:
                clock[stage] = sum(d[4] / 8 / (d[3] - d[2]) for d in long_ds) / len(long_ds)  # GHz

    alg_bytes, alg_flops = {}, {}
    for stage, g in bench.get("gemm_stages", {}).items():
        alg_bytes[stage] = g["GB/s"] * 1e9 * g["ms"] * 1e-3
        alg_flops[stage] = g["TFLOP/s"] * 1e12 * g["ms"] * 1e-3
    for stage, g in bench.get("bandwidth_kernels", {}).items():
        if "GB/s" in g:
            alg_bytes[stage] = g["GB/s"] * 1e9 * g["ms"] * 1e-3

    rows, js = [], {"source": a.md or "", "bench_ms_per_step": bench["ms_per_step"], "fetch_scale": fs,
                    "write_scale": ws}
    stages = [s for s in STAGE_ORDER if s in kernel_ms]
    for s in stages:
        km = kernel_ms[s]
        bm = bench["stages_ms"].get(s)
        rb, wb = read_b.get(s), write_b.get(s)
        ab = alg_bytes.get(s)
        fl = alg_flops.get(s)
        js[f"{s}_kernel_ms"] = km
        if rb is not None and wb is not None:
            js[f"{s}_bytes"] = rb + wb
            js[f"{s}_read_bytes"] = rb
            js[f"{s}_write_bytes"] = wb

        def f(v, fmt):
            return "-" if v is None else format(v, fmt)
        rows.append("| {} | {} | {} | {} | {} | {} | {} | {} | {} | {} | {} |".format(
            s, ", ".join(f"`{n}` {v:.3f}" for n, v in names.get(s, {}).items()), f(km, ".3f"), f(bm, ".3f"),
            f(None if rb is None else rb / 1e9, ".3f"), f(None if wb is None else wb / 1e9, ".3f"),
            f(None if ab is None else ab / 1e9, ".3f"),
            f(None if (ab is None or rb is None) else (rb + wb) / ab, ".2f"),
            f(None if ab is None else ab / (km * 1e-3) / 1e12, ".2f"),
            f(None if fl is None else fl / (km * 1e-3) / 1e12, ".0f"), f(clock.get(s), ".2f")))
    total = sum(kernel_ms[s] for s in stages)
    md = [f"# {a.title}", "", "Commands (the bench's own step counts; one PMC counter per run):", ""]
    md += ["    " + line for line in a.commands.strip().splitlines()] + [""]
    md += [f"Stages are assigned from the launch order of each step (a stage's tile-list build and operand "
           f"permutes belong to it). Kernel time = average over the {steps} timed steps of the trace. FETCH_SIZE "
           f"and WRITE_SIZE are scaled by a 1 GiB device copy measured the same way ({fs / 1024:.3f} KiB per "
           f"FETCH_SIZE unit, {ws / 1024:.3f} KiB per WRITE_SIZE unit); the clock is GRBM_COUNT / (8 XCDs x duration), averaged "
           f"over the stage's launches of 100 us or more.", "",
           f"Bench line of the traced run: {bench['ms_per_step']:.3f} ms per step; roofline stage "
           f"`{bench['roofline'].get('stage')}` {bench['roofline']['kernel_ms']:.3f} ms (HIP events).", "",
           "| stage | kernels (ms per step each) | kernel ms | bench stage ms | HBM read GB | HBM write GB | algorithmic GB | "
           "counter / algorithmic | algorithmic TB/s | TFLOP/s | clock GHz |",
           "|---|---|---|---|---|---|---|---|---|---|---|"] + rows + ["",
           f"Sum of stage kernel times: {total:.3f} ms per step."]
    stats = glob.glob(os.path.join(a.trace, "**", "*kernel_stats.csv"), recursive=True)
    if stats:
        # rocprofv3's own --stats summary of the same run (all launches of the
        # run, warm-up and input generation included), the layer's kernels only
        md += ["", "rocprofv3 `--stats` (kernel_stats.csv) of the traced run, the layer's kernels:", "",
               "| kernel | calls | average us | total ms | % of GPU time |", "|---|---|---|---|---|"]
        with open(stats[0], newline="") as f:
            for r in csv.DictReader(f):
                n = short_name(r["Name"])
                if _is_layer_kernel(n):
                    md.append(f"| `{n}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                              f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.2f} |")
    side = [s for s in stages if bench["stages_ms"].get(s) is None and s != "route"]
    if side:
        md += ["", "Stages without a bench stage time ({}) ran on the backward's second stream beside the "
               "next stage; their kernels overlap it, so the sum above exceeds the step time.".format(
                   ", ".join(f"`{s}`" for s in side))]
    md += [""]
    text = "\n".join(md)
    if a.md:
        open(a.md, "w").write(text)
    else:
        print(text)
    if a.json:
        json.dump(js, open(a.json, "w"), indent=1)


if __name__ == "__main__":
    main()
