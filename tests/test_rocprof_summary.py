"""CPU test of the rocprofv3 summary tool: stage assignment from launch
order, averaging over the timed steps, counter calibration and the overlap
note, on synthetic CSV files in rocprofv3's column layout."""

import csv
import json
import os

from mega_moe.runtime import rocprof_summary as R

STEP = [  # one fwd+bwd step, launch order, (kernel name, duration ns)
    ("route_count_kernel(int)", 10_000), ("route_scan_kernel(int)", 5_000), ("route_scatter_kernel(int)", 8_000),
    ("build_tiles_kernel(int)", 4_000), ("void grouped_rows_kernel<256, 256, 64, 2, 1, 1, 256, 0, true>(x)", 500_000),
    ("build_tiles_kernel(int)", 4_000), ("void grouped_rows_kernel<256, 256, 64, 2, 1, 0, 512, 0, false>(x)", 300_000),
    ("void combine_items_kernel<2, 8>(x)", 50_000),
    ("build_tiles_kernel(int)", 4_000), ("void grouped_rows_kernel<256, 256, 64, 2, 0, 0, 256, 0, true>(x)", 240_000),
    ("void swiglu_bwd_kernel<0, 0>(x)", 80_000),
    ("permute_kernel(x)", 20_000), ("void wgrad_persist_kernel<3>(x)", 280_000),
    ("build_tiles_kernel(int)", 4_000), ("void grouped_rows_kernel<256, 256, 64, 2, 0, 0, 256, 0, true>(x)", 480_000),
    ("void combine_items_kernel<2, 8>(x)", 55_000),
    ("permute_kernel(x)", 21_000), ("void wgrad_persist_kernel<3>(x)", 560_000),
]


def _write_trace(d, steps):
    os.makedirs(d)
    t, rows, did = 1_000, [], 1
    rows.append(dict(Dispatch_Id=did, Kernel_Name="void at::native::fill(x)", Start_Timestamp=t,
                     End_Timestamp=t + 100))
    t += 1_000
    for s in range(steps):
        for name, dur in STEP:
            did += 1
            rows.append(dict(Dispatch_Id=did, Kernel_Name=name, Start_Timestamp=t, End_Timestamp=t + dur * (1 + s)))
            t += dur * (1 + s) + 500
    with open(os.path.join(d, "s_kernel_trace.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def _write_pmc(d, counter, per_kernel, copies=None):
    os.makedirs(d)
    rows, did, t = [], 0, 1_000
    names = [(n, dur) for n, dur in STEP] * 2 if copies is None else [("__amd_rocclr_copyBuffer", 1000)] * copies
    for name, dur in names:
        did += 1
        rows.append(dict(Dispatch_Id=did, Kernel_Name=name, Counter_Name=counter,
                         Counter_Value=per_kernel(name), Start_Timestamp=t, End_Timestamp=t + dur))
        t += dur + 100
    with open(os.path.join(d, "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_stage_assignment_and_averages(tmp_path):
    steps = 3
    _write_trace(str(tmp_path / "t"), 2 + steps)  # 2 warm-up + 3 timed steps
    _write_pmc(str(tmp_path / "f"), "FETCH_SIZE", lambda n: 1000.0 if "wgrad" in n else 10.0)
    _write_pmc(str(tmp_path / "w"), "WRITE_SIZE", lambda n: 2000.0 if "wgrad" in n else 0.0)
    _write_pmc(str(tmp_path / "c"), "GRBM_COUNT", lambda n: 8 * 2.0 * dict(STEP)[n])  # 2 GHz
    _write_pmc(str(tmp_path / "cf"), "FETCH_SIZE", lambda n: 524288.0, copies=5)  # 2 KiB per unit
    _write_pmc(str(tmp_path / "cw"), "WRITE_SIZE", lambda n: 1048576.0, copies=5)  # 1 KiB per unit
    bench = {"steps": steps, "ms_per_step": 2.7, "roofline": {"stage": "fc1_wgrad", "kernel_ms": 1.7},
             "stages_ms": {"route": 0.05, "fc1_swiglu": 1.5, "fc2": 0.9, "combine": 0.15, "fc2_dgrad": 0.73, "swiglu_bwd": 0.08,
                           "fc2_wgrad": 0.9, "fc1_dgrad": 1.45, "combine_bwd": 0.17, "fc1_wgrad": 1.75},
             "gemm_stages": {"fc1_wgrad": {"ms": 1.75, "TFLOP/s": 100.0, "GB/s": 1000.0}},
             "bandwidth_kernels": {}}
    json.dump(bench, open(tmp_path / "b.json", "w"))
    md, js = str(tmp_path / "o.md"), str(tmp_path / "o.json")
    R.main(["--trace", str(tmp_path / "t"), "--fetch", str(tmp_path / "f"), "--write", str(tmp_path / "w"),
            "--clock", str(tmp_path / "c"), "--cal-fetch", str(tmp_path / "cf"), "--cal-write",
            str(tmp_path / "cw"), "--bench", str(tmp_path / "b.json"), "--md", md, "--json", js, "--title", "t"])
    out = json.load(open(js))
    # timed steps are the last 3 (durations scale with 3, 4, 5): mean factor 4
    assert abs(out["fc1_wgrad_kernel_ms"] - 4 * (21_000 + 560_000) * 1e-6) < 1e-9
    assert abs(out["fc1_swiglu_kernel_ms"] - 4 * (4_000 + 500_000) * 1e-6) < 1e-9
    assert abs(out["combine_bwd_kernel_ms"] - 4 * 55_000 * 1e-6) < 1e-9
    # calibration: 1 GiB per copy -> 2048 B per FETCH unit, 1024 B per WRITE unit
    assert out["fetch_scale"] == 2048.0 and out["write_scale"] == 1024.0
    assert out["fc2_wgrad_read_bytes"] == (10.0 + 1000.0) * 2048.0
    assert out["fc1_wgrad_write_bytes"] == 2000.0 * 1024.0
    text = open(md).read()
    assert "| fc1_wgrad | `permute_kernel`" in text and "2.00 |" in text  # clock column
    assert "second stream" not in text  # every stage has a bench time


def test_overlap_note_for_stage_without_bench_time(tmp_path):
    _write_trace(str(tmp_path / "t"), 1)
    for d, c in (("f", "FETCH_SIZE"), ("w", "WRITE_SIZE")):
        _write_pmc(str(tmp_path / d), c, lambda n: 1.0)
    _write_pmc(str(tmp_path / "cf"), "FETCH_SIZE", lambda n: 524288.0, copies=1)
    _write_pmc(str(tmp_path / "cw"), "WRITE_SIZE", lambda n: 1048576.0, copies=1)
    stages = {s: 1.0 for s in R.STAGE_ORDER if s not in ("swiglu_bwd", "act_recompute")}
    json.dump({"steps": 1, "ms_per_step": 3.0, "roofline": {"stage": "fc1_wgrad", "kernel_ms": 1.0},
               "stages_ms": stages, "gemm_stages": {}, "bandwidth_kernels": {}}, open(tmp_path / "b.json", "w"))
    md = str(tmp_path / "o.md")
    R.main(["--trace", str(tmp_path / "t"), "--fetch", str(tmp_path / "f"), "--write", str(tmp_path / "w"),
            "--cal-fetch", str(tmp_path / "cf"), "--cal-write", str(tmp_path / "cw"), "--bench",
            str(tmp_path / "b.json"), "--md", md])
    assert "(`swiglu_bwd`) ran on the backward's second stream" in open(md).read()
