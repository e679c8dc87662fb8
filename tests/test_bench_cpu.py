"""bench.py's command-line contract where it needs no GPU: more than one GPU is refused with a
message, and without a GPU the benchmark fails loudly instead of falling back to the CPU."""

import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU path")
def test_no_gpu_fails_loudly():
    r = run("--steps", "1", "--warmup", "0")
    assert r.returncode == 2 and "needs a GPU" in r.stderr and r.stdout == ""


def test_steps_below_one_are_refused():
    r = run("--steps", "0")
    assert r.returncode == 2 and "--steps >= 1" in r.stderr and r.stdout == ""


def _canned_rows():
    """One row of every kind bench.py reports, under every name the stdout line carries."""
    import bench

    rows = {}
    for n in bench.LINE_ROWS:
        if n.startswith("moe_layer"):
            r = {"ms_per_step": 1.158654754999997, "tokens_per_s": 863.0698624285218, "hit_rate": 0.67875,
                 "misses_per_token": 2.57, "refill_GB_s": 51.89520379606102, "tokens": 1, "steps": 200}
        elif n.startswith("expert_file_stack"):
            r = {"ms_per_token": 134.6397941666666, "tokens_per_s": 7.427224664070191, "hit_rate": 0.16071428571428573,
                 "demand_GB_read": 2.65089024, "prefetch": {"issued": 216}, "direct": True}
        elif n.startswith("expert_file"):
            r = {"ms_per_lookup_median": 7.738015999997572, "ms_per_lookup_p90": 8.854009000000218,
                 "ms_per_expert": 7.738015999997572, "GB_s": 2.4296460488070717, "direct": True, "readers": 8}
        else:
            r = {"ms_per_step": 0.0035183333333333336, "GB_s": 2221.8142857142857, "frac_hbm_peak": 0.27772678571428573,
                 "alg_bytes": 7817216, "steps": 20, "frac_of_read_floor": 0.874213}
            if "gemm" in n:
                r["TFLOP_s"] = 239.5312345
            if n.startswith(("moe", "ref_abi_moe")):
                r["tokens_per_s"] = 24987.755999560213
        r["workload"] = n
        rows[n] = r
    rows["cpu_scalar_oracle"] = {"workload": "cpu_scalar_oracle_fp4_gemv_2048x7168", "GB_s": 1.28, "cores": 1,
                                 "ms_per_gemv": 6.09, "sample": "x" * 120}
    # rows that only go to stderr and --rows-out
    rows["ref_method_gemv_fp8_512x5120"] = {"workload": "ref_method_gemv_fp8_512x5120", "us": 7.29, "GB_s": 359.5,
                                            "bytes": 2621440, "reps": 200}
    return rows


def _canned_head():
    return {"workload": "fp4_gemv_2048x7168_m1", "rows": 2048, "k": 7168, "m": 1, "ms_per_step": 0.0035083333333,
            "steps": 20, "alg_bytes": 7817216, "GB_s": 2228.2219, "frac_hbm_peak": 0.2785277, "weight_copies": 69,
            "graph": True, "frac_of_read_floor": 0.8742}


def _canned_timing():
    return {"samples": 35, "steps_per_sample": 20, "sample_ms_min": 0.0698712345, "sample_ms_median": 0.07016666,
            "sample_ms_max": 0.0712345678, "stamp_pair_us": 1.612345678, "clock_khz": 100000,
            "events_ms_per_step_whole_replay": 0.003712345678, "isolated_launches": 64,
            "isolated_launch_us": 3.81234567}


def test_stdout_line_is_compact_and_parses():
    # the driver keeps only a tail of stdout + stderr: the line must stay whole and small with every
    # row present, and json must read back the headline, roofline, CPU baseline and target rows
    import json

    import bench

    cpu = {"value": 0.92, "unit": "GB/s", "cores": 16, "kind": "port", "sample": "s" * 300}
    prof = {"kernel_dur_median_us": 3.84, "kernel_dur_mean_us": 3.78, "step_us_under_profiler": 8.54}
    line = bench.make_line(_canned_head(), _canned_rows(), cpu, _canned_timing(), 5, traffic=7982353, profiled=prof)
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) <= bench.LINE_MAX_BYTES, len(text)
    d = json.loads(text)
    assert d["value"] == round(_canned_head()["GB_s"], 2) and d["steps"] == 20 and d["warmup"] == 5
    assert d["roofline"]["achieved"] == d["value"] and d["roofline"]["frac"] == round(d["value"] / 8000.0, 4)
    assert d["roofline"]["traffic"] == 7982353 and d["roofline"]["profiled"] == prof
    assert abs(d["roofline"]["isolated_frac"] - 7817216 / 3.81234567e-6 / 1e9 / 8000.0) < 1e-4
    assert d["cpu_baseline"]["kind"] == "port" and d["cpu_baseline"]["cores"] == 16
    assert set(d["target_7168x2048"]) == {"fp4", "fp8", "fp4_batch16", "fp8_batch16", "fp4_batch64", "fp8_batch64"}
    assert set(d["extra"]) == set(bench.LINE_ROWS)
    assert d["extra"]["fp4_gemm_q_m64_2048x7168"][3] == 240.0  # TFLOP/s, 3 significant digits
    assert d["extra"]["moe_layer_t1_fp4_256x_top8_lru64"]["hit"] == 0.679


def test_whole_output_fits_the_driver_tail():
    # stderr gets one short line per row; with every row of a default run, stdout + stderr must stay
    # well under the ~14 KB the driver keeps
    import json

    import bench

    rows = _canned_rows()
    while len(rows) < 86:  # a default run reports 81 rows; names of 40 characters
        r = dict(rows["fp4_gemm_q_m64_2048x7168"])
        r["workload"] = f"workload_name_for_sizing_{len(rows):04d}x4096_m1"
        rows[r["workload"]] = r
    err = "\n".join(bench.stderr_text(r) for r in rows.values())
    line = json.dumps(bench.make_line(_canned_head(), rows, None, _canned_timing(), 5), separators=(",", ":"))
    assert len(err) + len(line) < 12000, (len(err), len(line))


def test_trace_summary_reads_a_kernel_trace(tmp_path):
    # start-to-start spacing counts only consecutive dispatches of the matched kernel
    import bench

    p = tmp_path / "t_kernel_trace.csv"
    hdr = '"Kind","Kernel_Name","Start_Timestamp","End_Timestamp"\n'
    rows = [("k_gemv<a>", 0, 30), ("k_gemv<a>", 50, 80), ("k_gemv<a>", 100, 140), ("k_other", 150, 160),
            ("k_gemv<a>", 200, 230)]
    p.write_text(hdr + "".join(f'"KERNEL_DISPATCH","{n}",{s},{e}\n' for n, s, e in rows))
    s = bench.trace_summary(str(p), r"k_gemv<")
    assert s["calls"] == 4 and s["pairs"] == 2
    assert s["dur_median_ns"] == 30 and s["spacing_median_ns"] == 50 and s["gap_median_ns"] == 20


def test_trace_table_groups_by_grid(tmp_path):
    import bench

    p = tmp_path / "t_kernel_trace.csv"
    hdr = '"Kind","Kernel_Name","Start_Timestamp","End_Timestamp","Grid_Size_X","Grid_Size_Y","Workgroup_Size_X"\n'
    rows = [("k_a", 0, 10, 64, 1), ("k_a", 20, 40, 64, 1), ("k_a", 50, 55, 128, 2), ("k_b", 60, 90, 64, 1)]
    p.write_text(hdr + "".join(f'"KERNEL_DISPATCH","{n}",{s},{e},{gx},{gy},64\n' for n, s, e, gx, gy in rows))
    t = {(r["kernel"], r["grid"]): r for r in bench.trace_table(str(p), r"k_a")}
    assert set(t) == {("k_a", "64x1"), ("k_a", "128x2")}
    assert t[("k_a", "64x1")]["calls"] == 2 and t[("k_a", "64x1")]["median_ns"] == 15
    assert t[("k_a", "128x2")]["mean_ns"] == 5


def test_counter_table_medians(tmp_path):
    import bench

    p = tmp_path / "p_counter_collection.csv"
    hdr = '"Dispatch_Id","Grid_Size","Kernel_Name","Counter_Name","Counter_Value"\n'
    rows = [(1, 64, "k_a", "FETCH_SIZE", 10.0), (2, 64, "k_a", "FETCH_SIZE", 30.0), (3, 64, "k_a", "FETCH_SIZE", 20.0),
            (4, 128, "k_a", "FETCH_SIZE", 5.0), (5, 64, "k_b", "FETCH_SIZE", 7.0)]
    p.write_text(hdr + "".join(f'{d},{g},"{n}","{c}",{v}\n' for d, g, n, c, v in rows))
    t = {(r["grid"], r["counter"]): r for r in bench.counter_table(str(p), r"k_a")}
    assert t[("64", "FETCH_SIZE")]["median"] == 20.0 and t[("64", "FETCH_SIZE")]["dispatches"] == 3
    assert t[("128", "FETCH_SIZE")]["median"] == 5.0 and len(t) == 2


def test_counter_last_dispatches(tmp_path):
    import bench

    p = tmp_path / "p_counter_collection.csv"
    hdr = '"Dispatch_Id","Grid_Size","Kernel_Name","Counter_Name","Counter_Value"\n'
    rows = [(3, 64, "copy", "FETCH_SIZE", 7.0), (1, 64, "copy", "FETCH_SIZE", 5.0), (9, 64, "copy", "FETCH_SIZE", 32.0),
            (7, 64, "copy", "FETCH_SIZE", 31.0), (8, 64, "k_a", "FETCH_SIZE", 1.0)]
    p.write_text(hdr + "".join(f'{d},{g},"{n}","{c}",{v}\n' for d, g, n, c, v in rows))
    got = bench.counter_last(str(p), r"copy", 2)
    assert [(r["dispatch"], r["value"]) for r in got] == [(7, 31.0), (9, 32.0)]
