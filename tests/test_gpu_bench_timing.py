"""The measurement instrument bench.py times steps with: clock stamps captured between launches.

A stamp records the GPU's wall clock as its one-thread launch starts (stbl_amd_clock_stamp); two
stamps around a streaming read must be ordered and a plausible time apart, and bench.timed_steps
must time exactly the requested steps per sample."""

import ctypes
import math

import pytest
import torch

import bench
from stblarge_amd import _lib, ops

pytestmark = pytest.mark.gpu


def test_clock_stamps_bracket_a_launch(gpu):
    lib = _lib.load()
    khz = ctypes.c_int(0)
    _lib.check(lib.stbl_amd_clock_rate_khz(ctypes.byref(khz)), "clock_rate_khz")
    assert khz.value > 0
    t = torch.zeros(2, dtype=torch.int64, device=gpu)
    nbytes = 64 << 20
    src = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    sink = torch.zeros(int(lib.stbl_amd_read_floor_sink_words(nbytes)), dtype=torch.int32, device=gpu)
    st = ops._stream()
    _lib.check(lib.stbl_amd_clock_stamp(ctypes.c_void_p(t.data_ptr()), 0, st), "clock_stamp")
    _lib.check(lib.stbl_amd_read_floor(ctypes.c_void_p(src.data_ptr()), nbytes, ops._ptr(sink), st), "read_floor")
    _lib.check(lib.stbl_amd_clock_stamp(ctypes.c_void_p(t.data_ptr()), 1, st), "clock_stamp")
    t0, t1 = t.cpu().tolist()
    ms = (t1 - t0) / khz.value
    # 64 MiB at no more than 8 TB/s takes at least 8 us; a stamp pair on an idle GPU well under 1 s
    assert 0.008 < ms < 1000.0, ms


def test_timed_steps_samples_exactly_the_requested_steps(gpu):
    lib = _lib.load()
    nbytes, copies = 1 << 20, 4
    buf = torch.zeros(copies * nbytes, dtype=torch.uint8, device=gpu)
    sink = torch.zeros(int(lib.stbl_amd_read_floor_sink_words(nbytes)), dtype=torch.int32, device=gpu)

    def launch(i):
        _lib.check(lib.stbl_amd_read_floor(ctypes.c_void_p(buf.data_ptr() + i * nbytes), nbytes, ops._ptr(sink),
                                           ops._stream()), "read_floor")

    ms, n = bench.timed_steps(torch, launch, copies, 7, 2)
    assert n == 7 and 0.0 < ms < 1.0
    tm = bench.LAST_TIMING
    assert tm["samples"] == math.ceil(10 * copies / 7) and tm["steps_per_sample"] == 7
    assert tm["sample_ms_min"] <= tm["sample_ms_median"] <= tm["sample_ms_max"]
    assert abs(tm["sample_ms_median"] / 7 - ms) < 1e-12


def test_bench_line_reports_the_requested_steps(gpu):
    # the driver's form: `--steps K --warmup W` gives one JSON line whose steps is K, with the
    # roofline and the timing samples (the CPU baseline leg is skipped here to keep the test short)
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--only", "fp4", "--no-cpu", "--steps", "20",
                        "--warmup", "5"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    assert d["steps"] == 20 and d["warmup"] == 5 and d["n_gpus"] == 1
    assert d["timing"]["steps_per_sample"] == 20 and d["timing"]["samples"] >= 10
    assert abs(d["value"] - 7817216 / (d["ms_per_step"] * 1e-3) / 1e9) < 0.01 * d["value"]
    assert d["roofline"]["achieved"] == d["value"] and 0 < d["roofline"]["frac"] < 1
    # the headline launch alone between stamps takes at least a bare launch and at most a few steps
    assert d["timing"]["isolated_launches"] == 64
    assert 0.5 * d["ms_per_step"] * 1e3 < d["roofline"]["isolated_launch_us"] < 10 * d["ms_per_step"] * 1e3


@pytest.mark.timeout(900)
def test_bench_driver_form_prints_one_whole_line(gpu):
    # exactly the driver's command: every row, the CPU baseline; stdout is one JSON line of at most
    # 4 KB carrying the roofline, the CPU baseline and the target shape's rows, and stdout + stderr
    # stay well inside the tail the driver keeps
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "1", "--steps", "20", "--warmup", "5"],
                       capture_output=True, text=True, timeout=850)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1 and len(lines[0]) <= bench.LINE_MAX_BYTES, [len(x) for x in lines]
    assert len(r.stdout) + len(r.stderr) < 12000, (len(r.stdout), len(r.stderr))
    d = json.loads(lines[0])
    assert d["steps"] == 20 and d["warmup"] == 5 and d["roofline"]["bound"] == "hbm"
    assert d["cpu_baseline"]["value"] > 0 and d["cpu_baseline"]["cores"] >= 1
    assert {"fp4", "fp8"} <= set(d["target_7168x2048"]) and len(d["extra"]) >= 20
