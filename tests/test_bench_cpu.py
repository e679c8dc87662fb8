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
