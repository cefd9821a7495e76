"""bench.py's host side, on the CPU: the one-GPU refusal and the CPU-baseline legs (the reference x86_avx2 family
over a small decode batch and a small prefill chunk), so a broken CPU leg shows here before a GPU run."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from silvann_amd import workloads as W  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_decode_cpu_baseline_line(ref):
    w = W.decode("cpu-leg", 16, 2, 128, [700, 33, 1500], page_size=256, seed=5)
    line = bench.cpu_baseline(w, threads=2, budget=0.3)
    assert line["kind"] == "reference" and line["cores"] == 2 and line["unit"] == "GB/s"
    assert line["value"] > 0
    assert "3 sequences" in line["sample"]


def test_prefill_cpu_baseline_line(ref):
    w = W.causal("cpu-leg", 8, 2, 128, 300, 40, page_size=32, seed=6)
    line = bench.cpu_baseline_prefill(w, threads=2, budget=0.2)
    assert line["kind"] == "reference" and line["unit"] == "TFLOP/s" and line["value"] > 0
