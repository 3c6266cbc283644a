"""bench.py's command-line contract and its CPU baseline, on the CPU.

- `--gpus N` above 1 exits with status 2 and says that only one GPU is
  measured (no GPU is touched before that check).
- An unknown `--secondary` name is a usage error.
- The CPU baseline (the oracle's gather + SDPA path, timed) returns the
  fields the bench line's `cpu_baseline` object carries.
"""

import importlib.util
import subprocess
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_unknown_secondary_is_a_usage_error():
    r = run_bench("--secondary", "config9")
    assert r.returncode == 2 and "unknown secondary config9" in r.stderr


def test_cpu_baseline_reports_its_sample():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    from moe_engine import workloads

    w = workloads.make_workload([40, 7, 0, 100, 16, 3, 64, 1, 33], block_size=16, dtype=torch.bfloat16, seed=2,
                                device="cpu")
    res = bench.cpu_baseline(torch, w, 0.05)
    assert res["kind"] == "port" and res["unit"] == "GB/s"
    assert res["value"] > 0 and res["cores"] == torch.get_num_threads()
    # every 8th sequence: 0 and 8
    assert "sequences [0, 8]" in res["sample"] and "73 tokens" in res["sample"]
    assert res["ms_per_pass"] > 0
