"""bench.py's command-line contract on the CPU: one GPU only (``--gpus N`` above 1 exits with a
message before anything touches a device), and no silent fallback when no GPU is present."""

from __future__ import annotations

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(REPO, "bench.py")


def _run(*args: str, env: dict | None = None) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=300,
                          env={**os.environ, **(env or {})})


def test_more_than_one_gpu_is_refused_with_a_message():
    res = _run("--gpus", "2")
    assert res.returncode == 2
    assert "measures one GPU" in res.stderr and "--gpus 2" in res.stderr
    assert res.stdout == ""  # no JSON line


def test_a_second_rank_is_refused_too():
    res = _run("--gpus", "1", env={"WORLD_SIZE": "2"})
    assert res.returncode == 2 and "measures one GPU" in res.stderr


def test_no_gpu_means_no_bench_line():
    res = _run("--steps", "1", "--warmup", "0", env={"HIP_VISIBLE_DEVICES": "", "CUDA_VISIBLE_DEVICES": ""})
    assert res.returncode != 0
    assert "needs a ROCm GPU" in res.stderr
    assert res.stdout == ""
