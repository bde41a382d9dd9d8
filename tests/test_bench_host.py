"""bench.py's command-line contract on a host without a GPU (CPU)."""

from __future__ import annotations

import pathlib
import subprocess
import sys

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""


@pytest.mark.skipif(torch.cuda.device_count() > 0, reason="a GPU is present: the bench would run")
def test_no_gpu_fails_loudly_instead_of_measuring_something_else():
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode != 0
    assert "GPU" in r.stderr
    assert r.stdout == ""
