"""bench.py's command-line contract, checked on the CPU: one GPU only, and
defaults that finish within minutes (K timed steps after W warmup steps,
preceded by an untimed settle phase of C5 steps)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


def test_defaults(monkeypatch):
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    a = bench.parse_args()
    assert (a.gpus, a.steps, a.warmup) == (1, 20, 5)
    assert a.settle_ms == 500.0 and not a.quick and not a.no_cpu


def test_flags(monkeypatch):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "7", "--warmup", "3",
                                      "--settle-ms", "0", "--quick", "--no-cpu"])
    a = bench.parse_args()
    assert (a.steps, a.warmup, a.settle_ms, a.quick, a.no_cpu) == (7, 3, 0.0, True, True)
