"""bench.py keeps its one JSON line when an auxiliary leg fails (CPU only).

The E2E and sweep legs run as child processes; a crash, a non-zero exit or a
time-out there is recorded in the line, never raised. The CPU baseline times
the GPU headline's own seeded operands."""
import json
import subprocess
import sys
import types
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def _args():
    return types.SimpleNamespace(steps=8, warmup=2)


def test_child_timeout_and_exit_code_are_reported(monkeypatch):
    assert bench._child([sys.executable, "-c", "import time; time.sleep(30)"], 1) == "timed out after 1 s"
    assert bench._child([sys.executable, "-c", "raise SystemExit(3)"], 30) == "exit code 3"
    assert bench._child([sys.executable, "-c", "pass"], 30) is None


def test_e2e_failure_is_recorded_not_raised(monkeypatch):
    monkeypatch.setattr(bench, "_child", lambda cmd, t: "timed out after 420 s")
    rep = bench.run_e2e()
    assert "timed out" in rep["error"]
    monkeypatch.setattr(bench, "_child", lambda cmd, t: None)   # exit 0 but no report file
    assert "no report" in bench.run_e2e()["error"]


def test_child_converts_subprocess_timeout(monkeypatch):
    def boom(*a, **kw):
        raise subprocess.TimeoutExpired("x", 5)
    monkeypatch.setattr(subprocess, "run", boom)
    assert bench._child(["x"], 5) == "timed out after 5 s"


def test_sweep_child_keeps_completed_records(monkeypatch):
    def fake_child(cmd, t):
        assert "--sweep-only" in cmd
        tag = cmd[cmd.index("--tag") + 1]
        bench.sweep_file(tag).write_text(json.dumps(dict(cfg="cfg1", mode="w8a16", M=64, N=6144, K=1024,
                                                         path="p", us=1.0, frac=0.5)) + "\n")
        return "exit code -11"
    monkeypatch.setattr(bench, "_child", fake_child)
    recs, err = bench.run_sweep_child(False, "unittest", False)
    try:
        assert len(recs) == 1 and "after 1 cases" in err and "-11" in err
    finally:
        bench.sweep_file("unittest").unlink()


def test_line_parses_with_failed_legs():
    roof = dict(bound="hbm", achieved=1.0, peak=8000.0, unit="GB/s", frac=0.1, traffic=None)
    line = bench.build_line(_args(), 123.4, 1e-5, 256, 4096, 1024, 100, roof,
                            dict(error="cpu baseline failed"), None, "sweep leg failed after 0 cases: exit code 1",
                            dict(error="e2e leg failed: timed out after 420 s"))
    back = json.loads(json.dumps(line))
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "roofline", "cpu_baseline"):
        assert key in back
    assert back["value"] == 123.4 and back["targets"] == {}
    assert "e2e" in back and "error" in back["e2e"] and back["sweep_error"].startswith("sweep leg failed")


def test_cpu_baseline_uses_headline_operands():
    """make_inputs is seeded on the host: the CPU call and a second call give
    identical operands, with BASELINE's distributions (outlier columns, per-channel int8)."""
    m, n, k = 8, 64, 1024
    x1, q1, s1 = bench.make_inputs("w8a8", m, n, k, "cpu", pool_bytes=0)
    x2, q2, s2 = bench.make_inputs("w8a8", m, n, k, None, pool_bytes=0)
    assert torch.equal(x1, x2) and torch.equal(q1[0], q2[0]) and torch.equal(s1[0], s2[0])
    assert x1.dtype == torch.bfloat16 and q1[0].dtype == torch.int8
    col_amax = x1.float().abs().amax(0)
    assert (col_amax > 15).sum() >= 1                      # the x20 outlier columns
    assert int(q1[0].abs().amax(1).min()) == 127            # absmax/127 per channel -> every row reaches 127
    assert 0.02 * 2 / 127 < float(s1[0].mean()) < 0.02 * 6 / 127
