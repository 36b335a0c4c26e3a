"""bench.py's command-line contract, checked without a GPU: one GPU only (a clear message and a
non-zero exit for --gpus N > 1, before any device work) and the documented options."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line for a refused run


def test_options_parse_with_their_defaults(monkeypatch):
    sys.path.insert(0, str(ROOT))
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py"])
    a = bench.parse()
    assert (a.gpus, a.steps, a.warmup) == (1, 200, 20)
    assert not a.no_sweep and not a.no_e2e and not a.no_cpu
    monkeypatch.setattr(sys, "argv", ["bench.py", "--no-sweep", "--no-e2e", "--no-cpu", "--steps", "5", "--warmup", "1"])
    a = bench.parse()
    assert a.no_sweep and a.no_e2e and a.no_cpu and (a.steps, a.warmup) == (5, 1)
