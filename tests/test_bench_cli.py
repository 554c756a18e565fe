"""bench.py's command line on the CPU: more than one GPU is refused with a message before
any device work, and the timing options parse to their documented defaults."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""


def test_default_options(monkeypatch):
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    a = bench.parse_args()
    assert (a.gpus, a.steps, a.warmup, a.warm) == (1, 50, 10, False)
    assert a.settle_ms == bench.SETTLE_MS == 50.0
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "20", "--warmup", "5",
                                      "--settle-ms", "0"])
    a = bench.parse_args()
    assert (a.steps, a.warmup, a.settle_ms) == (20, 5, 0.0)
