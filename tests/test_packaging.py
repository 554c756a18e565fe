"""A non-editable install ships the gfx950 library: `pip install .` into a temporary
target puts libbevk.so next to _bevk.py, and a fresh interpreter with only that target on
its path loads it (no GPU needed: the library loads and reports its version)."""
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_pip_install_ships_library(tmp_path):
    target = tmp_path / "site"
    res = subprocess.run([sys.executable, "-m", "pip", "install", ".", "--no-deps",
                          "--no-build-isolation", "--no-index", "--target", str(target), "-q"],
                         cwd=ROOT, capture_output=True, text=True, timeout=900)
    for d in ("build", "bev_kernels_amd.egg-info"):
        shutil.rmtree(os.path.join(ROOT, d), ignore_errors=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert (target / "libbevk.so").is_file()
    assert (target / "_bevk.py").is_file()
    code = ("import _bevk, os; print(_bevk.library_path()); print(_bevk.version()); "
            "import modulated_deform_conv, msda_opt2")
    env = dict(os.environ, PYTHONPATH=str(target))
    env.pop("BEVK_LIBRARY", None)
    out = subprocess.run([sys.executable, "-c", code], cwd=str(tmp_path), env=env,
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    lib_path, version = out.stdout.split()[:2]
    assert lib_path == str(target / "libbevk.so")
    assert version == "bevk"
