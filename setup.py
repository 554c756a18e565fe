"""Build & install the MI355X (gfx950) bev-kernels.

    python setup.py build_ext --inplace     # hipcc --offload-arch=gfx950 -> bev-kernels_amd/libbevk.so
    pip install . --no-build-isolation      # installs the packages and libbevk.so
    pip install -e . --no-build-isolation   # editable install (the in-tree library)

The native part is one shared library with a C ABI (include/bev_kernels.h) built by
bev-kernels_amd/csrc/build.py; the Python packages bind it with ctypes, so no PyTorch C++
extension (and no hipify step) is involved. _bevk loads the library from its own
directory, so an install puts libbevk.so next to _bevk.py.
"""
import glob
import os
import sys

from setuptools import Command, Distribution, setup
from setuptools.command.build_ext import build_ext
from setuptools.command.build_py import build_py

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = "bev-kernels_amd"
LIB = os.path.join(HERE, PKG_DIR, "libbevk.so")


def _library_stale() -> bool:
    if not os.path.exists(LIB):
        return True
    csrc = os.path.join(HERE, PKG_DIR, "csrc")
    srcs = [p for ext in ("*.hip", "*.cpp", "*.h", "build.py")
            for p in glob.glob(os.path.join(csrc, ext))]
    srcs += glob.glob(os.path.join(HERE, "include", "*.h"))
    return any(os.path.getmtime(s) > os.path.getmtime(LIB) for s in srcs)


def _build_library(force: bool = False) -> str:
    """hipcc for gfx950 (bev-kernels_amd/csrc/build.py), when forced or out of date."""
    if force or _library_stale():
        sys.path.insert(0, os.path.join(HERE, PKG_DIR, "csrc"))
        import build as hip_build
        hip_build.build(jobs=int(os.environ.get("MAX_JOBS", "8")), verbose=True)
    return LIB


class BuildHip(build_ext):
    """Compiles libbevk.so with hipcc for gfx950 (in-tree); outside --inplace builds the
    library also goes to the build tree next to _bevk.py."""

    def run(self):
        lib = _build_library(force=self.inplace)
        if not self.inplace and self.build_lib:
            os.makedirs(self.build_lib, exist_ok=True)
            self.copy_file(lib, os.path.join(self.build_lib, "libbevk.so"))


class BuildPy(build_py):
    """The Python modules plus libbevk.so, which _bevk loads from its own directory."""

    def run(self):
        super().run()
        lib = _build_library()
        self.copy_file(lib, os.path.join(self.build_lib, "libbevk.so"))


class BinaryDistribution(Distribution):
    """The wheel carries a gfx950 shared library: not a pure-Python distribution."""

    def has_ext_modules(self):
        return True


class Clean(Command):
    user_options = []

    def initialize_options(self):
        pass

    def finalize_options(self):
        pass

    def run(self):
        import shutil
        shutil.rmtree(os.path.join(HERE, PKG_DIR, "_build"), ignore_errors=True)
        if os.path.exists(LIB):
            os.remove(LIB)


setup(
    name="bev_kernels_amd",
    version="0.1.0",
    package_dir={"": PKG_DIR},
    packages=["modulated_deform_conv", "msda_opt2", "msda_musa_opt2"],
    py_modules=["_bevk", "_modulated_deform_conv_ext"],
    distclass=BinaryDistribution,
    cmdclass={"build_ext": BuildHip, "build_py": BuildPy, "clean": Clean},
)
