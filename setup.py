"""Build & install the MI355X (gfx950) bev-kernels.

    python setup.py build_ext --inplace     # hipcc --offload-arch=gfx950 -> bev-kernels_amd/libbevk.so
    pip install -e . --no-build-isolation   # editable install of the Python packages

The native part is one shared library with a C ABI (include/bev_kernels.h) built by
bev-kernels_amd/csrc/build.py; the Python packages bind it with ctypes, so no PyTorch C++
extension (and no hipify step) is involved.
"""
import os
import sys

from setuptools import Command, setup
from setuptools.command.build_ext import build_ext

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = "bev-kernels_amd"


class BuildHip(build_ext):
    """Compiles libbevk.so with hipcc for gfx950 (in-tree)."""

    def run(self):
        sys.path.insert(0, os.path.join(HERE, PKG_DIR, "csrc"))
        import build as hip_build
        lib = hip_build.build(jobs=int(os.environ.get("MAX_JOBS", "8")), verbose=True)
        print("built", lib)


class Clean(Command):
    user_options = []

    def initialize_options(self):
        pass

    def finalize_options(self):
        pass

    def run(self):
        import shutil
        shutil.rmtree(os.path.join(HERE, PKG_DIR, "_build"), ignore_errors=True)
        lib = os.path.join(HERE, PKG_DIR, "libbevk.so")
        if os.path.exists(lib):
            os.remove(lib)


setup(
    name="bev_kernels_amd",
    version="0.1.0",
    package_dir={"": PKG_DIR},
    packages=["modulated_deform_conv", "msda_opt2", "msda_musa_opt2"],
    py_modules=["_bevk", "_modulated_deform_conv_ext"],
    package_data={"": ["libbevk.so"]},
    cmdclass={"build_ext": BuildHip, "clean": Clean},
)
