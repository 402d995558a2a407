"""Packaging of `feather_ops` for MI355X (gfx950): `pip install --no-build-isolation ./feather-ops_amd`.

The reference installs the same package name with setuptools and a torch CUDAExtension
(`setup.py:132-145` there). Here the native code is built by this directory's Makefile, which the
build_py step runs before copying the package: `feather_ops/libfeather_ops_gfx950.so` (the HIP kernels and
the C ABI of include/feather_ops.h) and `feather_ops/_C.so` (the torch library, which finds the former
through its $ORIGIN run path). Both ship inside the package, so an installed `import feather_ops` loads
the installed native code. The build needs the repository's `include/` next to this directory, hipcc and
the ROCm torch it links against; it is a platform wheel (gfx950 code objects, a CPython-linked extension).
"""

import os
import pathlib
import subprocess

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

HERE = pathlib.Path(__file__).resolve().parent
NATIVE = ["libfeather_ops_gfx950.so", "_C.so"]


class MakeThenBuildPy(build_py):
    """Builds the native libraries in place (make is incremental), then copies the package."""

    def run(self):
        jobs = str(min(8, os.cpu_count() or 1))
        subprocess.run(["make", "-C", str(HERE), f"-j{jobs}"] + [f"feather_ops/{name}" for name in NATIVE],
                       check=True)
        super().run()


class NativeDistribution(Distribution):
    """A distribution with native code, so the wheel is tagged for this platform and Python."""

    def has_ext_modules(self):
        return True


setup(
    name="feather-ops",
    version="0.1.0+gfx950",
    description="fp16/bf16 x fp8 scaled matmul for MI355X (gfx950): hand-written CDNA4 HIP kernels",
    packages=["feather_ops"],
    package_data={"feather_ops": NATIVE},
    python_requires=">=3.10",
    install_requires=[],
    cmdclass={"build_py": MakeThenBuildPy},
    distclass=NativeDistribution,
    zip_safe=False,
)
