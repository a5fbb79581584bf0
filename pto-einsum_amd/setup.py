"""Build step of the package: compiles the gfx950 core library from csrc/
(make; incremental) into pto_einsum/lib/ (package data, setup.cfg) and copies
the C headers from the repository's include/ into the build tree's
pto_einsum/include/, so both ship in the wheel.  The headers are not copied
into the source tree: there the per-shape sources compile against include/
itself, and a copy would go stale when a header changes.  Set PTO_EINSUM_HIPCC / PTO_EINSUM_ARCH to override hipcc and the
target (gfx950)."""
import os
import shutil
import subprocess

from setuptools import Distribution, setup
from setuptools.command.build_py import build_py

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildWithKernels(build_py):
    def run(self):
        args = ["make", "-s", "-j", str(min(16, os.cpu_count() or 4)), "-C", os.path.join(HERE, "csrc")]
        if os.environ.get("PTO_EINSUM_HIPCC"):
            args.append("HIPCC=" + os.environ["PTO_EINSUM_HIPCC"])
        if os.environ.get("PTO_EINSUM_ARCH"):
            args.append("ARCH=" + os.environ["PTO_EINSUM_ARCH"])
        subprocess.run(args, check=True)
        super().run()
        inc_src = os.path.join(HERE, "..", "include")
        inc_dst = os.path.join(self.build_lib, "pto_einsum", "include")
        os.makedirs(inc_dst, exist_ok=True)
        for name in sorted(os.listdir(inc_src)):
            if name.endswith(".h"):
                shutil.copy2(os.path.join(inc_src, name), os.path.join(inc_dst, name))


class BinaryDistribution(Distribution):
    """The package carries a compiled library: platform-specific wheels."""

    def has_ext_modules(self):
        return True


setup(cmdclass={"build_py": BuildWithKernels}, distclass=BinaryDistribution)
