"""The package installs without the repository on sys.path: a wheel built
offline from pto-einsum_amd/ (setup.cfg + setup.py, mirroring the reference's
setup.cfg:11-28 with the kernel library and C headers as package data) is
installed into a scratch directory, and a fresh interpreter imports
pto_einsum from there, finds its bundled headers and library, and runs a CPU
einsum through the JIT path (no GPU needed)."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def installed(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("pkg")
    wheel_dir, target = tmp / "wheel", tmp / "site"
    r = subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-deps", "--no-build-isolation", "--no-index",
                        "-w", str(wheel_dir), os.path.join(ROOT, "pto-einsum_amd")],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    wheels = glob.glob(str(wheel_dir / "*.whl"))
    assert len(wheels) == 1 and "linux" in os.path.basename(wheels[0])
    # The build leaves no header copy in the source package (it would shadow
    # include/ for the in-tree JIT and go stale).
    assert not os.path.exists(os.path.join(ROOT, "pto-einsum_amd", "pto_einsum", "include"))
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-deps", "--no-index", "--target", str(target),
                        wheels[0]], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return target


def test_import_from_installed_tree(installed, tmp_path):
    code = f"""
import os, sys
sys.path = [p for p in sys.path if not p.startswith({ROOT!r})]
sys.path.insert(0, {str(installed)!r})
os.environ["EINSUM_BUILD_DIR"] = {str(tmp_path)!r}
import numpy as np, torch
import pto_einsum
from pto_einsum import EinsumBuilder, INCLUDE_DIR, einsum, runtime
assert pto_einsum.__file__.startswith({str(installed)!r}), pto_einsum.__file__
assert INCLUDE_DIR.startswith({str(installed)!r}) and os.path.isfile(os.path.join(INCLUDE_DIR, "pto_einsum_hip.h"))
assert os.path.isfile(runtime.core_library_path()) and runtime.core_library_path().startswith({str(installed)!r})
a, b = torch.rand(5, 7), torch.rand(7, 3)
got = einsum("ij,jk->ik", a, b, device="cpu")
assert np.allclose(got.numpy(), a.numpy() @ b.numpy(), rtol=1e-5, atol=1e-6)
print("ok", pto_einsum.__version__)
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600, cwd=str(tmp_path))
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
