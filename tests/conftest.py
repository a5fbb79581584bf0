import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "pto-einsum_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def build_dir(tmp_path_factory):
    """A per-session JIT cache so tests never share the user's ./build."""
    d = tmp_path_factory.mktemp("einsum_build")
    old = os.environ.get("EINSUM_BUILD_DIR")
    os.environ["EINSUM_BUILD_DIR"] = str(d)
    yield str(d)
    if old is None:
        os.environ.pop("EINSUM_BUILD_DIR", None)
    else:
        os.environ["EINSUM_BUILD_DIR"] = old


def gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False
