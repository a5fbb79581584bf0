"""JIT compilation of per-shape libraries and their on-disk cache.

Reference counterpart: ``compile`` (builder.py:685-736), which md5-keys the
generated source and shells out to bisheng / g++.  Differences:

* the cache key covers everything the library depends on -- the generated
  source, the bundled headers, the compiler identity and flags, the target
  architecture and ``EINSUM_EXTRA_DEFINES`` -- not just the source text
  (the reference's key ignores its headers, README.md:222-224);
* the library is written to a temporary name and renamed into place, so
  concurrent builders of one shape never load a half-written file;
* GPU wrappers contain host code only (the kernels are in the core library),
  so they are compiled by the ROCm host compiler in well under a second.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
from functools import lru_cache
from typing import List, Tuple

from . import runtime


def _which(*candidates: str) -> str:
    for c in candidates:
        if os.path.isabs(c) and os.access(c, os.X_OK):
            return c
        p = shutil.which(c)
        if p:
            return p
    raise RuntimeError(f"no compiler found among {candidates}")


def gpu_host_compiler() -> str:
    env = os.getenv("EINSUM_HOST_CXX")
    if env:
        return env
    return _which("/opt/rocm/llvm/bin/clang++", "/opt/rocm/bin/amdclang++", "clang++", "g++")


def cpu_compiler() -> str:
    return os.getenv("EINSUM_CPU_CXX") or _which("g++", "c++")


def offload_arch() -> str:
    return os.getenv("EINSUM_OFFLOAD_ARCH", "gfx950")


def extra_defines() -> List[str]:
    return os.environ.get("EINSUM_EXTRA_DEFINES", "").split()


@lru_cache(maxsize=None)
def _compiler_id(cxx: str) -> str:
    try:
        out = subprocess.run([cxx, "--version"], capture_output=True, text=True, timeout=60).stdout
    except Exception:  # pragma: no cover - reported at compile time
        out = cxx
    return out.strip().splitlines()[0] if out.strip() else cxx


def _headers_digest(include_dir: str) -> str:
    h = hashlib.sha256()
    for name in sorted(os.listdir(include_dir)):
        if name.endswith(".h"):
            with open(os.path.join(include_dir, name), "rb") as f:
                h.update(name.encode())
                h.update(f.read())
    return h.hexdigest()


def command(device: str, src: str, out: str) -> List[str]:
    inc = runtime.include_dir()
    if device == "cpu":
        # The reference CPU route's flags (builder.py:705-709).
        return [cpu_compiler(), "-O3", "-shared", "-fPIC", "-std=c++17", "-I", inc,
                *extra_defines(), src, "-o", out]
    libdir = os.path.dirname(runtime.core_library_path())
    return [gpu_host_compiler(), "-O2", "-shared", "-fPIC", "-std=c++17", "-I", inc,
            *extra_defines(), src, "-o", out, "-L", libdir, "-lpto_einsum_hip",
            f"-Wl,-rpath,{libdir}"]


def cache_key(device: str, code: str) -> str:
    h = hashlib.sha256()
    h.update(code.encode())
    h.update(_headers_digest(runtime.include_dir()).encode())
    cxx = cpu_compiler() if device == "cpu" else gpu_host_compiler()
    h.update(_compiler_id(cxx).encode())
    h.update(device.encode())
    if device != "cpu":
        h.update(offload_arch().encode())
        h.update(runtime.core_library_id().encode())
    h.update(" ".join(extra_defines()).encode())
    return h.hexdigest()[:32]


def paths(build_base: str, key: str) -> Tuple[str, str, str]:
    """(target_dir, source path, library path) for a cache key."""
    tag = ""
    ed = extra_defines()
    if ed:
        tag = "_" + hashlib.sha256(" ".join(ed).encode()).hexdigest()[:8]
    target = os.path.join(build_base, key)
    return target, os.path.join(target, f"einsum_{key}{tag}.cpp"), os.path.join(target, f"einsum_{key}{tag}.so")


def compile_library(device: str, code: str, cpp_path: str, so_path: str) -> None:
    """Write ``code`` and build it into ``so_path`` unless already cached."""
    if os.path.exists(so_path):
        return
    os.makedirs(os.path.dirname(so_path), exist_ok=True)
    tmp_src = f"{cpp_path}.tmp{os.getpid()}"
    with open(tmp_src, "w") as f:
        f.write(code)
    os.replace(tmp_src, cpp_path)
    tmp_so = f"{so_path}.tmp{os.getpid()}"
    cmd = command(device, cpp_path, tmp_so)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        try:
            os.remove(tmp_so)
        except OSError:
            pass
        raise RuntimeError(f"Compilation failed:\n{res.stderr}")
    os.replace(tmp_so, so_path)
