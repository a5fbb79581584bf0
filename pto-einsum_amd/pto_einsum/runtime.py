"""Loading of the gfx950 core library and HIP stream plumbing.

The core library (``lib/libpto_einsum_hip.so``) holds every device kernel and
is built once by ``python -m pto_einsum.build`` (or the repository's build
entry).  It is loaded with RTLD_GLOBAL after torch, so it binds to the HIP
runtime torch already loaded (both carry the soname libamdhip64.so.7) and the
per-shape libraries resolve their ``pe_*`` calls against it.  There is no
fallback: a GPU call without the built library raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
_lock = threading.Lock()
_core = None


def include_dir() -> str:
    """Headers the per-shape sources compile against: the package copy when
    installed, else the repository's ``include/``."""
    local = os.path.join(PKG_DIR, "include")
    if os.path.isfile(os.path.join(local, "pto_einsum_hip.h")):
        return local
    return os.path.abspath(os.path.join(PKG_DIR, "..", "..", "include"))


def core_library_path() -> str:
    return os.path.join(PKG_DIR, "lib", "libpto_einsum_hip.so")


_id_cache = {}


def core_library_id() -> str:
    """Content hash of the built core library, folded into the JIT cache key."""
    p = core_library_path()
    if not os.path.exists(p):
        return "missing"
    st = os.stat(p)
    stamp = (st.st_size, st.st_mtime_ns)
    if _id_cache.get("stamp") != stamp:
        with open(p, "rb") as f:
            _id_cache["id"] = hashlib.sha256(f.read()).hexdigest()[:16]
        _id_cache["stamp"] = stamp
    return _id_cache["id"]


def core():
    """The loaded core library (raises if it was never built)."""
    global _core
    with _lock:
        if _core is not None:
            return _core
        path = core_library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"pto_einsum: HIP core library not built ({path}); build it with "
                "`make -C pto-einsum_amd/csrc` or `python -c 'import __graft_entry__ as g; g.build()'`")
        import torch  # noqa: F401  (loads torch's HIP runtime first)

        lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        lib.pe_last_error.restype = ctypes.c_char_p
        lib.pe_last_error.argtypes = []
        lib.pe_version.restype = ctypes.c_char_p
        lib.pe_device_cu_count.restype = ctypes.c_int
        _core = lib
        return _core


def last_error() -> str:
    try:
        msg = core().pe_last_error()
        return msg.decode() if msg else ""
    except Exception:  # pragma: no cover
        return ""


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status}: {last_error()}")


def current_stream_ptr(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
