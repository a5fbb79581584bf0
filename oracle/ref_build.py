"""Build the reference's own CPU einsum (test infrastructure only).

Compiles ``/root/reference/src/pto_einsum/include/cpu_einsum.h`` -- the
reference CPU route's whole arithmetic, a self-contained C++17 header that
includes only ``<vector>`` -- for each case in ``oracle/ref_cases.py``.

For every case this writes, into ``oracle/_ref/`` only:

* ``ref_<key>.cpp`` -- the config structs ``cpu_einsum.h`` documents at its
  top (cpu_einsum.h:8-31) filled with the case's recipe, in the field layout
  of templates.py:1-19,64-67, plus the ``extern "C" run_einsum`` wrapper of
  templates.py:131-156;
* ``ref_<key>.so``  -- that file compiled exactly as the reference compiles
  its CPU route: ``g++ -O3 -shared -fPIC -std=c++17 -I <include>``
  (builder.py:705-709).

No reference file is copied; the header is included from where it lies.
``/root/reference`` is absent on the GPU machine, so the built ``.so`` files
travel there with the working tree (``oracle/_ref/`` is kept out of version
control only).  Run: ``python oracle/ref_build.py [-j N]``.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from math import prod

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(ORACLE_DIR, "_ref")
REF_INCLUDE = "/root/reference/src/pto_einsum/include"
sys.path.insert(0, ORACLE_DIR)

import oracle  # noqa: E402
from ref_cases import BENCH_CONFIG_CASES, REF_CASES  # noqa: E402


def case_key(eq, shape0, shape1):
    text = json.dumps([eq.replace(" ", ""), list(shape0), list(shape1)])
    return hashlib.sha1(text.encode()).hexdigest()[:16]


def so_path(eq, shape0, shape1):
    return os.path.join(REF_DIR, f"ref_{case_key(eq, shape0, shape1)}.so")


def available() -> bool:
    return os.path.isdir(REF_INCLUDE)


def _tconfig(name, shape, perm):
    shape = [int(s) for s in shape]
    st = oracle._strides(shape)
    to_shape = [shape[p] for p in perm]
    pst = [st[p] for p in perm]
    dims = len(shape)
    j = lambda xs: ", ".join(str(x) for x in xs)  # noqa: E731
    return (f"struct {name} {{\n"
            f"    static constexpr unsigned dims = {dims};\n"
            f"    static constexpr unsigned N = {prod(shape)};\n"
            f"    static constexpr unsigned from_shape[{dims}] = {{{j(shape)}}};\n"
            f"    static constexpr unsigned to_shape[{dims}] = {{{j(to_shape)}}};\n"
            f"    static constexpr unsigned perm[{dims}] = {{{j(perm)}}};\n"
            f"    static constexpr unsigned perm_strides[{dims}] = {{{j(pst)}}};\n"
            f"}};\n")


def source(eq, shape0, shape1):
    r, swapped = oracle.cpu_plan(eq, shape0, shape1)
    if r["kind"] == "hadamard":
        n = prod(r["out_shape"])
        return ('#include "cpu_einsum.h"\n\n'
                f"struct config_elementwise {{\n    static const unsigned N = {n};\n}};\n\n"
                'extern "C" void run_einsum(const float* input0, const float* input1, '
                "float* output, void* stream) {\n"
                "    cpu::elementwise_mul<float, config_elementwise>(input0, input1, output);\n}\n")
    s0, s1 = (shape1, shape0) if swapped else (shape0, shape1)
    parts = ['#include "cpu_einsum.h"\n',
             _tconfig("config_tpose_inp0", s0, r["perm0"]),
             _tconfig("config_tpose_inp1", s1, r["perm1"]),
             _tconfig("config_tpose_out", r["mid_shape"], r["out_perm"]),
             "struct config_einsum {\n"
             "    typedef config_tpose_inp0 tpose_inp0_config;\n"
             "    typedef config_tpose_inp1 tpose_inp1_config;\n"
             "    typedef config_tpose_out tpose_out_conf;\n"
             f"    static const unsigned n_free0 = {r['L0']};\n"
             f"    static const unsigned n_free1 = {r['L1']};\n"
             f"    static const unsigned n_contract = {r['C']};\n"
             f"    static const unsigned n_inplace = {r['I']};\n"
             "};\n",
             'extern "C" void run_einsum(const float* input0, const float* input1, '
             "float* output, void* stream) {\n"
             "    cpu::einsum<float, config_einsum>(input0, input1, output);\n}\n"]
    return "\n".join(parts)


def build_case(eq, shape0, shape1):
    key = case_key(eq, shape0, shape1)
    cpp = os.path.join(REF_DIR, f"ref_{key}.cpp")
    so = os.path.join(REF_DIR, f"ref_{key}.so")
    if os.path.exists(so):
        return so
    with open(cpp, "w") as f:
        f.write(source(eq, shape0, shape1))
    tmp = so + f".tmp{os.getpid()}"
    res = subprocess.run(["g++", "-O3", "-shared", "-fPIC", "-std=c++17", "-I", REF_INCLUDE,
                          cpp, "-o", tmp], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"reference CPU build failed for {eq} {shape0} {shape1}:\n{res.stderr}")
    os.replace(tmp, so)
    return so


def build_all(jobs=8, cases=None):
    if not available():
        print(f"ref_build: {REF_INCLUDE} not present; oracle/_ref not built")
        return []
    if cases is None:
        cases = list(dict.fromkeys(tuple(c) for c in REF_CASES + BENCH_CONFIG_CASES))
    os.makedirs(REF_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(lambda c: build_case(*c), cases))


_loaded = {}


def run(eq, a, b):
    """Run the prebuilt reference CPU einsum for ``eq`` on float32 arrays.

    Feeds the operands as the reference runner does (builder.py:846-875):
    contiguous, swapped when the planner swapped them, into a zeroed float32
    output.  Raises FileNotFoundError when the case was not built.
    """
    import ctypes

    import numpy as np

    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    b = np.ascontiguousarray(np.asarray(b, dtype=np.float32))
    path = so_path(eq, a.shape, b.shape)
    if not os.path.exists(path):
        raise FileNotFoundError(path)
    if path not in _loaded:
        L = ctypes.CDLL(path)
        L.run_einsum.argtypes = [ctypes.c_void_p] * 4
        L.run_einsum.restype = None
        _loaded[path] = L
    r, swapped = oracle.cpu_plan(eq, a.shape, b.shape)
    if swapped:
        a, b = b, a
    out = np.zeros(r["out_shape"], dtype=np.float32)
    _loaded[path].run_einsum(a.ctypes.data, b.ctypes.data, out.ctypes.data, None)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    args = ap.parse_args()
    built = build_all(args.j)
    print(f"ref_build: {len(built)} reference CPU builds in {REF_DIR}")


if __name__ == "__main__":
    main()
