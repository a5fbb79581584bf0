"""The C ABI: the core library loads and exports every function
include/pto_einsum_hip.h declares; per-shape libraries export the reference's
ctypes symbol set (builder.py:761-815); the ctypes struct mirrors match the C
layout.  No compute calls (no GPU needed)."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from pto_einsum import EinsumBuilder, abi, runtime

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pto_einsum_hip.h")
PER_SHAPE = {"run_einsum", "run_einsum_setup", "run_einsum_exec", "run_einsum_teardown",
             "run_transpose_inp0", "run_transpose_inp1", "run_transpose_out", "run_batched_matmul"}


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:pe|run)_[a-z0-9_]+)\s*\(", text))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_core_exports_every_declared_function():
    decl = declared_functions()
    core = decl - PER_SHAPE
    assert {"pe_product", "pe_permute", "pe_gemm", "pe_einsum_exec", "pe_einsum_setup"} <= core
    missing = core - exported(runtime.core_library_path())
    assert not missing, f"core library lacks {missing}"
    lib = runtime.core()
    for name in core:
        getattr(lib, name)
    assert b"gfx950" in lib.pe_version()


@pytest.mark.parametrize("eq,s0,s1,expect", [
    ("bji,bjk->bik", (2, 7, 10), (2, 7, 15), PER_SHAPE),
    ("ts,ts->ts", (8, 16), (8, 16), {"run_einsum", "run_einsum_setup", "run_einsum_exec", "run_einsum_teardown"}),
    ("bsd,d->bsd", (2, 8, 16), (16,), {"run_einsum", "run_einsum_setup", "run_einsum_exec", "run_einsum_teardown"}),
])
def test_per_shape_library_symbols(eq, s0, s1, expect, tmp_path, monkeypatch):
    monkeypatch.setenv("EINSUM_BUILD_DIR", str(tmp_path))
    b = EinsumBuilder(eq, [s0, s1], torch.float16)
    b.build()
    syms = exported(b.so_filename)
    assert expect <= syms
    assert not (PER_SHAPE - expect) & syms
    assert declared_functions() >= PER_SHAPE
    assert os.path.exists(b.cpp_filename) and b.target_dir.startswith(str(tmp_path))
    b.cleanup()
    assert not os.path.exists(b.target_dir)


def test_cache_reuses_library(tmp_path, monkeypatch):
    monkeypatch.setenv("EINSUM_BUILD_DIR", str(tmp_path))
    b1 = EinsumBuilder("ij,jk->ik", [(4, 5), (5, 6)], torch.float32)
    b1.build()
    mtime = os.path.getmtime(b1.so_filename)
    b2 = EinsumBuilder("ij,jk->ik", [(4, 5), (5, 6)], torch.float32)
    b2.build()
    assert b2.so_filename == b1.so_filename and os.path.getmtime(b2.so_filename) == mtime
    monkeypatch.setenv("EINSUM_EXTRA_DEFINES", "-DPE_TAG=1")
    b3 = EinsumBuilder("ij,jk->ik", [(4, 5), (5, 6)], torch.float32)
    b3.build()
    assert b3.so_filename != b1.so_filename


def test_compile_failure_raises(tmp_path, monkeypatch):
    monkeypatch.setenv("EINSUM_BUILD_DIR", str(tmp_path))
    monkeypatch.setenv("EINSUM_EXTRA_DEFINES", "-DPE_BROKEN=1 -include /nonexistent/header.h")
    b = EinsumBuilder("ij,jk->ik", [(4, 5), (5, 6)], torch.float32)
    with pytest.raises(RuntimeError, match="Compilation failed"):
        b.build()


STRUCT_PROBE = r"""
#include <cstddef>
#include <cstdio>
#include "pto_einsum_hip.h"
#define OFF(T, f) printf(#T "." #f " %zu\n", offsetof(T, f))
int main() {
  printf("pe_product_desc %zu\npe_permute_desc %zu\npe_gemm_desc %zu\npe_einsum_plan %zu\npe_linattn_desc %zu\n",
         sizeof(pe_product_desc), sizeof(pe_permute_desc), sizeof(pe_gemm_desc), sizeof(pe_einsum_plan),
         sizeof(pe_linattn_desc));
  OFF(pe_linattn_desc, m_numel); OFF(pe_linattn_desc, precise);
  OFF(pe_product_desc, b_numel); OFF(pe_permute_desc, src_numel); OFF(pe_gemm_desc, M);
  OFF(pe_gemm_desc, c_numel); OFF(pe_einsum_plan, gemm); OFF(pe_einsum_plan, ws_bytes);
  OFF(pe_einsum_plan, skip_phases);
  printf("pe_reduce_desc %zu\n", sizeof(pe_reduce_desc));
  OFF(pe_reduce_desc, red_stride); OFF(pe_reduce_desc, src_numel);
  return 0;
}
"""


def test_ctypes_struct_layout_matches_c(tmp_path):
    src = tmp_path / "probe.cpp"
    src.write_text(STRUCT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-std=c++17", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    vals = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                  check=True).stdout.splitlines())
    assert int(vals["pe_product_desc"]) == ctypes.sizeof(abi.ProductDesc)
    assert int(vals["pe_permute_desc"]) == ctypes.sizeof(abi.PermuteDesc)
    assert int(vals["pe_gemm_desc"]) == ctypes.sizeof(abi.GemmDesc)
    assert int(vals["pe_einsum_plan"]) == ctypes.sizeof(abi.EinsumPlan)
    assert int(vals["pe_product_desc.b_numel"]) == abi.ProductDesc.b_numel.offset
    assert int(vals["pe_permute_desc.src_numel"]) == abi.PermuteDesc.src_numel.offset
    assert int(vals["pe_gemm_desc.M"]) == abi.GemmDesc.M.offset
    assert int(vals["pe_gemm_desc.c_numel"]) == abi.GemmDesc.c_numel.offset
    assert int(vals["pe_einsum_plan.gemm"]) == abi.EinsumPlan.gemm.offset
    assert int(vals["pe_einsum_plan.ws_bytes"]) == abi.EinsumPlan.ws_bytes.offset
    assert int(vals["pe_einsum_plan.skip_phases"]) == abi.EinsumPlan.skip_phases.offset
    assert int(vals["pe_linattn_desc"]) == ctypes.sizeof(abi.LinAttnDesc)
    assert int(vals["pe_linattn_desc.m_numel"]) == abi.LinAttnDesc.m_numel.offset
    assert int(vals["pe_linattn_desc.precise"]) == abi.LinAttnDesc.precise.offset
    assert int(vals["pe_reduce_desc"]) == ctypes.sizeof(abi.ReduceDesc)
    assert int(vals["pe_reduce_desc.red_stride"]) == abi.ReduceDesc.red_stride.offset
    assert int(vals["pe_reduce_desc.src_numel"]) == abi.ReduceDesc.src_numel.offset


def test_descriptor_validation_rejects_out_of_bounds():
    """Host-side checks refuse descriptors that would address past an
    operand, before anything is launched (null pointers, no GPU touched)."""
    lib = abi.bind()
    d = abi.GemmDesc()
    d.dtype, d.M, d.N, d.K = 0, 4, 4, 4
    d.a_ms, d.a_ks, d.b_ks, d.b_ns, d.c_ms, d.c_ns = 4, 1, 4, 1, 4, 1
    d.a_numel, d.b_numel, d.c_numel = 15, 16, 16   # A is one element short
    assert lib.pe_gemm(ctypes.byref(d), None, None, None, None, 0, None) == -2
    assert b"operand 0" in lib.pe_last_error()
    p = abi.PermuteDesc()
    p.elem_bytes, p.ndims, p.src_numel = 4, 2, 11
    p.shape[0], p.shape[1], p.src_stride[0], p.src_stride[1] = 3, 4, 1, 3
    assert lib.pe_permute(ctypes.byref(p), None, None, None) == -2
    q = abi.ProductDesc()
    q.dtype, q.ndims, q.a_numel, q.b_numel = 3, 0, 1, 1
    assert lib.pe_product(ctypes.byref(q), None, None, None, None) == -3


def test_noalloc_rejects_oversized_plan_without_launch():
    """The allocation-free executor refuses a plan whose workspace exceeds its
    static scratch, before any device call (so this runs without a GPU)."""
    lib = abi.bind()
    b = EinsumBuilder("abc,cd->adb", [(1024, 8, 64), (64, 4096)], torch.float32)
    b.parse_equation()
    b.generate_code()
    assert b.launch_plan.scatter_out and b.launch_plan.ws_bytes > (64 << 20)
    plan = abi.einsum_plan(b.launch_plan)
    assert lib.pe_einsum_exec_noalloc(ctypes.byref(plan), None, None, None, None) == -4
    assert b"scratch limit" in lib.pe_last_error()


@pytest.mark.parametrize("stop,skip", [(None, 0), (3, 0), (2, 4), (1, 6), (0, 7)])
def test_phase_stop_define_reaches_the_plan(stop, skip, tmp_path):
    """EINSUM_PHASE_STOP (passed through EINSUM_EXTRA_DEFINES, as in the
    reference's builder.py:688-697) sets the plan's skip_phases in the
    per-shape source: the phases after the N-th are skipped."""
    b = EinsumBuilder("acb,cd->abd", [(48, 64, 6), (64, 72)], torch.float32)
    b.parse_equation()
    b.generate_code()
    assert "#define EINSUM_PHASE_STOP 3" in b.cpp_code
    src = tmp_path / "probe.cpp"
    src.write_text(b.cpp_code + '\n#include <cstdio>\nint main() { printf("%d\\n", kPlan.skip_phases); return 0; }\n')
    exe = tmp_path / "probe"
    libdir = os.path.dirname(runtime.core_library_path())
    cmd = ["g++", "-std=c++17", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe),
           "-L", libdir, "-lpto_einsum_hip", "-Wl,-rpath," + libdir]
    if stop is not None:
        cmd.insert(1, f"-DEINSUM_PHASE_STOP={stop}")
    subprocess.run(cmd, check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    assert int(out) == skip


@pytest.mark.parametrize("eq,s0,s1", [("ij,jk->ik", (0, 5), (5, 7)), ("ij,jk->ik", (5, 5), (5, 0)),
                                      ("bij,bjk->bik", (0, 3, 4), (0, 4, 5)), ("ij,jk->ki", (0, 4096), (4096, 16)),
                                      ("abc,cd->adb", (0, 6, 96), (96, 80)), ("he,ew->wh", (5, 0), (0, 0))])
def test_empty_outputs_plan_without_dividing_by_zero(eq, s0, s1):
    """Shapes with a zero extent plan and size their workspace (host code
    only; an integer division by the zero tile count would end the process)."""
    b = EinsumBuilder(eq, [s0, s1], torch.float32)
    b.parse_equation()
    b.generate_code()
    lib = abi.bind()
    assert lib.pe_einsum_workspace_bytes(ctypes.byref(abi.einsum_plan(b.launch_plan))) >= 0
    if b.launch_plan.route == 1:
        assert lib.pe_gemm_workspace_bytes(ctypes.byref(abi.einsum_plan(b.launch_plan).gemm)) == 0


def test_empty_reductions_and_chains_size_without_dividing_by_zero():
    from solo_reduce_order import reduce_desc

    lib = abi.bind()
    for shape, axes in (((0, 17, 5), (2,)), ((0, 3000), (1,)), ((17, 0, 5), (2,)), ((5, 0), ())):
        x = torch.zeros(shape)
        d = reduce_desc(x, axes)
        order = (ctypes.c_int64 * 3)()
        assert lib.pe_reduce_workspace_bytes(ctypes.byref(d)) == 0
        assert lib.pe_reduce_order(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), order) == 0
    for T, S, N, P in ((0, 64, 16, 16), (64, 64, 16, 0), (0, 0, 16, 16), (64, 0, 16, 16), (64, 64, 0, 16)):
        d = abi.LinAttnDesc()
        d.qk_dtype = d.v_dtype = d.m_dtype = 0
        d.T, d.S, d.N, d.P = T, S, N, P
        d.q_ts, d.k_ss, d.v_ss, d.m_ts = N, N, P, S
        d.q_numel, d.k_numel, d.v_numel, d.m_numel = max(1, T * N), max(1, S * N), max(1, S * P), max(1, T * S)
        assert lib.pe_linear_attention_workspace_bytes(ctypes.byref(d)) == 0
