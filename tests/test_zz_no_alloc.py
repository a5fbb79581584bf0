"""Allocation-free executor (pe_einsum_exec_noalloc) through the C ABI.

It runs the same kernels as pe_einsum_exec with the workspace from
pe_einsum_setup, so results must be bit-identical to that entry point's.
Each case calls the allocation-free entry point twice in a row, the second
time with a smaller input, and checks both calls (the scratch array keeps
the first call's contents, which the second call must not depend on)."""
import ctypes

import pytest
import torch

from pto_einsum import EinsumBuilder, abi, runtime

pytestmark = pytest.mark.gpu

# (equation, dtype, large shapes, smaller shapes); each large plan uses the
# workspace (split-K partials, operand gathers or a staged result) except the
# product route, which needs none.
CASES = [
    ("ts,sp->tp", torch.float32, ((1024, 4096), (4096, 128)), ((256, 2048), (2048, 64))),
    ("tn,sn->ts", torch.float16, ((512, 8192), (256, 8192)), ((128, 1024), (96, 1024))),
    ("abc,cd->adb", torch.float32, ((64, 6, 96), (96, 80)), ((16, 3, 40), (40, 30))),
    ("abc,cd->adb", torch.float16, ((40, 9, 70), (70, 50)), ((9, 10, 11), (11, 12))),
    ("acb,cd->abd", torch.float32, ((48, 64, 6), (64, 72)), ((5, 7, 6), (7, 9))),
    ("bji,bjk->bik", torch.float32, ((4, 300, 200), (4, 300, 260)), ((2, 37, 50), (2, 37, 41))),
    ("bsd,d->bsd", torch.float16, ((4, 256, 512), (512,)), ((2, 16, 64), (64,))),
]


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _plan(eq, shapes, dtype):
    b = EinsumBuilder(eq, list(shapes), dtype)
    b.parse_equation()
    b.generate_code()
    return b, abi.einsum_plan(b.launch_plan)


def _inputs(shapes, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g).to(dtype).cuda() for s in shapes]


def _run(lib, builder, plan, x, y, noalloc):
    if builder._swap_operands:
        x, y = y, x
    out = torch.full(builder.recipe["out_shape"], float("nan"), dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.pe_einsum_exec_noalloc(ctypes.byref(plan), _ptr(x), _ptr(y), _ptr(out), stream)
        assert rc == 0, runtime.last_error()
        return out, None
    ws = lib.pe_einsum_setup(ctypes.byref(plan), stream)
    assert ws, runtime.last_error()
    rc = lib.pe_einsum_exec(ctypes.byref(plan), _ptr(x), _ptr(y), _ptr(out), ctypes.c_void_p(ws), stream)
    assert rc == 0, runtime.last_error()
    return out, ws


@pytest.mark.parametrize("eq,dtype,big,small", CASES,
                         ids=[f"{c[0]}-{str(c[1])[6:]}-{i}" for i, c in enumerate(CASES)])
def test_noalloc_matches_exec(eq, dtype, big, small):
    lib = abi.bind()
    bb, pbig = _plan(eq, big, dtype)
    bs, psmall = _plan(eq, small, dtype)
    if eq != "bsd,d->bsd":
        lp = bb.launch_plan
        assert lp.gather0 or lp.gather1 or lp.scatter_out or lib.pe_gemm_workspace_bytes(ctypes.byref(pbig.gemm)) > 0
    xb, yb = _inputs(big, dtype, 1)
    xs, ys = _inputs(small, dtype, 2)
    print(f"noalloc: {eq} {dtype} {big} then {small}", flush=True)
    # Two allocation-free calls in a row, the second with the smaller input.
    got_big, _ = _run(lib, bb, pbig, xb, yb, True)
    got_small, _ = _run(lib, bs, psmall, xs, ys, True)
    torch.cuda.synchronize()
    want_big, ws_big = _run(lib, bb, pbig, xb, yb, False)
    want_small, ws_small = _run(lib, bs, psmall, xs, ys, False)
    torch.cuda.synchronize()
    assert lib.pe_einsum_teardown(ctypes.c_void_p(ws_big)) == 0
    assert lib.pe_einsum_teardown(ctypes.c_void_p(ws_small)) == 0
    assert torch.equal(got_big, want_big)
    assert torch.equal(got_small, want_small)
    # And the large plan again after the small one overwrote the scratch.
    again, _ = _run(lib, bb, pbig, xb, yb, True)
    torch.cuda.synchronize()
    assert torch.equal(again, want_big)


def test_noalloc_rejects_oversized_plan():
    lib = abi.bind()
    # A staged output of 128 MiB: above the scratch limit.
    b, plan = _plan("abc,cd->adb", ((1024, 8, 64), (64, 4096)), torch.float32)
    assert b.launch_plan.scatter_out
    x = torch.zeros(1, device="cuda")
    rc = lib.pe_einsum_exec_noalloc(ctypes.byref(plan), _ptr(x), _ptr(x), _ptr(x),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == -4
    assert "scratch limit" in runtime.last_error()
