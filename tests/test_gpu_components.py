"""Component entry points on the GPU: the per-shape run_transpose_* /
run_batched_matmul / run_einsum symbols (test_matmul.py:24-147 of the
reference) and the core permutation launcher on the reference's transpose
matrix (test_transpose.py:108-161), all through the C ABI."""
import ctypes
import itertools

import numpy as np
import pytest
import torch

import oracle
from parity_util import check
from pto_einsum import EinsumBuilder, abi, launch, runtime
from test_launch import EXTRA
from test_oracle import TRANSPOSE_CASES

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", [("ij,jk->ik", (32, 64), (64, 128)),
                                      ("bji,bjk->bik", (3, 37, 50), (3, 37, 41)),
                                      ("bshd,bthd->bsht", (2, 24, 3, 16), (2, 20, 3, 16)),
                                      ("ij,jk->ki", (33, 20), (20, 47))])
def test_staged_components(eq, s0, s1, dtype, build_dir):
    builder = EinsumBuilder(eq, [s0, s1], dtype)
    builder.build()
    lib = builder.lib
    r = builder.recipe
    g = torch.Generator().manual_seed(1)
    x, y = torch.rand(s0, generator=g).to(dtype), torch.rand(s1, generator=g).to(dtype)
    if builder._swap_operands:
        x, y = y, x
    p0, p1 = r["in_transpose_idxs"]
    t0 = torch.empty([x.shape[i] for i in p0], dtype=dtype, device="cuda")
    t1 = torch.empty([y.shape[i] for i in p1], dtype=dtype, device="cuda")
    xc, yc = x.cuda(), y.cuda()
    assert lib.run_transpose_inp0(ctypes.cast(_ptr(xc), ctypes.POINTER(builder.c_type)),
                                  ctypes.cast(_ptr(t0), ctypes.POINTER(builder.c_type)), _stream()) == 0
    assert lib.run_transpose_inp1(ctypes.cast(_ptr(yc), ctypes.POINTER(builder.c_type)),
                                  ctypes.cast(_ptr(t1), ctypes.POINTER(builder.c_type)), _stream()) == 0
    assert torch.equal(t0.cpu(), x.permute(p0).contiguous())
    assert torch.equal(t1.cpu(), y.permute(p1).contiguous())
    I, L0, L1, C = r["I"], r["L0"], r["L1"], r["C"]
    res = torch.empty(I * L0 * L1, dtype=torch.float32, device="cuda")
    rc = lib.run_batched_matmul(ctypes.cast(_ptr(t0), ctypes.POINTER(builder.c_type)),
                                ctypes.cast(_ptr(t1), ctypes.POINTER(builder.c_type)),
                                ctypes.cast(_ptr(res), ctypes.POINTER(ctypes.c_float)), _stream())
    assert rc == 0
    want = oracle.bmm(t0.float().cpu().numpy().reshape(I, L0, C), t1.float().cpu().numpy().reshape(I, C, L1))
    check(res.cpu().numpy().reshape(I, L0, L1), want, False, 1e-4 if dtype == torch.float32 else 2e-3, "bmm")
    out = torch.empty(r["out_shape"], dtype=torch.float32, device="cuda")
    rc = lib.run_transpose_out(ctypes.cast(_ptr(res), ctypes.POINTER(ctypes.c_float)),
                               ctypes.cast(_ptr(out), ctypes.POINTER(ctypes.c_float)), _stream())
    assert rc == 0
    assert torch.equal(out.cpu(), res.cpu().reshape(r["out_interpret_shape"]).permute(r["out_transpose_idxs"]))
    # One-shot entry point (setup + exec + sync + teardown).
    out2 = torch.empty(r["out_shape"], dtype=torch.float32, device="cuda")
    assert lib.run_einsum(ctypes.cast(_ptr(xc), ctypes.POINTER(builder.c_type)),
                          ctypes.cast(_ptr(yc), ctypes.POINTER(builder.c_type)),
                          ctypes.cast(_ptr(out2), ctypes.POINTER(ctypes.c_float)), _stream()) == 0
    user0, user1 = (y, x) if builder._swap_operands else (x, y)
    want_full = oracle.einsum(eq, user0.float().numpy(), user1.float().numpy())
    check(out2.cpu().numpy(), want_full, False, 1e-4 if dtype == torch.float32 else 2e-3, "run_einsum")
    builder.cleanup()


def _permute_gpu(x: torch.Tensor, perm):
    lib = abi.bind()
    d = abi.permute_desc(launch._permute_desc(tuple(x.shape), perm, x.element_size()))
    xc = x.cuda()
    out = torch.empty([x.shape[p] for p in perm], dtype=x.dtype, device="cuda")
    rc = lib.pe_permute(ctypes.byref(d), _ptr(xc), _ptr(out), _stream())
    assert rc == 0, runtime.last_error()
    return out.cpu()


ND = [((2, 3, 4, 5), p) for p in itertools.permutations(range(4))] + [
    ((64, 3, 130), (2, 1, 0)), ((7, 65, 66, 3), (0, 2, 1, 3)), ((5, 129, 2, 67), (3, 1, 2, 0)),
    ((1, 1, 1), (2, 0, 1)), ((4096, 33), (1, 0))]


@pytest.mark.parametrize("shape,perm,dt", TRANSPOSE_CASES + [(s, p, np.float32) for s, p in ND]
                         + [(s, p, np.float16) for s, p in ND[-5:]])
def test_permute_bit_exact(shape, perm, dt):
    x = torch.from_numpy(np.random.default_rng(42).random(shape).astype(dt))
    got = _permute_gpu(x, perm)
    assert torch.equal(got.view(torch.int16 if dt == np.float16 else torch.int32),
                       x.permute(perm).contiguous().view(torch.int16 if dt == np.float16 else torch.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", EXTRA)
def test_staged_plans_on_gpu(eq, s0, s1, dtype, build_dir):
    """Equations whose axis groups force operand gathers / an output
    permutation through the workspace."""
    from parity_util import RTOL, contraction_size, make_inputs
    from pto_einsum import einsum

    a, b = make_inputs(eq, s0, s1, dtype)
    got = einsum(eq, a.cuda(), b.cuda()).cpu().numpy()
    want = oracle.einsum(eq, a.float().numpy(), b.float().numpy())
    check(got, want, contraction_size(eq, s0, s1) <= 1, RTOL[dtype], eq)
