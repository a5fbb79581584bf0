"""Opt-in single-operand reduction axes on the GPU.

The reduction stage (pe_reduce_axes) is checked bit for bit against float32
loops on the CPU in its documented order: the terms of an output, row-major
over the reduced index, cut into C contiguous chunks (the first nterm % C one
term longer), each chunk summed from +0 and the partial sums added in chunk
order from +0; C = 1 when nterm <= 256 or there are at least 32768 outputs,
else min(256, ceil(nterm / 256)).  Whole einsums are checked against float64
torch.einsum with the contraction tolerance (the reference has no result to
compare with: it rejects these equations)."""
import ctypes

import numpy as np
import pytest
import torch

from pto_einsum import abi, einsum, runtime

pytestmark = pytest.mark.gpu

CHUNK_TERMS, WIDE_OUTPUTS, CHUNK_THREADS = 256, 32768, 256


def _ordered_sum(x: np.ndarray, axes):
    """float32 sum over `axes` in the chunked order above, the other axes
    kept in order.  Each loop step adds one term to every output at once, so
    the per-output order is sequential."""
    keep = [i for i in range(x.ndim) if i not in axes]
    xt = np.transpose(x, keep + list(axes)).astype(np.float32)
    nout = int(np.prod([x.shape[i] for i in keep], dtype=np.int64))
    flat = xt.reshape(nout, -1)
    nterm = flat.shape[1]
    nchunk = 1 if nterm <= CHUNK_TERMS or nout >= WIDE_OUTPUTS else min(CHUNK_THREADS, -(-nterm // CHUNK_TERMS))
    q, r = divmod(nterm, nchunk)
    total = np.zeros(nout, dtype=np.float32)
    t = 0
    for c in range(nchunk):
        acc = np.zeros(nout, dtype=np.float32)
        for _ in range(q + (1 if c < r else 0)):
            acc = acc + flat[:, t]
            t += 1
        total = total + acc
    assert t == nterm
    return total.reshape([x.shape[i] for i in keep])


def test_ordered_sum_restates_the_plain_loop_for_one_chunk():
    """The checker itself: with one chunk it is the scalar sequential loop."""
    x = np.random.default_rng(1).standard_normal((3, 200)).astype(np.float32)
    want = np.zeros(3, dtype=np.float32)
    for i in range(3):
        acc = np.float32(0.0)
        for v in x[i]:
            acc = np.float32(acc + v)
        want[i] = acc
    assert np.array_equal(_ordered_sum(x, (1,)).view(np.uint32), want.view(np.uint32))
    # more chunks: the same total to rounding, a different (chunked) order
    y = np.random.default_rng(2).standard_normal((2, 5000)).astype(np.float32)
    assert np.allclose(_ordered_sum(y, (1,)), y.astype(np.float64).sum(1), rtol=0, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("shape,axes,transpose", [((5, 7, 9), (1,), False), ((5, 7, 9), (0, 2), False),
                                                  ((6, 33), (1,), True), ((4, 3), (), False),
                                                  ((3, 0, 2), (1,), False),
                                                  ((3, 70001), (1,), False), ((2, 37, 300), (1, 2), False),
                                                  ((300, 5), (0,), True), ((40000, 300), (1,), False)])
def test_reduce_axes_is_the_sequential_sum(dtype, shape, axes, transpose):
    from pto_einsum.builder import _reduce_operand

    g = torch.Generator().manual_seed(sum(shape) + len(axes))
    x = torch.randn(*shape, generator=g).to(dtype)
    subs = "abcde"[: len(shape)]
    xd = x.cuda()
    if transpose:  # a non-contiguous view
        xd = x.t().contiguous().cuda().t()
    got = _reduce_operand(xd, subs, "".join(subs[i] for i in axes)).cpu().numpy()
    want = _ordered_sum(x.float().numpy(), axes)
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


EQS = [
    ("ij,jk->k", (300, 70), (70, 90)),
    ("ij,jk->i", (300, 70), (70, 90)),
    ("ij,k->k", (30, 40), (50,)),
    ("ijx,jky->ik", (20, 30, 40), (30, 50, 6)),
    ("bij,bjk->bk", (4, 60, 70), (4, 70, 80)),
    ("abc,cd->ad", (20, 30, 40), (40, 50)),
    ("i,j->", (300,), (400,)),
    ("ij,jk->k", (70000, 8), (8, 40)),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", EQS)
def test_einsum_with_solo_axes(eq, s0, s1, dtype):
    g = torch.Generator().manual_seed(len(eq) * 31 + sum(s0))
    a = torch.randn(*s0, generator=g).to(dtype)
    b = torch.randn(*s1, generator=g).to(dtype)
    got = einsum(eq, a.cuda(), b.cuda(), reduce_solo_axes=True)
    assert got.dtype == torch.float32
    want = torch.einsum(eq, a.double(), b.double())
    # float32 sums over at most a few thousand terms of |a||b| products
    bound = torch.einsum(eq, a.double().abs(), b.double().abs())
    err = (got.cpu().double() - want).abs()
    assert got.shape == want.shape
    assert bool((err <= 1e-5 * bound + 1e-6).all()), float((err - 1e-5 * bound).max())
    again = einsum(eq, a.cuda(), b.cuda(), reduce_solo_axes=True)
    assert torch.equal(got, again)  # deterministic


def test_solo_axes_on_non_contiguous_and_empty_operands():
    g = torch.Generator().manual_seed(5)
    a = torch.randn(70, 300, generator=g).cuda().t()        # [300, 70] view
    b = torch.randn(70, 90, generator=g).cuda()
    got = einsum("ij,jk->k", a, b, reduce_solo_axes=True)
    want = torch.einsum("ij,jk->k", a.double(), b.double())
    assert torch.allclose(got.double(), want, rtol=1e-4, atol=1e-4)
    z = torch.zeros(0, 70, device="cuda")                  # the solo axis has no terms
    got = einsum("ij,jk->k", z, b, reduce_solo_axes=True)
    assert torch.equal(got.cpu(), torch.zeros(90))


def test_reduce_axes_validation():
    lib = abi.bind()
    d = abi.ReduceDesc()
    d.dtype, d.nkeep, d.nred = 0, 1, 1
    d.keep_shape[0], d.keep_stride[0], d.red_shape[0], d.red_stride[0] = 4, 1, 5, 4
    d.src_numel = 19  # one short of the 20 elements addressed
    x = torch.zeros(20, device="cuda")
    out = torch.empty(4, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), st)
    assert rc == -2 and "past the source" in runtime.last_error()
    d.src_numel, d.reserved = 20, 1
    rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), st)
    assert rc == -1 and "reserved" in runtime.last_error()
    d.reserved, d.dtype = 0, 7
    rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), st)
    assert rc == -3
