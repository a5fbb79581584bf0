"""Opt-in single-operand reduction axes on the GPU.

The reduction stage (pe_reduce_axes) is checked bit for bit against float32
loops on the CPU in its documented order, with the (V, L, C) the library
reports for each call (pe_reduce_order): the terms of an output, row-major
over the reduced index, form ceil(nterm / V) groups of V; the groups are cut
into C contiguous chunks (the first G % C one longer); lane l of L sums groups
l, l + L, ... of its chunk term by term from +0; lane sums, then chunk sums,
are combined by a pairwise tree.  Whole einsums are checked against float64
torch.einsum with the contraction tolerance (the reference has no result to
compare with: it rejects these equations)."""
import ctypes

import numpy as np
import pytest
import torch

from pto_einsum import abi, einsum, runtime
from solo_reduce_order import ordered_sum, reduce_desc

pytestmark = pytest.mark.gpu


def _order(x: torch.Tensor, axes):
    d = reduce_desc(x, axes)
    order = (ctypes.c_int64 * 3)()
    rc = abi.bind().pe_reduce_order(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), order)
    runtime.check(rc, "pe_reduce_order")
    return tuple(int(v) for v in order)


def _view(x: torch.Tensor, how: str) -> torch.Tensor:
    if how == "t":        # a transposed (non-contiguous) view of x's values
        return x.t().contiguous().cuda().t()
    if how == "off":      # x's values one element into a larger buffer (rows misaligned)
        big = torch.zeros(x.shape[0], x.shape[1] + 1, dtype=x.dtype)
        big[:, 1:] = x
        return big.cuda()[:, 1:]
    if how == "shift":    # x's values one element into a flat buffer (contiguous, base not 16-byte aligned)
        flat = torch.zeros(x.numel() + 1, dtype=x.dtype)
        flat[1:] = x.reshape(-1)
        return flat.cuda()[1:].reshape(x.shape)
    return x.cuda()


CASES = [
    # shape, reduced axes, view, expected mode: "row" (V*L > 1) or "col"
    ((5, 7, 9), (1,), "", "col"),
    ((5, 7, 9), (0, 2), "", "col"),              # two reduced runs: odometer
    ((6, 33), (1,), "t", "col"),
    ((4, 3), (), "", "col"),                     # conversion only
    ((3000, 333), (), "", "col"),                # conversion of a contiguous run (vector path)
    ((300, 5), (), "t", "col"),                  # conversion of a strided view
    ((3, 0, 2), (1,), "", None),                 # no terms: +0
    ((3, 70001), (1,), "", "row"),               # few outputs, chunked, partial last group
    ((2, 37, 300), (1, 2), "", "row"),           # two axes merging into one run
    ((300, 5), (0,), "t", "row"),
    ((40000, 300), (1,), "", "row"),
    ((5000, 300), (1,), "", "row"),              # more than 2048 outputs of more than 256 terms
    ((64, 1025), (1,), "off", "row"),            # misaligned rows: V = 1
    ((64, 100000), (1,), "", "row"),             # C > 1 with 64 outputs
    ((20000, 64), (0,), "", "col"),              # strided reduced axis, C > 1
    ((300, 8, 200), (0, 2), "", "col"),          # odometer chunks starting mid-run
    ((7, 20), (1,), "", "col"),                  # short runs go lane-per-output
    ((1000, 40), (1,), "", "row"),               # four lanes per output, 16 outputs per wave
    ((1000, 1000), (0, 1), "shift", "row"),      # whole sum from an unaligned base: more chunks
    ((5, 1, 257), (0, 1, 2), "shift", "row"),    # ... two chunks where an aligned base needs one
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("shape,axes,how,mode", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in CASES])
def test_reduce_axes_is_the_documented_sum(dtype, shape, axes, how, mode):
    from pto_einsum.builder import _reduce_operand

    g = torch.Generator().manual_seed(sum(shape) + len(axes))
    x = torch.randn(*shape, generator=g).to(dtype)
    subs = "abcde"[: len(shape)]
    xd = _view(x, how)
    V, L, C = _order(xd, axes)
    if mode == "row":
        # groups of 16 bytes when every output's run starts 16-byte aligned
        eb = x.element_size()
        keep_strides = [xd.stride(i) for i in range(xd.dim()) if i not in axes and xd.shape[i] > 1]
        al = xd.data_ptr() % 16 == 0 and all(s * eb % 16 == 0 for s in keep_strides)
        assert L in (4, 8, 16, 32, 64) and V == (16 // eb if al else 1)
    elif mode == "col":
        assert (V, L) == (1, 1)
    got = _reduce_operand(xd, subs, "".join(subs[i] for i in axes)).cpu().numpy()
    want = ordered_sum(x.float().numpy(), axes, V, L, C)
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    again = _reduce_operand(xd, subs, "".join(subs[i] for i in axes)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_chunked_orders_use_several_chunks():
    """The cases above reach the two-pass path (C > 1) in both modes."""
    x = torch.zeros(64, 100000, device="cuda")
    assert _order(x, (1,))[2] > 1
    y = torch.zeros(20000, 64, device="cuda")
    assert _order(y, (0,))[2] > 1


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
    def call(ws=None, ws_bytes=0):
        return lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                  ctypes.c_void_p(ws), ws_bytes, st)

    rc = call()
    assert rc == -2 and "past the source" in runtime.last_error()
    d.src_numel, d.reserved = 20, 1
    rc = call()
    assert rc == -1 and "reserved" in runtime.last_error()
    d.reserved, d.dtype = 0, 7
    rc = call()
    assert rc == -3
    # a chunked order without its workspace: refused before any launch
    big = torch.zeros(64, 100000, device="cuda")
    d = reduce_desc(big, (1,))
    need = int(lib.pe_reduce_workspace_bytes(ctypes.byref(d)))
    req = 64 * _order(big, (1,))[2] * 4           # this (aligned) source's chunk sums
    assert need >= req                            # the query covers any base address
    out = torch.empty(64, device="cuda")
    for ws, nb in ((None, 0), (out.data_ptr(), req - 4)):
        rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(big.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                ctypes.c_void_p(ws), nb, st)
        assert rc == -4 and "workspace" in runtime.last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_conversion_is_a_one_term_sum(dtype):
    """No reduced axis: every output is +0 + x (so -0 becomes +0), on the
    vector path (contiguous source, aligned destination) and on the
    lane-per-output path (an unaligned destination through the C ABI)."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1003, generator=g).to(dtype)
    x[::7] = -0.0
    x[1] = float("inf")
    want = (torch.zeros(1003) + x.float()).numpy()
    xd = x.cuda()
    d = reduce_desc(xd, ())
    lib = abi.bind()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    buf = torch.full((1003 + 4,), float("nan"), device="cuda")
    for off in (0, 1):  # dst 16-byte aligned, then 4 bytes past that
        dst = buf[off:off + 1003]
        rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                ctypes.c_void_p(None), 0, st)
        assert rc == 0, runtime.last_error()
        got = dst.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
