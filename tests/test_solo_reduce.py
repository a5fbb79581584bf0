"""Single-operand reduction axes (opt-in ``einsum(..., reduce_solo_axes=True)``).

The reference rejects an index found in one operand only and not in the output
(builder.py:218-229, tests/test_einsum.py:188-192); the build keeps that
default and, on request, sums such axes out of their operand first (the
reduction stage of IMPLEMENTATION.md:812-821).  These CPU tests pin the
equation rewriting against float64 numpy: contracting the reduced operands
must give the direct einsum sum (a rewriting that dropped or kept the wrong
index fails)."""
import numpy as np
import pytest
import torch

from pto_einsum import einsum, planner

CASES = [
    ("ij,jk->k", (3, 4), (4, 5)),
    ("ij,jk->i", (3, 4), (4, 5)),
    ("ij,k->k", (3, 4), (5,)),
    ("ijx,jky->ik", (2, 3, 4), (3, 5, 6)),
    ("bij,bjk->bk", (2, 3, 4), (2, 4, 5)),
    ("abc,cd->ad", (2, 3, 4), (4, 5)),
    ("i,j->", (3,), (4,)),
    ("xi,ij->j", (0, 3), (3, 4)),
    ("ij,jk->ik", (3, 4), (4, 5)),
]


@pytest.mark.parametrize("eq,s0,s1", CASES)
def test_solo_split_matches_direct_sum(eq, s0, s1):
    rng = np.random.default_rng(len(eq) + sum(s0) + sum(s1))
    a = rng.standard_normal(s0)
    b = rng.standard_normal(s1)
    reduced, in0, in1, solo0, solo1 = planner.solo_split(eq, s0, s1)
    ra = a.sum(axis=tuple(in0.index(c) for c in solo0)) if solo0 else a
    rb = b.sum(axis=tuple(in1.index(c) for c in solo1)) if solo1 else b
    got = np.einsum(reduced.replace("->", "->"), ra, rb)
    want = np.einsum(eq, a, b)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_solo_split_identifies_each_operand():
    assert planner.solo_split("ij,jk->k", (3, 4), (4, 5)) == ("j,jk->k", "ij", "jk", "i", "")
    assert planner.solo_split("ijx,jky->ik", (2, 3, 4), (3, 5, 6)) == ("ij,jk->ik", "ijx", "jky", "x", "y")
    assert planner.solo_split("ij,jk->ik", (3, 4), (4, 5))[3:] == ("", "")


def test_default_keeps_the_reference_rejection():
    a, b = torch.randn(3, 4), torch.randn(4, 5)
    with pytest.raises(ValueError, match="single-operand reduction is not supported"):
        einsum("ij,jk->k", a, b, device="cpu")


def test_opt_in_needs_gpu_operands():
    a, b = torch.randn(3, 4), torch.randn(4, 5)
    with pytest.raises(ValueError, match="GPU"):
        einsum("ij,jk->k", a, b, device="cpu", reduce_solo_axes=True)


# --------------------------------------------- pe_reduce_axes' summation order

from solo_reduce_order import ordered_sum, reduce_desc, scalar_ordered_sum  # noqa: E402


@pytest.mark.parametrize("shape,axes,V,L,C", [((3, 1000), (1,), 4, 64, 3), ((2, 37, 30), (1, 2), 8, 64, 1),
                                              ((5, 7, 9), (0, 2), 1, 1, 4), ((4, 130), (1,), 1, 64, 2),
                                              ((3, 64), (1,), 4, 64, 5), ((2, 0), (1,), 4, 64, 1)])
def test_vectorised_order_checker_matches_the_scalar_statement(shape, axes, V, L, C):
    x = np.random.default_rng(sum(shape)).standard_normal(shape).astype(np.float32) * 1e3
    x[..., ::7] *= 1e-4  # mixed magnitudes, so that orders differ in the last bits
    got = ordered_sum(x, axes, V, L, C)
    want = scalar_ordered_sum(x, axes, V, L, C)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_order_checker_with_one_lane_is_the_sequential_loop():
    x = np.random.default_rng(1).standard_normal((3, 200)).astype(np.float32)
    want = np.zeros(3, dtype=np.float32)
    for i in range(3):
        acc = np.float32(0.0)
        for v in x[i]:
            acc = np.float32(acc + v)
        want[i] = acc
    for V in (1, 4):  # groups of consecutive terms do not change a one-lane order
        assert np.array_equal(ordered_sum(x, (1,), V, 1, 1).view(np.uint32), want.view(np.uint32))
    # several lanes or chunks: a different order (the same total to rounding)
    assert not np.array_equal(ordered_sum(x, (1,), 4, 64, 1), want)
    assert np.allclose(ordered_sum(x, (1,), 4, 64, 3), x.astype(np.float64).sum(1), rtol=0, atol=1e-4)


def test_order_checker_sums_exactly_on_integers():
    x = np.random.default_rng(2).integers(-1000, 1000, size=(6, 5, 777)).astype(np.float32)
    want = x.astype(np.int64).sum(axis=(0, 2))
    for V, L, C in ((1, 1, 1), (4, 64, 7), (8, 64, 2), (1, 1, 300)):
        assert np.array_equal(ordered_sum(x, (0, 2), V, L, C).astype(np.int64), want)


def _order_of(x, axes):
    import ctypes

    from pto_einsum import abi, runtime

    d = reduce_desc(x, axes)
    out = (ctypes.c_int64 * 3)()
    runtime.check(abi.bind().pe_reduce_order(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), out), "order")
    return tuple(int(v) for v in out), int(abi.bind().pe_reduce_workspace_bytes(ctypes.byref(d)))


def test_reduce_order_choice():
    """Row mode (up to a wave per output, 16-byte groups) when the reduced axes
    form one contiguous run of >= 32 terms; lane-per-output otherwise; chunks
    (and a workspace) when outputs are too few to fill the chip."""
    (o, ws) = _order_of(torch.zeros(5000, 3000), (1,))
    assert o == (4, 64, 1) and ws == 0
    (o, ws) = _order_of(torch.zeros(5000, 300), (1,))             # 75 groups: 16 lanes of >= 4
    assert o == (4, 16, 1) and ws == 0
    (o, ws) = _order_of(torch.zeros(5000, 304, dtype=torch.float16), (1,))
    assert o == (8, 8, 1) and ws == 0
    (o, _) = _order_of(torch.zeros(64, 1026)[:, 1:], (1,))       # rows not 16-byte aligned
    assert o[:2] == (1, 64)
    (o, ws) = _order_of(torch.zeros(64, 100000), (1,))           # (the size covers unaligned bases too)
    assert o[:2] == (4, 64) and o[2] > 1 and ws >= 64 * o[2] * 4
    (o, _) = _order_of(torch.zeros(5000, 100), (1,))             # 25 groups: the fewest lanes
    assert o == (4, 4, 1)
    (o, _) = _order_of(torch.zeros(5000, 20), (1,))              # short runs: a lane per output
    assert o == (1, 1, 1)
    (o, ws) = _order_of(torch.zeros(20000, 64), (0,))            # strided reduced axis, 64 outputs
    assert o[:2] == (1, 1) and o[2] > 1 and ws == 64 * o[2] * 4
    (o, ws) = _order_of(torch.zeros(3, 0, 2), (1,))              # no terms
    assert ws == 0


def test_workspace_query_covers_unaligned_sources():
    """pe_reduce_workspace_bytes takes no source address, so its size holds
    for a base that is not 16-byte aligned too (one-element groups, hence
    more groups and chunks than an aligned base gets)."""
    buf = torch.zeros(1000 * 1000 + 4)
    h = torch.zeros(5 * 257 + 8, dtype=torch.float16)
    for whole, shifted, axes in ((buf[:-4].reshape(1000, 1000), buf[1:-3].reshape(1000, 1000), (0, 1)),
                                 (h[:5 * 257].reshape(5, 1, 257), h[1:1 + 5 * 257].reshape(5, 1, 257), (0, 1, 2))):
        (oa, wa), (ou, wu) = _order_of(whole, axes), _order_of(shifted, axes)
        assert oa[0] > 1 and ou[0] == 1 and ou[2] > oa[2]      # the unaligned plan needs more chunks
        assert wa == wu == ou[2] * 4                            # one output: C float32 chunk sums
