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
