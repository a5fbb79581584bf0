"""Shared helpers for the parity tests: seeded inputs and the comparison bar.

The bar (per the oracle's contract):
* outputs that are single products -- the Hadamard route, and every
  contraction-free route (a C=1 matmul on the reference CPU path) -- must be
  bit-identical to the oracle, sign of zero included;
* contractions must satisfy |gpu - oracle| <= rtol * max|oracle| elementwise
  with rtol = 1e-4 for float32 inputs and 2e-3 for float16 inputs (the
  oracle runs on the float32 up-cast of the same float16 values).
"""
import hashlib
from math import prod

import numpy as np
import torch

import oracle

RTOL = {torch.float32: 1e-4, torch.float16: 2e-3}


def seed_of(*parts) -> int:
    return int(hashlib.sha1(repr(parts).encode()).hexdigest()[:8], 16)


def make_inputs(eq, s0, s1, dtype, dist="rand"):
    g = torch.Generator().manual_seed(seed_of(eq, s0, s1, str(dtype), dist))
    if dist == "rand":
        a = torch.rand(s0, generator=g)
        b = torch.rand(s1, generator=g)
    else:
        a = torch.randn(s0, generator=g)
        b = torch.randn(s1, generator=g)
    return a.to(dtype), b.to(dtype)


def contraction_size(eq, s0, s1) -> int:
    r, _ = oracle.cpu_plan(eq, s0, s1)
    return 1 if r["kind"] == "hadamard" else r["C"]


def check(got: np.ndarray, want: np.ndarray, exact: bool, rtol: float, what: str = ""):
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert got.dtype == np.float32
    if exact:
        same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
        if not same:
            bad = np.flatnonzero(got.view(np.uint32).ravel() != want.view(np.uint32).ravel())
            i = bad[0]
            raise AssertionError(f"{what}: {len(bad)} elements differ bitwise; first at {i}: "
                                 f"{got.ravel()[i]!r} vs {want.ravel()[i]!r}")
        return
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = float(np.abs(want).max()) if want.size else 0.0
    atol = rtol * max(scale, 1e-30)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float(err.max()) if err.size else 0.0
    assert worst <= atol, f"{what}: max abs err {worst:.3e} > {atol:.3e} (rtol {rtol} x max|oracle| {scale:.3e})"


def ref64_gpu(eq, a, b):
    """float64 reference on the GPU: operands permuted into contiguous
    [I, L0, C] / [I, C, L1] blocks (the CPU route's recipe), one batched
    matmul, then the output permutation.  Avoids torch.einsum's internal
    transposed views."""
    r, swapped = oracle.cpu_plan(eq, tuple(a.shape), tuple(b.shape))
    if swapped:
        a, b = b, a
    a = a.cuda().double().permute(r["perm0"]).contiguous().reshape(r["I"], r["L0"], r["C"])
    b = b.cuda().double().permute(r["perm1"]).contiguous().reshape(r["I"], r["C"], r["L1"])
    mid = torch.bmm(a, b).reshape(r["mid_shape"])
    return mid.permute(r["out_perm"]).contiguous()
