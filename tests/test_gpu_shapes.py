"""A seeded sweep of contraction shapes through the public einsum: sizes
from 1 to ~700 along M / N, K from 1 to ~6000, batch 1-3, both dtypes and
operand layouts that reach every loader (rows or k contiguous, strided
batches).  It exercises the tile / split-K choice over its whole range (64^2 or
128^2 tiles, 256-wide tiles, long-K splits, partial tiles and K tails)
against a float64 GPU reference with the contraction tolerance, and checks
run-to-run equality."""
import random

import pytest
import torch

from pto_einsum import einsum

pytestmark = pytest.mark.gpu


def _cases():
    rng = random.Random(20261202)
    eqs = ["bij,bjk->bik", "bji,bjk->bik", "bij,bkj->bik", "bji,bkj->bik", "ij,jk->ik", "ji,kj->ik"]
    out = []
    for n in range(48):
        eq = eqs[n % len(eqs)]
        M = rng.choice([1, 7, 64, 100, 128, 257, 513, 700])
        N = rng.choice([1, 9, 64, 130, 256, 320, 640])
        K = rng.choice([1, 5, 16, 100, 512, 777, 2048, 6000])
        B = rng.choice([1, 2, 3])
        dtype = torch.float32 if n % 2 == 0 else torch.float16
        out.append((eq, M, N, K, B, dtype))
    return out


def _shape(sub, dims):
    return tuple(dims[c] for c in sub)


@pytest.mark.parametrize("eq,M,N,K,B,dtype", _cases(),
                         ids=lambda v: str(v).replace("torch.", "") if not isinstance(v, int) else str(v))
def test_shape_sweep(eq, M, N, K, B, dtype):
    dims = {"b": B, "i": M, "k": N, "j": K}
    s0, s1 = eq.split("->")[0].split(",")
    g = torch.Generator().manual_seed(M * 131 + N * 17 + K + B)
    a = (torch.randn(*_shape(s0, dims), generator=g) * 0.5).to(dtype).cuda()
    b = (torch.randn(*_shape(s1, dims), generator=g) * 0.5).to(dtype).cuda()
    got = einsum(eq, a, b)
    want = torch.einsum(eq, a.double(), b.double())
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    scale = max(1.0, float(want.abs().max())) if want.numel() else 1.0
    assert got.shape == want.shape and got.dtype == torch.float32
    assert float((got.double() - want).abs().max()) <= rtol * scale if want.numel() else True
    assert torch.equal(got, einsum(eq, a, b))
