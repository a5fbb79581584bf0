"""device="cpu": the reference's CPU route, rebuilt in this package
(include/pto_einsum_cpu.h), must reproduce the oracle bit-for-bit."""
import os

import numpy as np
import pytest
import torch

import oracle
from pto_einsum import EinsumBuilder, einsum
from ref_cases import ATTENTION_CASES, BROADCAST_CASES, CHAIN_CASES, CONFIG_CASES, EINSUM_CASES

CASES = EINSUM_CASES + ATTENTION_CASES + BROADCAST_CASES + CHAIN_CASES + CONFIG_CASES


@pytest.mark.parametrize("eq,s0,s1", CASES)
def test_cpu_route_bit_exact(eq, s0, s1, build_dir):
    g = torch.Generator().manual_seed(5)
    a, b = torch.rand(s0, generator=g), torch.rand(s1, generator=g)
    got = einsum(eq, a, b, device="cpu").numpy()
    want = oracle.einsum(eq, a.numpy(), b.numpy())
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_cpu_runner_reuse_and_cleanup(build_dir):
    """test_einsum.py:208-241 and :428-448 on the CPU route."""
    builder = EinsumBuilder("ij,jk->ik", [(16, 32), (32, 16)], torch.float32, device="cpu")
    run = builder.build()
    assert os.path.exists(builder.cpp_filename) and os.path.exists(builder.so_filename)
    for seed in range(3):
        g = torch.Generator().manual_seed(seed)
        a, b = torch.rand(16, 32, generator=g), torch.rand(32, 16, generator=g)
        assert np.array_equal(run(a, b).numpy(), oracle.einsum("ij,jk->ik", a.numpy(), b.numpy()))
    with pytest.raises(ValueError, match="do not match built shapes"):
        run(torch.rand(16, 16), torch.rand(32, 16))
    with pytest.raises(TypeError, match="do not match built datatype"):
        run(torch.rand(16, 32), torch.rand(32, 16).double())
    builder.cleanup()
    assert not os.path.exists(builder.target_dir)


def test_cpu_route_rejects_float16(build_dir):
    with pytest.raises(TypeError, match="float16 is not supported on CPU"):
        einsum("ij,jk->ik", torch.rand(2, 3).half(), torch.rand(3, 4).half(), device="cpu")


def test_einsum_argument_contracts():
    a = torch.rand(3, 4)
    with pytest.raises(ValueError, match="Only exactly two operands are supported."):
        einsum("ij,jk->ik", a, device="cpu")
    with pytest.raises(ValueError, match="Operands must have the same datatype."):
        einsum("ij,jk->ik", a, torch.rand(4, 5).double(), device="cpu")
