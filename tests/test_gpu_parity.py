"""GPU parity: the gfx950 path against the CPU oracle, through the public API.

Case lists follow the reference's own test matrices (tests/test_einsum.py:22-129,
tests/test_llm_ops.py:34-125) plus the benchmark equations at reduced sizes and
edge shapes.  Every case runs in float32 and float16.
"""
import numpy as np
import pytest
import torch

import oracle
from parity_util import RTOL, check, contraction_size, make_inputs, ref64_gpu
from ref_cases import ATTENTION_CASES, BROADCAST_CASES, CHAIN_CASES, CONFIG_CASES, EINSUM_CASES

pytestmark = pytest.mark.gpu

ALL_CASES = EINSUM_CASES + ATTENTION_CASES + BROADCAST_CASES + CHAIN_CASES + CONFIG_CASES


def _id(c):
    eq, s0, s1 = c
    return f"{eq}-{'x'.join(map(str, s0))}-{'x'.join(map(str, s1))}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", ALL_CASES, ids=[_id(c) for c in ALL_CASES])
def test_parity(eq, s0, s1, dtype, build_dir):
    from pto_einsum import einsum

    a, b = make_inputs(eq, s0, s1, dtype)
    got = einsum(eq, a.cuda(), b.cuda()).cpu().numpy()
    want = oracle.einsum(eq, a.float().numpy(), b.float().numpy())
    exact = contraction_size(eq, s0, s1) <= 1
    check(got, want, exact, RTOL[dtype], f"{eq} {s0} {s1} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", [
    ("bij,bjk->bik", (64, 128, 128), (64, 128, 128)),       # test_einsum.py:244-272
    ("bihd,bjhd->bihj", (2, 128, 16, 128), (2, 128, 16, 128)),  # :275-304 (NT)
    ("bihj,bjhd->bihd", (2, 128, 16, 128), (2, 128, 16, 128)),  # :307-334 (NN-strided)
    ("bvhd,bvhe->bhde", (2, 128, 16, 128), (2, 128, 16, 128)),  # :337-364 (TN)
    ("ts,sp->tp", (512, 2048), (2048, 64)),                     # split-K reduction
])
def test_deterministic(eq, s0, s1, dtype, build_dir):
    """Eight more runs on the same inputs are bit-identical to the first."""
    from pto_einsum import EinsumBuilder

    builder = EinsumBuilder(eq, [s0, s1], dtype)
    run = builder.build()
    a, b = make_inputs(eq, s0, s1, dtype)
    a, b = a.cuda(), b.cuda()
    ref = run(a, b).clone()
    want = oracle.einsum(eq, a.float().cpu().numpy(), b.float().cpu().numpy())
    check(ref.cpu().numpy(), want, False, RTOL[dtype], eq)
    for _ in range(8):
        assert torch.equal(run(a, b), ref), f"{eq}: run-to-run difference"
    builder.cleanup()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_broadcast_multi_op_sequence(dtype, build_dir):
    """tests/test_llm_ops.py:146-165: distinct broadcast builders built, run and
    cleaned up back to back, each with the same seed, so an op that read a
    stale buffer of the previous one (or a store still in flight) would show
    up as a wrong result; every output is checked bit for bit against the
    oracle (the broadcast route is exact: one product per element)."""
    from pto_einsum import EinsumBuilder

    for eq, s0, s1 in BROADCAST_CASES:
        torch.manual_seed(0)
        a, b = torch.rand(s0).to(dtype), torch.rand(s1).to(dtype)
        builder = EinsumBuilder(eq, [s0, s1], dtype)
        got = builder.build()(a.cuda(), b.cuda()).cpu().numpy()
        check(got, oracle.einsum(eq, a.float().numpy(), b.float().numpy()), True, 0.0, f"{eq} {dtype}")
        builder.cleanup()


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_einsums_against_the_oracle(seed, build_dir):
    """150 seeded random equations per seed (tests/random_einsum.py: batch,
    free and contracted axes in random counts, sizes and orders, both dtypes,
    a third of the operands as non-contiguous views and some contiguous at a
    base one element into a buffer, so not 16-byte aligned) through the
    public einsum against the oracle; equations with single-operand reduction
    axes (reduce_solo_axes=True) against torch's float64 einsum."""
    import random

    from pto_einsum import einsum
    from random_einsum import EMPTY_SIZES, SIZES, random_case

    rng = random.Random(seed)
    for i in range(150):
        # seed 3 draws extents with zeros: empty outputs and empty sums
        sizes = EMPTY_SIZES if seed == 3 else SIZES
        eq, s0, s1, solo = random_case(rng, solo=True, max_elems=1e6, max_work=5e7, sizes=sizes)
        dtype = rng.choice([torch.float32, torch.float16])
        a, b = make_inputs(eq, s0, s1, dtype)
        ga, gb = a.cuda(), b.cuda()
        if ga.dim() >= 2 and rng.random() < 0.33:
            ga = ga.t().contiguous().t() if ga.dim() == 2 else ga.transpose(0, -1).contiguous().transpose(0, -1)
        if gb.dim() >= 2 and rng.random() < 0.33:
            gb = gb.t().contiguous().t() if gb.dim() == 2 else gb.transpose(0, -1).contiguous().transpose(0, -1)
        if rng.random() < 0.25:
            flat = torch.zeros(ga.numel() + 1, dtype=dtype, device="cuda")
            flat[1:] = ga.reshape(-1)
            ga = flat[1:].view(ga.shape)
        what = f"random case {seed}.{i}: {eq} {s0} {s1} {dtype}{' solo' if solo else ''}"
        print(what, flush=True)
        got = einsum(eq, ga, gb, reduce_solo_axes=solo).cpu()
        if solo:
            want = torch.einsum(eq, a.double(), b.double())
            scale = float(want.abs().max()) if want.numel() else 0.0
            err = float((got.double() - want).abs().max()) if want.numel() else 0.0
            assert err <= RTOL[dtype] * max(scale, 1e-30), f"{what}: err {err:.3e} scale {scale:.3e}"
        else:
            want = oracle.einsum(eq, a.float().numpy(), b.float().numpy())
            check(got.numpy(), want, contraction_size(eq, s0, s1) <= 1, RTOL[dtype], what)


def test_random_contractions_with_inf_and_nan(build_dir):
    """60 seeded random contractions whose operands carry a sprinkle of +inf,
    -inf and NaN: which outputs are NaN, +inf or -inf does not depend on the
    summation order (no finite sum here comes near overflow), so the pattern
    must equal the oracle's exactly; finite outputs meet the contraction bar."""
    import random

    from pto_einsum import einsum
    from random_einsum import random_case

    rng = random.Random(41)
    specials = torch.tensor([float("inf"), float("-inf"), float("nan")])
    n = 0
    while n < 60:
        eq, s0, s1, _ = random_case(rng, max_elems=3e5, max_work=2e7)
        if contraction_size(eq, s0, s1) <= 1:
            continue
        n += 1
        dtype = rng.choice([torch.float32, torch.float16])
        g = torch.Generator().manual_seed(n)
        a, b = torch.rand(s0, generator=g), torch.rand(s1, generator=g)
        for x in (a, b):
            flat = x.view(-1)
            k = max(1, flat.numel() // 200)
            flat[torch.randint(0, flat.numel(), (k,), generator=g)] = specials[torch.randint(0, 3, (k,), generator=g)]
        a, b = a.to(dtype), b.to(dtype)
        what = f"special case {n}: {eq} {s0} {s1} {dtype}"
        print(what, flush=True)
        got = einsum(eq, a.cuda(), b.cuda()).cpu().numpy()
        want = oracle.einsum(eq, a.float().numpy(), b.float().numpy())
        for f in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(f(got), f(want)), f"{what}: {f.__name__} pattern differs"
        fin = np.isfinite(want)
        if fin.any():
            scale = float(np.abs(want[fin]).max())
            assert float(np.abs(got[fin].astype(np.float64) - want[fin]).max()) <= RTOL[dtype] * max(scale, 1e-30), what


@pytest.mark.parametrize("dtype,tiny", [(torch.float32, 1e-41), (torch.float16, 1e-6)], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", [("ij,jk->ik", (64, 128), (128, 96)), ("bji,bjk->bik", (4, 77, 100), (4, 77, 150)),
                                      ("ik,jk->ij", (512, 256), (512, 256)), ("ts,sp->tp", (256, 4096), (4096, 128)),
                                      ("ij,jk->ik", (4096, 2048), (2048, 4096))])
def test_subnormal_operands_are_not_flushed(eq, s0, s1, dtype, tiny, build_dir):
    """Every A element subnormal in its own dtype, so every output is tiny:
    a kernel that flushed subnormal inputs (or results) to zero would be off
    by 100 % of the output scale.  Staged, direct-load, split-K and (float16
    4096 x 2048 x 4096) 256x256 GEMMs are reached; the reference is float64
    on the GPU, where these values are normal numbers."""
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(1)
    a = (torch.rand(s0, generator=g) * tiny).to(dtype)
    b = torch.rand(s1, generator=g).to(dtype)
    got = einsum(eq, a.cuda(), b.cuda()).double()
    want = ref64_gpu(eq, a, b)
    scale = float(want.abs().max())
    assert scale > 0
    assert float((got - want).abs().max()) <= RTOL[dtype] * scale, f"{eq} subnormal {dtype}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_batched_partial_output_tiles(dtype, build_dir):
    """tests/test_einsum.py:161-178: the reference's case for batched (I > 1)
    partial output tiles, which it skips (and rejects, :193-197) until that
    path lands; here it runs, against the oracle."""
    from pto_einsum import einsum

    eq, s0, s1 = "bij,bjk->bik", (4, 200, 64), (4, 64, 128)
    a, b = make_inputs(eq, s0, s1, dtype)
    got = einsum("bij, bjk -> bik", a.cuda(), b.cuda()).cpu().numpy()
    check(got, oracle.einsum(eq, a.float().numpy(), b.float().numpy()), False, RTOL[dtype], eq)


def test_builder_reuse(build_dir):
    """test_einsum.py:208-241: a runner reused with fresh data, incl. K != C."""
    from pto_einsum import EinsumBuilder

    for eq, s0, s1, reps in (("ij,jk->ik", (32, 64), (64, 32), 3),
                             ("bij,bjk->bik", (8, 16, 20), (8, 20, 64), 10)):
        run = EinsumBuilder(eq, [s0, s1], torch.float32).build()
        g = torch.Generator().manual_seed(7)
        for _ in range(reps):
            a, b = torch.rand(s0, generator=g), torch.rand(s1, generator=g)
            got = run(a.cuda(), b.cuda()).cpu().numpy()
            check(got, oracle.einsum(eq, a.numpy(), b.numpy()), False, 1e-4, eq)


def test_special_values_bit_exact(build_dir):
    """Hadamard and broadcast keep subnormals, signed zeros, inf and NaN
    exactly as the oracle does (Hadamard: a*b; broadcast route: 0 + a*b)."""
    from pto_einsum import einsum

    specials = np.array([0.0, -0.0, 1e-40, -1e-40, 1.17549435e-38, 3.4e38, -3.4e38,
                         np.inf, -np.inf, 1.0, -1.0, 0.5, 2.0, 1e-20, -1e-20, 7.0], dtype=np.float32)
    a = np.tile(specials, 16)
    b = np.repeat(specials, 16)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    got = einsum("i,i->i", ta, tb).cpu().numpy()
    want = oracle.einsum("i,i->i", a, b)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    check(np.where(nan, 0, got).astype(np.float32), np.where(nan, 0, want).astype(np.float32), True, 0, "hadamard")
    a2 = a.reshape(16, 16)
    got2 = einsum("ij,j->ij", torch.from_numpy(a2).cuda(), torch.from_numpy(specials).cuda()).cpu().numpy()
    want2 = oracle.einsum("ij,j->ij", a2, specials)
    nan2 = np.isnan(want2)
    assert np.array_equal(np.isnan(got2), nan2)
    check(np.where(nan2, 0, got2).astype(np.float32), np.where(nan2, 0, want2).astype(np.float32), True, 0, "bcast")


def test_decay_mask_subnormals(build_dir):
    """Config-4a shape family at a reduced size: with gamma = 0.96 the decay
    0.96^(t-s) falls below FLT_MIN inside a 2048 window, so the products
    cover normals, subnormals and underflow to zero."""
    from pto_einsum import einsum

    t = 2048
    g = torch.Generator().manual_seed(3)
    x = torch.rand(t, t, generator=g)
    i = torch.arange(t, dtype=torch.float64)
    m = torch.where(i[:, None] >= i[None, :], 0.96 ** (i[:, None] - i[None, :]), torch.zeros(())).float()
    got = einsum("ts,ts->ts", x.cuda(), m.cuda()).cpu().numpy()
    want = oracle.hadamard(x.numpy(), m.numpy())
    assert np.count_nonzero((want != 0) & (np.abs(want) < 1.17549435e-38)) > 0
    check(got, want, True, 0, "decay mask")


def test_validation_errors(build_dir):
    """test_einsum.py:400-425 contracts on the GPU device."""
    from pto_einsum import EinsumBuilder, einsum

    a = torch.rand(32, 64, device="cuda")
    b = torch.rand(64, 32, device="cuda")
    with pytest.raises(ValueError, match="Only exactly two operands are supported."):
        einsum("ij,jk->ik", a)
    with pytest.raises(ValueError, match="Operands must have the same datatype."):
        einsum("ij,jk->ik", a, b.to(torch.int32))
    run = EinsumBuilder("ij,jk->ik", [(32, 64), (64, 32)], torch.float32).build()
    with pytest.raises(ValueError, match="do not match built shapes"):
        run(torch.rand(32, 32, device="cuda"), b)
    with pytest.raises(TypeError, match="do not match built datatype"):
        run(a, b.to(torch.int32))
    with pytest.raises(ValueError, match="single-operand reduction is not supported"):
        einsum("ij,jk->k", a, b)
    with pytest.raises(TypeError, match="Unsupported torch dtype"):
        einsum("ij,jk->ik", a.bfloat16(), b.bfloat16())


def test_non_contiguous_and_npu_alias(build_dir):
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(11)
    base = torch.rand(64, 96, generator=g)
    b = torch.rand(64, 40, generator=g)
    at = base.cuda().t()  # non-contiguous view (96, 64)
    got = einsum("ij,jk->ik", at, b.cuda(), device="npu").cpu().numpy()
    check(got, oracle.einsum("ij,jk->ik", base.t().contiguous().numpy(), b.numpy()), False, 1e-4, "view")
