"""Launch-plan descriptors, checked on the CPU.

The GPU kernels execute exactly the strided maps a plan's descriptors
describe.  Here those maps are evaluated with numpy (as_strided views, a
float64 batched product) and compared with the oracle, so every planner
decision -- axis-group flattening, staging, strides, workspace layout -- is
checked without a GPU.  A wrong stride or staging choice shows up as a value
mismatch."""
import numpy as np
import pytest
import torch
from numpy.lib.stride_tricks import as_strided

import oracle
from pto_einsum import EinsumBuilder, launch
from ref_cases import ATTENTION_CASES, BROADCAST_CASES, CHAIN_CASES, CONFIG_CASES, EINSUM_CASES

EXTRA = [
    ("abc,cd->adb", (5, 6, 7), (7, 8)),        # free0 group split by free1 in the output
    ("acb,cd->adb", (5, 7, 6), (7, 8)),
    ("ikj,jlk->il", (5, 6, 7), (7, 8, 6)),     # contract group in opposite orders
    ("xyz,zyw->wx", (3, 4, 5), (5, 4, 6)),
    ("abcd,cdbe->ae", (2, 3, 4, 5), (4, 5, 3, 6)),
    ("ab,bc->ca", (7, 9), (9, 11)),
    ("ba,cb->ac", (9, 7), (11, 9)),
    ("bi,ib->b", (6, 7), (7, 6)),
    ("ij,ij->ji", (5, 6), (5, 6)),
    ("i,j->ji", (5,), (6,)),
    ("abcdefghij,abcdefghij->abcdefghij", (1, 2, 1, 2, 1, 2, 1, 2, 1, 3), (1, 2, 1, 2, 1, 2, 1, 2, 1, 3)),
    ("abc,abd->cd", (0, 3, 4), (0, 3, 5)),     # empty contraction -> zeros
    ("abc,cd->adb", (6, 20, 7), (7, 8)),       # free0 split in the output: a made batch
    ("acb,cd->abd", (5, 7, 18), (7, 8)),       # ... split in operand 0
    ("abcd,de->bcea", (4, 5, 6, 8), (8, 24)),  # free0 {a,b,c}: {b,c} kept, a made batch
    ("bac,cdb->adb", (3, 4, 7), (7, 20, 3)),   # a true batch axis beside a promoted one
    ("nrD,nDr->n", (33, 7, 2), (33, 2, 7)),    # operand 1 staged with a batch axis
    ("qx,xsaq->asx", (31, 64), (64, 3, 32, 31)),
    ("AoeEy,nymE->meAno", (2, 31, 1, 64, 64), (3, 64, 33, 64)),  # subscripts A / B / C
]
CASES = EINSUM_CASES + ATTENTION_CASES + BROADCAST_CASES + CHAIN_CASES + CONFIG_CASES + EXTRA


def _view(flat, shape, strides):
    return as_strided(flat, shape=tuple(shape), strides=tuple(8 * s for s in strides), writeable=False)


def _permute(d: launch.PermuteDesc, flat):
    return np.ascontiguousarray(_view(flat, d.shape, d.src_stride)).ravel()


def emulate(plan: launch.LaunchPlan, a, b, out_shape):
    a = np.ascontiguousarray(a, dtype=np.float64).ravel()
    b = np.ascontiguousarray(b, dtype=np.float64).ravel()
    if plan.route == launch.ROUTE_PRODUCT:
        d = plan.product
        prod = _view(a, d.shape, d.a_stride) * _view(b, d.shape, d.b_stride)
        return np.ascontiguousarray(prod).reshape(out_shape)
    if plan.gather0:
        a = _permute(plan.perm0, a)
    if plan.gather1:
        b = _permute(plan.perm1, b)
    g = plan.gemm
    A = _view(a, g.batch_shape + [g.M, g.K], g.a_bstride + [g.a_ms, g.a_ks])
    B = _view(b, g.batch_shape + [g.K, g.N], g.b_bstride + [g.b_ks, g.b_ns])
    c = np.full(max(1, g.c_numel), np.nan)
    C = as_strided(c, shape=tuple(g.batch_shape + [g.M, g.N]),
                   strides=tuple(8 * s for s in g.c_bstride + [g.c_ms, g.c_ns]))
    C[...] = A @ B
    if plan.scatter_out:
        c = _permute(plan.perm_out, c)
    n = int(np.prod(out_shape))
    return c[:n].reshape(out_shape)


def _plan(eq, s0, s1, dtype=torch.float32):
    b = EinsumBuilder(eq, [s0, s1], dtype)
    b.parse_equation()
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    plan = launch.plan_launch(b.recipe, b._exec_equation, b._exec_shapes[0], b._exec_shapes[1], code)
    return b, plan


@pytest.mark.parametrize("eq,s0,s1", CASES)
def test_plan_descriptors_compute_the_einsum(eq, s0, s1):
    b, plan = _plan(eq, s0, s1)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(s0).astype(np.float32)
    y = rng.standard_normal(s1).astype(np.float32)
    xe, ye = (y, x) if b._swap_operands else (x, y)
    got = emulate(plan, xe, ye, b.recipe["out_shape"])
    want = torch.einsum(eq, torch.from_numpy(x).double(), torch.from_numpy(y).double()).numpy()
    assert got.shape == want.shape
    assert not np.isnan(got).any(), "an output element was never written"
    assert np.allclose(got, want, rtol=1e-9, atol=1e-9)
    if plan.route == launch.ROUTE_GEMM:
        g = plan.gemm
        assert len(g.batch_shape) <= launch.MAX_DIMS
        # The footprint of every view stays inside its operand.
        def span(shape, strides):
            return sum((n - 1) * s for n, s in zip(shape, strides) if n > 0)
        if g.M and g.N and g.K and all(g.batch_shape):
            assert span(g.batch_shape + [g.M, g.K], g.a_bstride + [g.a_ms, g.a_ks]) < g.a_numel
            assert span(g.batch_shape + [g.K, g.N], g.b_bstride + [g.b_ks, g.b_ns]) < g.b_numel
            assert span(g.batch_shape + [g.M, g.N], g.c_bstride + [g.c_ms, g.c_ns]) < g.c_numel


@pytest.mark.parametrize("eq,s0,s1,staged", [
    ("bji,bjk->bik", (16, 777, 1000), (16, 777, 1536), (False, False, False)),       # config 2
    ("bshd,bthd->bsht", (4, 2048, 32, 128), (4, 2048, 32, 128), (False, False, False)),  # config 3
    ("tn,sn->ts", (4096, 128), (4096, 128), (False, False, False)),                  # 5.1
    ("ts,sp->tp", (4096, 4096), (4096, 128), (False, False, False)),                 # 5.3
    ("bvhd,bvhe->bhde", (2, 128, 16, 128), (2, 128, 16, 128), (False, False, False)),  # TN
    ("bhsc,bcht->bsht", (2, 8, 16, 20), (2, 20, 8, 24), (False, False, False)),
    ("abc,cd->adb", (5, 6, 7), (7, 8), (False, False, True)),                      # free0 split in output
    ("abc,cd->adb", (64, 48, 96), (96, 80), (False, False, False)),                # ... a made batch
    ("abc,cd->adb", (64, 6, 96), (96, 80), (False, False, True)),                  # ... b too small to keep
    ("acb,cd->abd", (48, 64, 40), (64, 72), (False, False, False)),                # split in operand 0
    ("abcd,de->aebc", (4, 5, 40, 8), (8, 24), (False, False, False)),              # {b, c} kept, a batch
    ("ikj,jlk->il", (5, 6, 7), (7, 8, 6), (False, True, False)),                   # only B moves
])
def test_staging_decisions(eq, s0, s1, staged):
    _, plan = _plan(eq, s0, s1)
    assert (plan.gather0, plan.gather1, plan.scatter_out) == staged


@pytest.mark.parametrize("eq,s0,s1", [("ts,ts->ts", (8192, 8192), (8192, 8192)),
                                      ("bsd,d->bsd", (8, 4096, 4096), (4096,)),
                                      ("bshd,sd->bshd", (2, 4096, 32, 128), (4096, 128)),
                                      ("i,j->ij", (64,), (96,))])
def test_products_take_the_stream_route(eq, s0, s1):
    b, plan = _plan(eq, s0, s1)
    assert plan.route == launch.ROUTE_PRODUCT
    assert plan.product.add_zero == (0 if b.recipe["elementwise"] else 1)


def test_random_plans_compute_the_einsum():
    """800 seeded random equations (tests/random_einsum.py; 200 of them with
    zero extents), single-operand reduction axes summed first as
    einsum(reduce_solo_axes=True) does: every plan, emulated in float64, gives
    torch's float64 einsum."""
    import random

    from pto_einsum import planner
    from random_einsum import random_case

    from random_einsum import EMPTY_SIZES

    rng = random.Random(20261202)
    for i in range(800):
        # the last 200 with zero extents (empty outputs, empty sums)
        sizes = EMPTY_SIZES if i >= 600 else None
        eq, s0, s1, solo = random_case(rng, solo=True, max_elems=2e5, max_work=2e6, **({"sizes": sizes} if sizes else {}))
        g = np.random.default_rng(i)
        x, y = g.standard_normal(s0), g.standard_normal(s1)
        want = torch.einsum(eq, torch.from_numpy(x), torch.from_numpy(y)).numpy()
        if solo:
            eq, in0, in1, solo0, solo1 = planner.solo_split(eq, s0, s1)
            x = x.sum(axis=tuple(in0.index(a) for a in solo0)) if solo0 else x
            y = y.sum(axis=tuple(in1.index(a) for a in solo1)) if solo1 else y
        b, plan = _plan(eq, x.shape, y.shape)
        xe, ye = (y, x) if b._swap_operands else (x, y)
        got = emulate(plan, xe, ye, b.recipe["out_shape"])
        assert not np.isnan(got).any(), f"case {i} {eq}: an output element was never written"
        scale = max(1.0, float(np.abs(want).max())) if want.size else 1.0
        assert np.allclose(got, want, rtol=1e-9, atol=1e-9 * scale), f"case {i} {eq} {x.shape} {y.shape}"
