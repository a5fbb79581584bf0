"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked by something other than a retyping of its
own formula:

* oracle/_ref -- the reference's own cpu_einsum.h compiled from its source
  (present when this container or a box that received the built files has
  them): bit-for-bit on every case;
* tests/golden/golden.npz -- vectors produced by that same reference build:
  bit-for-bit;
* closed forms: torch.permute(...).contiguous() for every permutation,
  torch.mul for the Hadamard route (both exact);
* a brute-force float32 loop (numpy scalars, c ascending) on tiny shapes:
  bit-for-bit;
* a float64 einsum: tolerance, catching a wrong perm / operand / axis role;
* planted mistakes (a dropped term, a transposed operand, a swapped sum
  order, a wrong output permutation) made in a copy of the oracle must fail
  at least one of those checks.
"""
import itertools
import os

import numpy as np
import pytest
import torch

import oracle
import ref_build
from ref_cases import BENCH_SAMPLE, REF_CASES

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
CASES = [c for c in REF_CASES if c != BENCH_SAMPLE]


def _inputs(eq, s0, s1, seed=0):
    rng = np.random.default_rng(abs(hash((eq, s0, s1, seed))) % (2 ** 32))
    return rng.standard_normal(s0).astype(np.float32), rng.standard_normal(s1).astype(np.float32)


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def _fp64(eq, a, b):
    return torch.einsum(eq, torch.from_numpy(a).double(), torch.from_numpy(b).double()).numpy()


@pytest.mark.parametrize("eq,s0,s1", CASES)
def test_oracle_matches_reference_build(eq, s0, s1):
    if not os.path.exists(ref_build.so_path(eq, s0, s1)):
        pytest.skip("reference CPU build not present (python oracle/ref_build.py)")
    a, b = _inputs(eq, s0, s1)
    want = ref_build.run(eq, a, b)
    got = oracle.einsum(eq, a, b)
    assert got.shape == want.shape
    assert np.array_equal(_bits(got), _bits(want))


def test_oracle_matches_golden_vectors():
    data = np.load(GOLDEN)
    n = 0
    for entry in data["index"]:
        key, eq, dt = str(entry).split("|")
        a, b, want = data[key + "_a"], data[key + "_b"], data[key + "_out"]
        got = oracle.einsum(eq, a.astype(np.float32), b.astype(np.float32))
        assert np.array_equal(_bits(got), _bits(want)), f"{eq} {dt}"
        n += 1
    assert n >= 60


@pytest.mark.parametrize("eq,s0,s1", CASES)
def test_oracle_close_to_float64(eq, s0, s1):
    a, b = _inputs(eq, s0, s1, seed=1)
    got = oracle.einsum(eq, a, b).astype(np.float64)
    want = _fp64(eq, a, b)
    scale = max(1.0, float(np.abs(want).max()) if want.size else 1.0)
    assert np.abs(got - want).max() <= 2e-5 * scale


TINY = [
    ("ij,jk->ik", (3, 4), (4, 5)),
    ("bji,bjk->bik", (2, 3, 4), (2, 3, 5)),
    ("bshd,bthd->bsht", (2, 3, 2, 4), (2, 2, 2, 4)),
    ("ijk,jkl->il", (2, 3, 4), (3, 4, 2)),
    ("ikj,jlk->il", (2, 4, 3), (3, 2, 4)),
    ("ij,jk->ki", (3, 4), (4, 5)),
    ("i,i->", (7,), (7,)),
    ("bsd,d->bsd", (2, 3, 4), (4,)),
    ("abc,cd->adb", (2, 3, 4), (4, 5)),
]


def _brute(eq, a, b):
    """Sequential float32 loop in the CPU route's term order."""
    r, swapped = oracle.cpu_plan(eq, a.shape, b.shape)
    lhs, to = eq.split("->")
    t0, t1 = lhs.split(",")
    if swapped:
        a, b, t0, t1 = b, a, t1, t0
    size = dict(zip(t0, a.shape))
    size.update(zip(t1, b.shape))
    out = np.zeros([size[x] for x in to], dtype=np.float32)
    kax = r["contract"]
    for oi in itertools.product(*[range(size[x]) for x in to]):
        idx = dict(zip(to, oi))
        acc = np.float32(0.0)
        for ki in itertools.product(*[range(size[x]) for x in kax]):
            idx.update(zip(kax, ki))
            p = np.float32(a[tuple(idx[x] for x in t0)]) * np.float32(b[tuple(idx[x] for x in t1)])
            acc = np.float32(acc + p)
        out[oi] = acc
    return out


@pytest.mark.parametrize("eq,s0,s1", TINY)
def test_oracle_matches_brute_force(eq, s0, s1):
    a, b = _inputs(eq, s0, s1, seed=2)
    assert np.array_equal(_bits(oracle.einsum(eq, a, b)), _bits(_brute(eq, a, b)))


# The 33 (shape, perm, dtype) cases of the reference's transpose tests
# (tests/test_transpose.py:108-161).
TRANSPOSE_CASES = [
    ((128,), (0,), np.float32), ((256,), (0,), np.float16), ((32, 64), (0, 1), np.float32),
    ((16, 32), (0, 1), np.float16), ((8, 16, 32), (0, 1, 2), np.float32),
    ((4, 8, 16, 32), (0, 1, 2, 3), np.float32), ((123,), (0,), np.float32),
    ((17, 35), (0, 1), np.float32), ((3, 7, 13), (0, 1, 2), np.float32),
    ((32, 64), (1, 0), np.float32), ((64, 32), (1, 0), np.float32), ((16, 16), (1, 0), np.float32),
    ((32, 64), (1, 0), np.float16), ((10, 20), (1, 0), np.float32), ((8, 12), (1, 0), np.float32),
    ((10, 24), (1, 0), np.float16), ((256, 256), (1, 0), np.float32), ((256, 128), (1, 0), np.float32),
    ((128, 256), (1, 0), np.float16), ((512, 64), (1, 0), np.float32), ((80, 256), (1, 0), np.float32),
    ((256, 80), (1, 0), np.float32), ((144, 144), (1, 0), np.float32), ((144, 208), (1, 0), np.float16),
    ((200, 200), (1, 0), np.float32), ((250, 130), (1, 0), np.float32), ((130, 250), (1, 0), np.float32),
    ((201, 199), (1, 0), np.float32), ((333, 257), (1, 0), np.float32), ((1000, 64), (1, 0), np.float32),
    ((250, 130), (1, 0), np.float16), ((255, 255), (1, 0), np.float16), ((257, 257), (1, 0), np.float16),
]
ND_PERMS = [((2, 3, 4, 5), p) for p in itertools.permutations(range(4))]


@pytest.mark.parametrize("shape,perm,dt", TRANSPOSE_CASES + [(s, p, np.float32) for s, p in ND_PERMS])
def test_oracle_transpose_is_permute(shape, perm, dt):
    x = np.random.default_rng(42).random(shape).astype(dt)
    want = torch.from_numpy(x).permute(perm).contiguous().numpy()
    got = oracle.transpose(x, perm)
    assert got.dtype == x.dtype and np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_oracle_hadamard_is_ieee_multiply():
    specials = np.array([0.0, -0.0, 1e-40, -1e-45, 3.4e38, np.inf, -np.inf, 1.5, -2.25, 1e-20],
                        dtype=np.float32)
    a = np.tile(specials, 10)
    b = np.repeat(specials, 10)
    want = (torch.from_numpy(a) * torch.from_numpy(b)).numpy()
    got = oracle.einsum("i,i->i", a, b)
    assert np.array_equal(_bits(got), _bits(want))


def test_oracle_sampled_matches_full():
    for eq, s0, s1 in [("bji,bjk->bik", (3, 37, 50), (3, 37, 41)),
                       ("bshd,bthd->bsht", (2, 24, 3, 16), (2, 20, 3, 16)),
                       ("ikj,jlk->il", (5, 6, 7), (7, 8, 6)),
                       ("ij,jk->ki", (9, 10), (10, 11))]:
        a, b = _inputs(eq, s0, s1, seed=3)
        full = oracle.einsum(eq, a, b).ravel()
        idx = np.random.default_rng(0).integers(0, full.size, 200)
        assert np.array_equal(_bits(oracle.sampled(eq, a, b, idx)), _bits(full[idx]))


def test_cpu_broadcast_route_adds_zero():
    """The CPU route sends broadcast equations through the C=1 matmul, whose
    sum starts at +0: a -0 product becomes +0 (cpu_einsum.h:71-76)."""
    a = np.array([[-0.0, 1.0, -1.0]], dtype=np.float32)
    b = np.array([1.0, 0.0, 0.0], dtype=np.float32)
    got = oracle.einsum("ij,j->ij", a, b)
    assert np.array_equal(_bits(got), _bits(np.array([[0.0, 0.0, 0.0]], dtype=np.float32)))


# ---------------------------------------------------------------- teeth ----

class _Planted:
    """Apply one plausible mistake to the oracle for the duration of a check."""

    def __init__(self, kind):
        self.kind = kind

    def __enter__(self):
        self._plan = oracle.cpu_plan
        self._bmm = oracle.lib().oracle_bmm_f32
        kind = self.kind

        def plan(eq, s0, s1):
            r, sw = self._plan(eq, s0, s1)
            r = dict(r)
            if kind == "transposed_operand" and r["kind"] == "matmul":
                p = list(r["perm1"])
                p[-1], p[-2] = p[-2], p[-1]
                r["perm1"] = p
            if kind == "wrong_out_perm" and r["kind"] == "matmul" and len(r["out_perm"]) > 1:
                r["out_perm"] = list(reversed(r["out_perm"]))
            if kind == "dropped_term" and r["kind"] == "matmul":
                r["drop"] = True
            return r, sw

        oracle.cpu_plan = plan
        if kind == "dropped_term":
            import ctypes

            orig = self._bmm

            def bmm(A, B, R, I, L0, L1, C):
                # Sum only c < C-1 by shrinking C on a repacked copy.
                Aa = np.ctypeslib.as_array(ctypes.cast(A, ctypes.POINTER(ctypes.c_float)), (I * L0 * C,))
                Bb = np.ctypeslib.as_array(ctypes.cast(B, ctypes.POINTER(ctypes.c_float)), (I * C * L1,))
                A2 = np.ascontiguousarray(Aa.reshape(I, L0, C)[:, :, : C - 1])
                B2 = np.ascontiguousarray(Bb.reshape(I, C, L1)[:, : C - 1, :])
                orig(A2.ctypes.data, B2.ctypes.data, R, I, L0, L1, C - 1)

            oracle.lib().oracle_bmm_f32 = bmm
        return self

    def __exit__(self, *exc):
        oracle.cpu_plan = self._plan
        oracle.lib().oracle_bmm_f32 = self._bmm


@pytest.mark.parametrize("kind", ["transposed_operand", "wrong_out_perm", "dropped_term"])
def test_checks_catch_planted_mistakes(kind):
    eq, s0, s1 = "bji,bjk->bik", (2, 6, 6), (2, 6, 6)
    if kind == "wrong_out_perm":
        eq, s0, s1 = "ij,jk->ki", (5, 6), (6, 5)
    a, b = _inputs(eq, s0, s1, seed=4)
    want = _fp64(eq, a, b)
    with _Planted(kind):
        got = oracle.einsum(eq, a, b).astype(np.float64)
    assert got.shape != want.shape or np.abs(got - want).max() > 1e-3, f"{kind} went unnoticed"


def test_summation_order_is_pinned():
    """A reversed sum order gives different bits on a cancellation-heavy
    case, and the brute-force check (ascending c) sees it."""
    a = np.array([[1e8, 1.0, -1e8, 1.0]], dtype=np.float32)
    b = np.ones((4, 1), dtype=np.float32)
    fwd = oracle.einsum("ij,jk->ik", a, b)
    rev = oracle.einsum("ij,jk->ik", a[:, ::-1].copy(), b)
    assert not np.array_equal(_bits(fwd), _bits(rev))
    assert np.array_equal(_bits(fwd), _bits(_brute("ij,jk->ik", a, b)))


# ---- linear-attention chain (composition of pinned einsum steps) ----

LINATTN_CASES = [(96, 96, 64, 128), (320, 320, 64, 128)]


def _linattn_inputs(T, S, N, P, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, N)).astype(np.float32)
    k = rng.standard_normal((S, N)).astype(np.float32)
    v = rng.standard_normal((S, P)).astype(np.float32)
    m = np.tril(rng.random((T, S))).astype(np.float32)   # not symmetric: a transposed mask is caught
    return q, k, v, m


@pytest.mark.parametrize("T,S,N,P", LINATTN_CASES)
def test_oracle_linear_attention_matches_reference_steps(T, S, N, P):
    """The composed chain equals the reference build run step by step (the
    steps are the reference's own test shapes, tests/test_llm_ops.py:81-107)."""
    q, k, v, m = _linattn_inputs(T, S, N, P, seed=3)
    steps = [("tn,sn->ts", (T, N), (S, N)), ("ts,ts->ts", (T, S), (T, S)), ("ts,sp->tp", (T, S), (S, P))]
    if not all(os.path.exists(ref_build.so_path(*st)) for st in steps):
        pytest.skip("oracle/_ref not built (no /root/reference here)")
    a = ref_build.run(steps[0][0], q, k)
    a = ref_build.run(steps[1][0], a, m)
    want = ref_build.run(steps[2][0], a, v)
    assert np.array_equal(_bits(oracle.linear_attention(q, k, v, m)), _bits(want))


@pytest.mark.parametrize("T,S,N,P", LINATTN_CASES + [(7, 5, 3, 4), (1, 9, 16, 2)])
def test_oracle_linear_attention_close_to_float64(T, S, N, P):
    q, k, v, m = _linattn_inputs(T, S, N, P, seed=4)
    ref = torch.einsum("tn,sn,sp,ts->tp", *(torch.from_numpy(x).double() for x in (q, k, v, m))).numpy()
    got = oracle.linear_attention(q, k, v, m)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(ref).max()


def _linattn_brute(q, k, v, m):
    T, N = q.shape
    S, P = v.shape
    a = np.zeros((T, S), dtype=np.float32)
    for t in range(T):
        for s in range(S):
            acc = np.float32(0.0)
            for n in range(N):
                acc = np.float32(acc + np.float32(q[t, n]) * np.float32(k[s, n]))
            a[t, s] = np.float32(acc * m[t, s])
    out = np.zeros((T, P), dtype=np.float32)
    for t in range(T):
        for p in range(P):
            acc = np.float32(0.0)
            for s in range(S):
                acc = np.float32(acc + a[t, s] * np.float32(v[s, p]))
            out[t, p] = acc
    return out


def test_oracle_linear_attention_brute_force():
    q, k, v, m = _linattn_inputs(6, 7, 5, 3, seed=5)
    assert np.array_equal(_bits(oracle.linear_attention(q, k, v, m)), _bits(_linattn_brute(q, k, v, m)))


def test_linear_attention_checks_catch_a_transposed_mask():
    """A chain that applied the mask transposed must fail the float64 pin."""
    q, k, v, m = _linattn_inputs(12, 12, 8, 4, seed=6)
    ref = torch.einsum("tn,sn,sp,ts->tp", *(torch.from_numpy(x).double() for x in (q, k, v, m))).numpy()
    wrong = oracle.linear_attention(q, k, v, np.ascontiguousarray(m.T))
    assert np.abs(wrong - ref).max() > 2e-5 * np.abs(ref).max()
