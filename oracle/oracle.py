"""CPU ORACLE -- test infrastructure only (tests/, smoke(), bench cpu_baseline).

A restatement of the reference's CPU einsum route, the parity checker for the
MI355X path.  Nothing in the product package imports this module.

Pieces and the reference code each one follows:

* ``cpu_plan``     -- the CPU-route recipe: roles, permutations and the
  operand-swap decision (builder.py:148-183, 185-261, 270-273, 555-586;
  ``_try_broadcast`` returns None on CPU, builder.py:375-376).  Written
  independently of the product planner so a planner mistake cannot hide in
  both.
* ``transpose``    -- cpu_einsum.h:35-51 (``transfer_idx`` / ``transpose``).
* ``einsum``       -- cpu_einsum.h:53-83 (gathers, fp32 triple loop from +0,
  c ascending, output gather) or cpu_einsum.h:87-92 for the Hadamard route.
  float16 operands are up-cast to float32 first: the reference CPU route
  rejects float16 (builder.py:612-613), so parity for float16 inputs is
  defined on the up-cast values.
* ``sampled``      -- the same per-output sum for selected outputs only,
  addressed in the raw operands; bit-identical to ``einsum`` there.
* ``linear_attention`` -- the reference's three-einsum linear-attention chain
  (tests/test_llm_ops.py:81-107) composed from ``einsum``, float32
  intermediates.

Parity pins: tests/test_oracle.py checks each piece against oracle/_ref (the
reference header compiled from /root/reference when present), the committed
golden vectors in tests/golden/ (made from oracle/_ref), torch.permute and
torch.mul closed forms, a brute-force float32 loop on tiny shapes and a
float64 einsum.  Nothing here is "parity unpinned".
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading
from math import prod

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "_build", "liboracle.so")

_lib = None
_lock = threading.Lock()

_I64P = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compile the C restatement (oracle/Makefile) and return the library path."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    return LIB_PATH


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                build()
            L = ctypes.CDLL(LIB_PATH)
            vp = ctypes.c_void_p
            L.oracle_gather_b32.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int, _I64P, _I64P]
            L.oracle_gather_b16.argtypes = [vp, vp, ctypes.c_int64, ctypes.c_int, _I64P, _I64P]
            L.oracle_bmm_f32.argtypes = [vp, vp, vp] + [ctypes.c_int64] * 4
            L.oracle_sampled_f32.argtypes = [vp, vp, ctypes.c_int64, _I64P, _I64P, ctypes.c_int,
                                             _I64P, _I64P, _I64P, vp]
            L.oracle_hadamard_f32.argtypes = [vp, vp, vp, ctypes.c_int64]
            for f in ("oracle_gather_b32", "oracle_gather_b16", "oracle_bmm_f32",
                      "oracle_sampled_f32", "oracle_hadamard_f32"):
                getattr(L, f).restype = None
            _lib = L
        return _lib


def _i64(seq):
    arr = (ctypes.c_int64 * max(1, len(seq)))(*[int(x) for x in seq])
    return arr


def _strides(shape):
    st, run = [1] * len(shape), 1
    for p in range(len(shape) - 1, -1, -1):
        st[p] = run
        run *= int(shape[p])
    return st


# --------------------------------------------------------------------------
# CPU-route recipe
# --------------------------------------------------------------------------

def _terms(eq):
    lhs, out = eq.split("->")
    a, b = lhs.split(",")
    return a.strip(), b.strip(), out.strip()


def _recipe(eq, shape0, shape1):
    t0, t1, to = _terms(eq)
    dim = {}
    for t, s in ((t0, shape0), (t1, shape1)):
        for ax, n in zip(t, s):
            dim[ax] = int(n)
    out_shape = tuple(dim[ax] for ax in to)
    if t0 == t1 == to:
        return dict(kind="hadamard", out_shape=out_shape)
    shared = set(t0) & set(t1)
    lone = (set(t0) - set(t1) - set(to)) | (set(t1) - set(t0) - set(to))
    if lone:
        raise ValueError("single-operand reduction is not supported")
    # Role order: batch and contract axes by input1 position, free axes by
    # their own input's position (builder.py:240-243).
    batch = [ax for ax in t1 if ax in shared and ax in to]
    contract = [ax for ax in t1 if ax in shared and ax not in to]
    free0 = [ax for ax in t0 if ax not in shared and ax in to]
    free1 = [ax for ax in t1 if ax not in shared and ax in to]
    perm0 = [t0.index(ax) for ax in batch + free0 + contract]
    perm1 = [t1.index(ax) for ax in batch + contract + free1]
    mid = batch + free0 + free1
    # Output perm: the k-th output axis is mid[out_perm[k]].
    out_perm = [mid.index(ax) for ax in to]
    identity = out_perm == list(range(len(out_perm)))
    fusible = (len(free0) == 1 and len(free1) == 1 and to[-1] == free1[0] and not identity)
    return dict(
        kind="matmul", out_shape=out_shape, perm0=perm0, perm1=perm1, out_perm=out_perm,
        mid_shape=tuple(dim[ax] for ax in mid), identity=identity, fusible=fusible,
        I=prod(dim[a] for a in batch), L0=prod(dim[a] for a in free0),
        L1=prod(dim[a] for a in free1), C=prod(dim[a] for a in contract),
        batch=batch, contract=contract, free0=free0, free1=free1,
    )


def cpu_plan(eq, shape0, shape1):
    """The CPU route's recipe and operand order (builder.py:555-586).

    Returns ``(recipe, swapped)``; when ``swapped`` the recipe is built on
    ``in1, in0`` and the operands are fed in that order.
    """
    shape0, shape1 = tuple(shape0), tuple(shape1)
    r = _recipe(eq, shape0, shape1)
    if (os.getenv("EINSUM_DISABLE_OPERAND_SWAP", "0") == "0" and r["kind"] == "matmul"
            and not r["fusible"] and not r["identity"]):
        t0, t1, to = _terms(eq)
        s = _recipe(f"{t1},{t0}->{to}", shape1, shape0)
        if s["fusible"] or s["identity"]:
            return s, True
    return r, False


# --------------------------------------------------------------------------
# Arithmetic
# --------------------------------------------------------------------------

def _as_f32(x):
    x = np.asarray(x)
    if x.dtype == np.float16:
        x = x.astype(np.float32)
    if x.dtype != np.float32:
        raise TypeError(f"oracle takes float32/float16 arrays, got {x.dtype}")
    return np.ascontiguousarray(x)


def transpose(x, perm):
    """``x.transpose(perm)`` materialised through the reference index map."""
    x = np.ascontiguousarray(np.asarray(x))
    perm = [int(p) for p in perm]
    shape = x.shape
    to_shape = [shape[p] for p in perm]
    st = _strides(shape)
    perm_strides = [st[p] for p in perm]
    res = np.empty(to_shape, dtype=x.dtype)
    n = int(np.prod(to_shape)) if to_shape else 1
    if x.dtype.itemsize == 4:
        fn = lib().oracle_gather_b32
    elif x.dtype.itemsize == 2:
        fn = lib().oracle_gather_b16
    else:
        raise TypeError(f"oracle transpose takes 2- or 4-byte elements, got {x.dtype}")
    fn(x.ctypes.data, res.ctypes.data, n, len(perm), _i64(to_shape), _i64(perm_strides))
    return res


def einsum(eq, a, b):
    """The reference CPU route's result for ``eq`` on float32 (or up-cast) inputs."""
    a, b = _as_f32(a), _as_f32(b)
    lhs = eq.replace(" ", "").split("->")[0].split(",")
    sizes = {}
    for labels, shape in ((lhs[0], a.shape), (lhs[1], b.shape)):
        if len(labels) != len(shape):
            raise ValueError(f"oracle einsum: {labels!r} does not match shape {shape}")
        for c, n in zip(labels, shape):
            if sizes.setdefault(c, n) != n:
                raise ValueError(f"oracle einsum: axis {c!r} has sizes {sizes[c]} and {n}")
    r, swapped = cpu_plan(eq, a.shape, b.shape)
    if r["kind"] == "hadamard":
        out = np.empty(r["out_shape"], dtype=np.float32)
        lib().oracle_hadamard_f32(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
        return out
    if swapped:
        a, b = b, a
    A = transpose(a, r["perm0"])
    B = transpose(b, r["perm1"])
    mid = np.empty(r["mid_shape"], dtype=np.float32)
    lib().oracle_bmm_f32(A.ctypes.data, B.ctypes.data, mid.ctypes.data,
                         r["I"], r["L0"], r["L1"], r["C"])
    return transpose(mid, r["out_perm"])


def sampled(eq, a, b, out_index):
    """Oracle values at the given output positions (flat C-order indices).

    Bit-identical to ``einsum(eq, a, b).ravel()[out_index]``: same recipe,
    same operand order and the same c-ascending float32 sum.
    """
    a, b = _as_f32(a), _as_f32(b)
    r, swapped = cpu_plan(eq, a.shape, b.shape)
    out_index = np.ascontiguousarray(np.asarray(out_index, dtype=np.int64).ravel())
    if r["kind"] == "hadamard":
        return (a.ravel()[out_index] * b.ravel()[out_index]).astype(np.float32)
    t0, t1, to = _terms(eq)
    if swapped:
        a, b = b, a
        t0, t1 = t1, t0
    sa = dict(zip(t0, _strides(a.shape)))
    sb = dict(zip(t1, _strides(b.shape)))
    out_shape = r["out_shape"]
    coords = np.unravel_index(out_index, out_shape) if out_shape else ()
    a_base = np.zeros(len(out_index), dtype=np.int64)
    b_base = np.zeros(len(out_index), dtype=np.int64)
    for ax, c in zip(to, coords):
        c = c.astype(np.int64)
        if ax in sa:
            a_base += c * sa[ax]
        if ax in sb:
            b_base += c * sb[ax]
    kdims = r["contract"]
    k_shape = [a.shape[t0.index(ax)] for ax in kdims]
    res = np.empty(len(out_index), dtype=np.float32)
    lib().oracle_sampled_f32(
        a.ctypes.data, b.ctypes.data, len(out_index),
        a_base.ctypes.data_as(_I64P), b_base.ctypes.data_as(_I64P), len(kdims),
        _i64(k_shape), _i64([sa[ax] for ax in kdims]), _i64([sb[ax] for ax in kdims]),
        res.ctypes.data)
    return res


def bmm(A, B):
    """The raw triple loop on canonical ``[I,L0,C] x [I,C,L1]`` float32 operands."""
    A, B = _as_f32(A), _as_f32(B)
    I, L0, C = A.shape
    I2, C2, L1 = B.shape
    assert I == I2 and C == C2
    R = np.empty((I, L0, L1), dtype=np.float32)
    lib().oracle_bmm_f32(A.ctypes.data, B.ctypes.data, R.ctypes.data, I, L0, L1, C)
    return R


def hadamard(a, b):
    a, b = _as_f32(a), _as_f32(b)
    if a.shape != b.shape:
        raise ValueError(f"hadamard: operand shapes {a.shape} and {b.shape} differ")
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_hadamard_f32(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def linear_attention(q, k, v, m):
    """The linear-attention chain as the reference runs it, three einsums with
    float32 intermediates (tests/test_llm_ops.py:97-99 of the reference, with
    the ``.to(dtype)`` casts read as float32):

        A = einsum("tn,sn->ts", q, k); A = einsum("ts,ts->ts", A, m);
        out = einsum("ts,sp->tp", A, v)

    float16 operands are up-cast to float32 first (exact)."""
    a = einsum("tn,sn->ts", q, k)
    a = einsum("ts,ts->ts", a, m)
    return einsum("ts,sp->tp", a, v)
