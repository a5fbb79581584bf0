"""Equation planner: validation, role classification and the einsum recipe.

Restates the reference planner (`src/pto_einsum/builder.py:148-604`) in the
same field vocabulary so the recipe a caller inspects is the one the reference
would produce:

* ``validate_expr``      <- ``_validate_einsum_expr`` (builder.py:148-183)
* ``parse_recipe``       <- ``parse_recipe``          (builder.py:185-367)
* ``try_broadcast``      <- ``_try_broadcast``        (builder.py:369-447)
* ``transpose_config``   <- ``transpose_config_gen``  (builder.py:449-461)
* ``plan_operand_order`` <- ``parse_equation`` swap   (builder.py:555-586)

Two deliberate differences from the reference:

* the broadcast classifier has no 4096 / 8192 size caps (builder.py:411-421);
  those bound an Ascend on-chip buffer, the MI355X kernel streams any size;
* there is no batched partial-tile guard (builder.py:593-604); the MI355X GEMM
  masks partial tiles of any batch count.

The recipe fields that steer the Ascend kernels (``in_nt``, ``out_fusible``)
are kept with the reference's exact gating (tile size from
``EINSUM_TILE_SIZE``), because callers and tests read them as path gates.  The
MI355X launch plan (``launch.py``) derives its own descriptors from the roles.
"""
from __future__ import annotations

import os
from math import prod
from typing import Dict, List, Optional, Sequence, Tuple

_ALPHABET = frozenset("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ")

# Neutral field groups, mirroring builder.py:25-42.
NO_BCAST = dict(
    broadcast=False, bc_mode=0, bc_Cc=1, bc_Rr=1, bc_Inner=1, bc_Outer=1,
    bc_sizeB=1, bc_full_is_in0=True, bc_outer_dims=(), bc_outer_bstride=(),
)
NO_FUSE = dict(
    out_fusible=0, out_row_stride=0, out_n_batch=0,
    out_batch_sizes=(), out_batch_strides=(),
)
NO_NT = dict(
    in_nt=0, in_n_batch=0, in0_row_stride=0, in0_k_stride=0, in1_col_stride=0,
    in1_k_stride=0, in_batch_sizes=(), in0_batch_strides=(), in1_batch_strides=(),
)


def row_major_strides(shape: Sequence[int]) -> List[int]:
    """Element strides of a C-order tensor of ``shape``."""
    strides = [1] * len(shape)
    run = 1
    for p in range(len(shape) - 1, -1, -1):
        strides[p] = run
        run *= int(shape[p])
    return strides


def split_equation(fn: str) -> Tuple[str, str, str]:
    """Split ``'in0,in1->out'`` (whitespace allowed) into its three subscripts."""
    if "->" not in fn:
        raise ValueError(f"einsum string {fn} is invalid: an explicit '->' output is required")
    lhs, out = fn.split("->", 1)
    parts = lhs.split(",")
    if len(parts) != 2:
        raise ValueError(f"einsum string {fn} is invalid: exactly two input operands are required")
    return parts[0].strip(), parts[1].strip(), out.strip()


def validate_expr(fn: str, shape0: Sequence[int], shape1: Sequence[int]):
    """Check the equation against the shapes and compute the output shape.

    Same rules and messages as builder.py:148-183: subscripts in [a-zA-Z] (no
    ellipsis), no repeated subscript within one term, every output subscript
    present in an input, operand ranks match their terms, and shared subscripts
    agree in size.  Returns ``(normalised_equation, out_shape)``.
    """
    in0, in1, out = split_equation(fn)
    if not (_ALPHABET >= set(in0 + in1 + out)):
        raise ValueError(f"einsum string {fn} is invalid: subscripts should be in [a-zA-Z]")
    for label, subs in (("input0", in0), ("input1", in1), ("output", out)):
        for a in subs:
            if subs.count(a) > 1:
                raise ValueError(
                    f"einsum string {fn} is invalid: {label} subscripts includes '{a}' multiple times")
    remaining = set(out) - set(in0) - set(in1)
    if remaining:
        raise ValueError(f"einsum string {fn} is invalid: output subscripts {remaining} not found in inputs")
    if len(set(in0)) != len(shape0):
        raise ValueError(f"Input0 requires {len(set(in0))} dimensions, but {len(shape0)} is given")
    if len(set(in1)) != len(shape1):
        raise ValueError(f"Input1 requires {len(set(in1))} dimensions, but {len(shape1)} is given")
    for a in set(in0) & set(in1):
        s0, s1 = shape0[in0.index(a)], shape1[in1.index(a)]
        if s0 != s1:
            raise ValueError(
                f"Input dimension size mismatches for common subscript '{a}': {s0} and {s1}")
    out_shape = tuple(int(shape0[in0.index(a)]) if a in in0 else int(shape1[in1.index(a)])
                      for a in out)
    return f"{in0},{in1}->{out}", out_shape


def solo_split(fn: str, shape0: Sequence[int], shape1: Sequence[int]):
    """Single-operand reduction axes of a validated equation: the indices of
    each input found in neither the other input nor the output (torch sums
    them; the reference rejects them, builder.py:218-229).  Returns
    ``(reduced_equation, in0, in1, solo0, solo1)``: the equation with those
    indices removed, the two input subscripts and the solo indices of each
    input in subscript order.  Summing them out of their operands first and
    contracting the rest gives the same sum."""
    norm, _ = validate_expr(fn, shape0, shape1)
    in0, in1, out = split_equation(norm)
    solo0 = "".join(a for a in in0 if a not in in1 and a not in out)
    solo1 = "".join(a for a in in1 if a not in in0 and a not in out)
    e0 = "".join(a for a in in0 if a not in solo0)
    e1 = "".join(a for a in in1 if a not in solo1)
    return f"{e0},{e1}->{out}", in0, in1, solo0, solo1


def _tile_size() -> int:
    return int(os.getenv("EINSUM_TILE_SIZE", "128"))


def _pad16(x: int) -> int:
    return (x + 15) // 16 * 16


def try_broadcast(in0: str, in1: str, out: str, shape0, shape1, out_shape, device: str):
    """Classify a contraction-free equation as a broadcast multiply, else ``None``.

    Restates builder.py:369-447: exactly one operand ("full") carries every
    output axis, already in output order; the other ("broadcast") operand's
    axes appear in output order.  Mode 0 (column expand) when the innermost
    output axis is present in the broadcast operand, mode 1 (scalar per group)
    otherwise.  The CPU route has no broadcast kernel (builder.py:375-376).
    Unlike the reference there is no size cap on ``Cc`` or ``sizeB``.
    """
    if device == "cpu":
        return None
    s_in0, s_in1, s_out = set(in0), set(in1), set(out)
    full_is_in0 = s_in0 == s_out
    full_is_in1 = s_in1 == s_out
    if full_is_in0 == full_is_in1:
        return None
    full, bc = (in0, in1) if full_is_in0 else (in1, in0)
    if full != out:
        return None
    n = len(out)
    sizes = list(out_shape)
    positions = [out.index(ax) for ax in bc]
    if positions != sorted(positions):
        return None
    present = [out[p] in set(bc) for p in range(n)]
    bstride = [0] * n
    run = 1
    for p in range(n - 1, -1, -1):
        if present[p]:
            bstride[p] = run
            run *= sizes[p]
    size_b = prod(sizes[p] for p in positions) if positions else 1
    p = n - 1
    if n and present[n - 1]:
        mode = 0
        cc = 1
        while p >= 0 and present[p]:
            cc *= sizes[p]
            p -= 1
        rr = 1
        while p >= 0 and not present[p]:
            rr *= sizes[p]
            p -= 1
        inner = rr * cc
    else:
        mode = 1
        inner = 1
        while p >= 0 and not present[p]:
            inner *= sizes[p]
            p -= 1
        cc, rr = 1, 1
    outer_dims = tuple(sizes[q] for q in range(p + 1))
    outer_bstride = tuple(bstride[q] for q in range(p + 1))
    return dict(
        in_transpose_idxs=((), ()),
        out_interpret_shape=tuple(out_shape),
        out_transpose_idxs=tuple(range(n)),
        out_shape=tuple(out_shape),
        L0=1, L1=1, I=prod(out_shape), C=1,
        elementwise=False,
        n_elem=prod(out_shape),
        broadcast=True, bc_mode=mode, bc_Cc=cc, bc_Rr=rr, bc_Inner=inner,
        bc_Outer=prod(outer_dims) if outer_dims else 1,
        bc_sizeB=size_b, bc_full_is_in0=full_is_in0,
        bc_outer_dims=outer_dims, bc_outer_bstride=outer_bstride,
        **NO_FUSE, **NO_NT,
    )


def parse_recipe(fn: str, shape0, shape1, device: str = "cuda") -> Dict:
    """Build the transpose -> batched matmul -> transpose recipe for ``fn``.

    Restates builder.py:185-367.  Roles: ``contract`` (in both inputs, not in
    the output) and ``inplace`` (in both inputs and the output) are ordered by
    their position in input1; ``invariant0``/``invariant1`` (output axes of one
    input) by their position in their own input.  Input0 is permuted to
    ``[inplace, invariant0, contract]``, input1 to ``[inplace, contract,
    invariant1]`` and the matmul result ``[inplace, invariant0, invariant1]`` is
    permuted into the output by ``argsort`` of the output positions.
    """
    fn, out_shape = validate_expr(fn, shape0, shape1)
    s0, s1, so = split_equation(fn)
    in0, in1, out = list(s0), list(s1), list(so)

    if in0 == in1 == out:
        n = prod(out_shape)
        return dict(
            in_transpose_idxs=((), ()),
            out_interpret_shape=tuple(out_shape),
            out_transpose_idxs=tuple(range(len(out_shape))),
            out_shape=tuple(out_shape),
            L0=1, L1=1, I=n, C=1,
            elementwise=True, n_elem=n,
            **NO_BCAST, **NO_FUSE, **NO_NT,
        )

    set0, set1, seto = set(in0), set(in1), set(out)
    common = set0 & set1
    contract_set = common - seto
    inplace_set = common & seto
    solo = (set0 - set1 - seto) | (set1 - set0 - seto)
    if solo:
        raise ValueError(
            f"einsum '{fn}': index {sorted(solo)} appears in only one operand and "
            "is reduced away; single-operand reduction is not supported.")

    if not contract_set:
        bc = try_broadcast(in0, in1, out, shape0, shape1, out_shape, device)
        if bc is not None:
            return bc

    contract = sorted(contract_set, key=in1.index)
    inplace = sorted(inplace_set, key=in1.index)
    inv0 = sorted((seto - common) & set0, key=in0.index)
    inv1 = sorted((seto - common) & set1, key=in1.index)

    inplace_shape = tuple(int(shape0[in0.index(a)]) for a in inplace)
    inv0_shape = tuple(int(shape0[in0.index(a)]) for a in inv0)
    inv1_shape = tuple(int(shape1[in1.index(a)]) for a in inv1)
    I = prod(inplace_shape)
    C = prod(int(shape0[in0.index(a)]) for a in contract)
    L0, L1 = prod(inv0_shape), prod(inv1_shape)

    perm0 = tuple(in0.index(a) for a in inplace + inv0 + contract)
    perm1 = tuple(in1.index(a) for a in inplace + contract + inv1)
    interp_labels = inplace + inv0 + inv1
    positions = [out.index(a) for a in interp_labels]
    out_perm = tuple(sorted(range(len(positions)), key=positions.__getitem__))

    out_identity = out_perm == tuple(range(len(out_perm)))
    fusible = (len(inv0) == 1 and len(inv1) == 1 and out.index(inv1[0]) == len(out) - 1
               and not out_identity)
    if fusible:
        ostr = dict(zip(out, row_major_strides(out_shape)))
        fuse = dict(
            out_fusible=1,
            out_row_stride=int(ostr[inv0[0]]),
            out_n_batch=len(inplace),
            out_batch_sizes=inplace_shape,
            out_batch_strides=tuple(int(ostr[a]) for a in inplace),
        )
    else:
        fuse = dict(NO_FUSE)

    nt = dict(NO_NT)
    single = (os.getenv("EINSUM_DISABLE_NT", "0") == "0" and len(contract) == 1
              and len(inv0) == 1 and len(inv1) == 1 and C % 16 == 0)
    if single:
        a_natural = in0[-1] == contract[0]
        a_transposed = in0[-1] == inv0[0]
        b_nn = in1[-1] == inv1[0]
        nt_mode = a_natural and in1[-1] == contract[0]
        nn_mode = a_natural and not nt_mode and b_nn
        tn_mode = a_transposed and b_nn
        if nt_mode or nn_mode or tn_mode:
            tile = _tile_size()
            mpad, npad = _pad16(L0), _pad16(L1)
            mt, ntl = min(tile, mpad), min(tile, npad)
            # (A zero extent pads to 0; the reference's modulo by that 0,
            # builder.py:318-322, raises.  Such an output is empty and takes
            # the general path.)
            if mt > 0 and ntl > 0 and mpad % mt == 0 and npad % ntl == 0:
                st0 = dict(zip(in0, row_major_strides(shape0)))
                st1 = dict(zip(in1, row_major_strides(shape1)))
                nt = dict(
                    in_nt=1 if nt_mode else (2 if nn_mode else 3),
                    in_n_batch=len(inplace),
                    in0_row_stride=int(st0[inv0[0]]),
                    in0_k_stride=int(st0[contract[0]]),
                    in1_col_stride=int(st1[inv1[0]]),
                    in1_k_stride=int(st1[contract[0]]),
                    in_batch_sizes=inplace_shape,
                    in0_batch_strides=tuple(int(st0[a]) for a in inplace),
                    in1_batch_strides=tuple(int(st1[a]) for a in inplace),
                )

    return dict(
        in_transpose_idxs=(perm0, perm1),
        out_interpret_shape=inplace_shape + inv0_shape + inv1_shape,
        out_transpose_idxs=out_perm,
        out_shape=tuple(out_shape),
        L0=L0, L1=L1, I=I, C=C,
        elementwise=False, n_elem=prod(out_shape),
        **NO_BCAST, **fuse, **nt,
        # Role labels, in recipe order.  Not in the reference recipe; the
        # MI355X launch planner reads them to build strided descriptors.
        roles=dict(inplace=tuple(inplace), contract=tuple(contract),
                   invariant0=tuple(inv0), invariant1=tuple(inv1)),
    )


def plan_operand_order(fn: str, shape0, shape1, device: str = "cuda"):
    """Recipe plus operand-swap decision, as in builder.py:555-586.

    The swap is adopted only when the natural order has a non-identity,
    non-fusible output of a matmul-routed equation and the swapped order makes
    the output fusible or identity.  Returns ``(recipe, swapped, exec_shapes,
    exec_equation)``.
    """
    recipe = parse_recipe(fn, shape0, shape1, device)
    is_matmul = not recipe["elementwise"] and not recipe["broadcast"]
    nat_identity = recipe["out_transpose_idxs"] == tuple(range(len(recipe["out_transpose_idxs"])))
    swap_enabled = os.getenv("EINSUM_DISABLE_OPERAND_SWAP", "0") == "0"
    e0, e1, eo = split_equation(fn)
    if swap_enabled and is_matmul and not recipe["out_fusible"] and not nat_identity:
        swapped_fn = f"{e1},{e0}->{eo}"
        swapped = parse_recipe(swapped_fn, shape1, shape0, device)
        sw_identity = swapped["out_transpose_idxs"] == tuple(range(len(swapped["out_transpose_idxs"])))
        if swapped["out_fusible"] or sw_identity:
            return swapped, True, (tuple(shape1), tuple(shape0)), swapped_fn
    return recipe, False, (tuple(shape0), tuple(shape1)), f"{e0},{e1}->{eo}"


def transpose_config(name: str, shape: Sequence[int], perm: Sequence[int]) -> Dict:
    """Permutation config: ``to_shape = shape[perm]`` and the source stride of
    each destination axis (``perm_strides``), as builder.py:449-461."""
    shape = tuple(int(s) for s in shape)
    perm = tuple(int(p) for p in perm)
    st = row_major_strides(shape)
    return dict(
        config_name=name,
        dims=len(shape),
        N=prod(shape),
        from_shape=shape,
        to_shape=tuple(shape[p] for p in perm),
        perm=perm,
        perm_strides=tuple(st[p] for p in perm),
    )
