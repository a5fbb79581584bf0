"""MI355X launch plan: turn an einsum recipe into kernel descriptors.

The reference executes every contraction as Phase A (operand transposes into
``[I, L0, C]`` / ``[I, C, L1]``), Phase B (GEMM) and Phase C (output
transpose), dropping A or C only for a fixed set of read / store modes
(builder.py:263-346).  Here the GEMM reads each operand at its own strides,
so a phase is only kept when an axis group genuinely does not collapse:

* every role group (free0 = M, free1 = N, contract = K) is flattened to one
  (extent, stride) pair in each tensor that carries it, trying axis orders
  that follow the memory layout;
* batch (inplace) axes stay separate, each with its own stride per tensor;
* a tensor in which some group cannot be flattened is staged in the
  canonical recipe layout -- the operand gathered into the workspace
  (Phase A) or the result written there and permuted into the output
  (Phase C) -- and groups touching a staged tensor use the recipe's axis
  order everywhere.

Contraction-free equations whose every output is a single product (C == 1)
take the product route: one strided stream kernel.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from math import prod
from typing import Dict, List, Optional, Sequence, Tuple

from .planner import row_major_strides, split_equation, transpose_config

ROUTE_PRODUCT = 0
ROUTE_GEMM = 1
MAX_DIMS = 8
DT_F32, DT_F16 = 0, 1


@dataclass
class ProductDesc:
    dtype: int
    add_zero: int
    shape: List[int]
    a_stride: List[int]
    b_stride: List[int]
    a_numel: int
    b_numel: int


@dataclass
class PermuteDesc:
    elem_bytes: int
    shape: List[int]
    src_stride: List[int]
    src_numel: int


@dataclass
class GemmDesc:
    dtype: int
    batch_shape: List[int]
    a_bstride: List[int]
    b_bstride: List[int]
    c_bstride: List[int]
    M: int
    N: int
    K: int
    a_ms: int
    a_ks: int
    b_ks: int
    b_ns: int
    c_ms: int
    c_ns: int
    a_numel: int
    b_numel: int
    c_numel: int
    split_k: int = 0
    tile: int = 0


@dataclass
class LaunchPlan:
    route: int
    product: Optional[ProductDesc] = None
    gemm: Optional[GemmDesc] = None
    gather0: bool = False
    gather1: bool = False
    scatter_out: bool = False
    perm0: Optional[PermuteDesc] = None
    perm1: Optional[PermuteDesc] = None
    perm_out: Optional[PermuteDesc] = None
    ws0_off: int = 0
    ws1_off: int = 0
    wsout_off: int = 0
    ws_bytes: int = 0
    # Component descriptors (run_transpose_inp0/inp1/out, run_batched_matmul).
    comp_perm0: Optional[PermuteDesc] = None
    comp_perm1: Optional[PermuteDesc] = None
    comp_perm_out: Optional[PermuteDesc] = None
    comp_gemm: Optional[GemmDesc] = None
    notes: Dict[str, str] = field(default_factory=dict)


def _align(x: int, a: int = 256) -> int:
    return (x + a - 1) // a * a


def _permute_desc(shape, perm, elem_bytes) -> PermuteDesc:
    cfg = transpose_config("p", shape, perm)
    return PermuteDesc(elem_bytes, list(cfg["to_shape"]), list(cfg["perm_strides"]),
                       max(1, cfg["N"]))


def _mergeable(order: Sequence[str], size: Dict[str, int], stride: Dict[str, int]) -> bool:
    """True when axes ``order`` (outermost first) address like one axis."""
    axes = [a for a in order if size[a] != 1]
    for x, y in zip(axes, axes[1:]):
        if stride[x] != size[y] * stride[y]:
            return False
    return True


def _inner_stride(order: Sequence[str], size: Dict[str, int], stride: Dict[str, int]) -> int:
    axes = [a for a in order if size[a] != 1]
    return stride[axes[-1]] if axes else 0


def _candidate_orders(group: Sequence[str], size, strides: Sequence[Dict[str, int]]):
    seen = []
    for st in strides:
        order = tuple(sorted(group, key=lambda a: (-st[a], group.index(a))))
        if order not in seen:
            seen.append(order)
    if tuple(group) not in seen:
        seen.append(tuple(group))
    return seen


# Smallest extent a free group keeps when its other axes become batch axes.
kMinKeptFree = 16


def _group_order(group: Sequence[str], size, strides: Sequence[Dict[str, int]]):
    """An order of ``group`` that addresses like one axis in every tensor of
    ``strides``, or None."""
    for cand in _candidate_orders(list(group), size, strides):
        if all(_mergeable(cand, size, st) for st in strides):
            return cand
    return None


def _largest_collapsing_subset(group: Sequence[str], size, strides: Sequence[Dict[str, int]], required: str):
    """The subset of ``group`` holding ``required`` with the largest extent
    that collapses in every tensor of ``strides`` (ordered as it collapses),
    or None."""
    from itertools import combinations

    best, best_ext = None, 0
    for r in range(len(group) - 1, 0, -1):
        for sub in combinations(group, r):
            if required not in sub:
                continue
            order = _group_order(sub, size, strides)
            ext = prod(size[a] for a in sub)
            if order is not None and ext > best_ext:
                best, best_ext = order, ext
    return best


def _component_descs(plan: LaunchPlan, recipe: Dict, shape0, shape1, dtype_code: int, elem: int):
    """Descriptors of the staged component entry points: the operand
    permutations into ``[I, L0, C]`` / ``[I, C, L1]``, the canonical batched
    GEMM and the output permutation (reference: templates.py:166-177)."""
    I, L0, L1, C = recipe["I"], recipe["L0"], recipe["L1"], recipe["C"]
    perm0, perm1 = recipe["in_transpose_idxs"]
    plan.comp_perm0 = _permute_desc(shape0, perm0, elem)
    plan.comp_perm1 = _permute_desc(shape1, perm1, elem)
    plan.comp_perm_out = _permute_desc(tuple(recipe["out_interpret_shape"]),
                                       recipe["out_transpose_idxs"], 4)
    batched = I != 1
    plan.comp_gemm = GemmDesc(
        dtype=dtype_code, batch_shape=[I] if batched else [],
        a_bstride=[L0 * C] if batched else [], b_bstride=[C * L1] if batched else [],
        c_bstride=[L0 * L1] if batched else [],
        M=L0, N=L1, K=C, a_ms=C, a_ks=1, b_ks=L1, b_ns=1, c_ms=L1, c_ns=1,
        a_numel=max(1, I * L0 * C), b_numel=max(1, I * C * L1), c_numel=max(1, I * L0 * L1),
        split_k=1)


def plan_launch(recipe: Dict, exec_eq: str, shape0, shape1, dtype_code: int) -> LaunchPlan:
    """Build the launch plan for ``exec_eq`` on operands of ``shape0``/``shape1``
    (already in execution order, i.e. after any operand swap)."""
    t0, t1, to = split_equation(exec_eq)
    shape0, shape1 = tuple(int(s) for s in shape0), tuple(int(s) for s in shape1)
    out_shape = tuple(recipe["out_shape"])
    elem = 4 if dtype_code == DT_F32 else 2
    size: Dict[str, int] = {}
    for t, s in ((t0, shape0), (t1, shape1)):
        size.update({a: int(n) for a, n in zip(t, s)})
    st0 = dict(zip(t0, row_major_strides(shape0)))
    st1 = dict(zip(t1, row_major_strides(shape1)))
    sto = dict(zip(to, row_major_strides(out_shape)))
    numel0, numel1, numelo = max(1, prod(shape0)), max(1, prod(shape1)), max(1, prod(out_shape))

    contract_set = set(t0) & set(t1) - set(to)
    C = prod(size[a] for a in contract_set)
    if C == 1:
        prod_desc = ProductDesc(
            dtype=dtype_code,
            add_zero=0 if recipe["elementwise"] else 1,
            shape=list(out_shape),
            a_stride=[st0.get(a, 0) for a in to],
            b_stride=[st1.get(a, 0) for a in to],
            a_numel=numel0, b_numel=numel1)
        # Drop extent-1 axes so the rank fits the descriptor.
        keep = [i for i, n in enumerate(out_shape) if n != 1]
        prod_desc.shape = [out_shape[i] for i in keep]
        prod_desc.a_stride = [prod_desc.a_stride[i] for i in keep]
        prod_desc.b_stride = [prod_desc.b_stride[i] for i in keep]
        if len(keep) > MAX_DIMS:
            raise ValueError(f"einsum '{exec_eq}': more than {MAX_DIMS} non-unit output axes")
        plan = LaunchPlan(route=ROUTE_PRODUCT, product=prod_desc)
        if not recipe["elementwise"] and not recipe["broadcast"]:
            _component_descs(plan, recipe, shape0, shape1, dtype_code, elem)
        return plan

    roles = recipe["roles"]
    batch = [a for a in roles["inplace"]]
    mgrp = list(roles["invariant0"])
    ngrp = list(roles["invariant1"])
    kgrp = list(roles["contract"])
    # A free group (M or N) that collapses to one stride in neither order of
    # its two tensors keeps its largest subset that does and hands the other
    # axes to the batch: e.g. abc,cd->adb runs as a batch over a of
    # (b, c) x (c, d) GEMMs storing straight into the output, one launch and
    # no workspace.  (A free axis made batch has stride 0 in the tensor that
    # lacks it.)  The kept subset holds the group's axis that is innermost in
    # the output, so the fused store stays coalesced.  Only when no such
    # subset reaches kMinKeptFree elements does the tensor that breaks the
    # group go through the workspace instead.
    for grp, tensors in ((mgrp, (st0, sto)), (ngrp, (st1, sto))):
        if len(grp) < 2 or _group_order(grp, size, tensors) is not None:
            continue
        inner = min((a for a in grp if size[a] != 1), key=lambda a: sto[a], default=grp[-1])
        kept = _largest_collapsing_subset(grp, size, tensors, inner)
        if kept is not None and prod(size[a] for a in kept) >= kMinKeptFree:
            moved = [a for a in grp if a not in kept]
            grp[:] = list(kept)
            batch += moved
    I, L0, L1 = prod(size[a] for a in batch), prod(size[a] for a in mgrp), prod(size[a] for a in ngrp)

    # Staging: a tensor in which some axis group does not collapse is staged
    # in the workspace with its groups contiguous -- [batch, M, K] for A,
    # [batch, K, N] for B, [batch, M, N] for C -- and each group in the order
    # its unstaged partner tensor wants, so only the offending tensor moves.
    natural = {"A": st0, "B": st1, "C": sto}
    staged = {"A": False, "B": False, "C": False}
    groups = (("M", mgrp, ("A", "C")), ("N", ngrp, ("B", "C")), ("K", kgrp, ("A", "B")))

    def own_order(grp, t):
        """An axis order in which ``grp`` collapses in unstaged tensor t, or None."""
        for cand in _candidate_orders(grp, size, [natural[t]]):
            if _mergeable(cand, size, natural[t]):
                return cand
        return None

    orders: Dict[str, Tuple[str, ...]] = {}
    for _ in range(4):
        changed = False
        # (ta, tb: the two tensor names that carry the group; t0 / t1 stay the
        # operands' subscripts, which the layouts below read.)
        for name, grp, (ta, tb) in groups:
            live = [t for t in (ta, tb) if not staged[t]]
            order = None
            if len(live) == 2:
                for cand in _candidate_orders(grp, size, [natural[ta], natural[tb]]):
                    if _mergeable(cand, size, natural[ta]) and _mergeable(cand, size, natural[tb]):
                        order = cand
                        break
                if order is None:
                    # Keep the tensor that can hold the group by itself; stage the
                    # other (output last: staging C costs a full extra pass).
                    keep = tb if (tb == "C" or own_order(grp, ta) is None) and own_order(grp, tb) else ta
                    drop = ta if keep == tb else tb
                    staged[drop] = True
                    changed = True
                    order = own_order(grp, keep)
                    if order is None:
                        staged[keep] = True
                        order = tuple(grp)
            elif len(live) == 1:
                order = own_order(grp, live[0])
                if order is None:
                    staged[live[0]] = True
                    changed = True
                    order = tuple(grp)
            else:
                order = tuple(grp)
            orders[name] = order
        if not changed:
            break

    border = sorted(batch, key=to.index)

    def staged_strides(layout):
        axes = [a for part in layout for a in part]
        return dict(zip(axes, row_major_strides([size[a] for a in axes])))

    # (Batch axes a staged tensor does not carry -- free axes made batch --
    # are left out of its layout.)
    layouts = {"A": ([a for a in border if a in t0], orders["M"], orders["K"]),
               "B": ([a for a in border if a in t1], orders["K"], orders["N"]),
               "C": (border, orders["M"], orders["N"])}
    stage_st = {t: staged_strides(layouts[t]) for t in layouts}

    def strides_of(t):
        return stage_st[t] if staged[t] else natural[t]

    sA, sB, sC = strides_of("A"), strides_of("B"), strides_of("C")
    # Batch axes in output order, extent-1 axes dropped, adjacent axes merged
    # when they compose in all three tensors.
    bax = [a for a in sorted(batch, key=to.index) if size[a] != 1]
    bshape, ba, bb, bc = [], [], [], []
    for a in bax:
        xa, xb, xc = sA.get(a, 0), sB.get(a, 0), sC[a]
        if bshape and ba[-1] == size[a] * xa and bb[-1] == size[a] * xb and bc[-1] == size[a] * xc:
            bshape[-1] *= size[a]
            ba[-1], bb[-1], bc[-1] = xa, xb, xc
        else:
            bshape.append(size[a])
            ba.append(xa)
            bb.append(xb)
            bc.append(xc)
    if len(bshape) > MAX_DIMS:
        raise ValueError(f"einsum '{exec_eq}': more than {MAX_DIMS} independent batch axes")

    gemm = GemmDesc(
        dtype=dtype_code, batch_shape=bshape, a_bstride=ba, b_bstride=bb, c_bstride=bc,
        M=L0, N=L1, K=C,
        a_ms=_inner_stride(orders["M"], size, sA), a_ks=_inner_stride(orders["K"], size, sA),
        b_ks=_inner_stride(orders["K"], size, sB), b_ns=_inner_stride(orders["N"], size, sB),
        c_ms=_inner_stride(orders["M"], size, sC), c_ns=_inner_stride(orders["N"], size, sC),
        a_numel=numel0, b_numel=numel1, c_numel=numelo)

    plan = LaunchPlan(route=ROUTE_GEMM, gemm=gemm, gather0=staged["A"], gather1=staged["B"],
                      scatter_out=staged["C"])
    _component_descs(plan, recipe, shape0, shape1, dtype_code, elem)

    def gather_desc(t, src_strides, eb):
        axes = [a for part in layouts[t] for a in part]
        return PermuteDesc(eb, [size[a] for a in axes], [src_strides[a] for a in axes],
                           max(1, prod(size[a] for a in src_strides)))

    off = 0
    if plan.gather0:
        plan.perm0 = gather_desc("A", st0, elem)
        plan.ws0_off = off
        off = _align(off + numel0 * elem)
    if plan.gather1:
        plan.perm1 = gather_desc("B", st1, elem)
        plan.ws1_off = off
        off = _align(off + numel1 * elem)
    if plan.scatter_out:
        cst = stage_st["C"]
        plan.perm_out = PermuteDesc(4, list(out_shape), [cst[a] for a in to], numelo)
        plan.wsout_off = off
        off = _align(off + numelo * 4)
    plan.ws_bytes = off
    plan.notes = dict(M_order="".join(orders["M"]), N_order="".join(orders["N"]),
                      K_order="".join(orders["K"]))
    return plan
