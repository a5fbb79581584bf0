"""Seeded random two-operand einsums for the planner and parity sweeps (test
infrastructure only).

Each equation mixes the four axis roles of the GEMM route -- batch (both
inputs and the output), free0 / free1 (one input and the output) and
contracted (both inputs) -- with random counts, sizes and axis orders in
every tensor, so groups collapse in some tensors and not in others and the
planner's staging, promotion and batch-merging choices are all reached.
With ``solo=True`` some equations also carry single-operand reduction axes
(an input-0 axis in neither the other input nor the output)."""
import random
from math import prod

SIZES = [1, 2, 3, 5, 7, 8, 16, 17, 31, 32, 33, 64, 100, 128, 130, 257]
EMPTY_SIZES = [0, 0, 1, 2, 3, 5, 17, 33, 64]  # with zero extents: empty outputs and empty sums
LETTERS = "abcdefghijklmnopqrstuvwxyzABCDEF"


def random_case(rng: random.Random, solo: bool = False, max_elems: float = 3e6, max_work: float = 1.5e8,
                sizes=SIZES):
    """(equation, shape0, shape1, has_solo_axes), axis extents drawn from
    ``sizes``."""
    while True:
        nb = rng.choice([0, 0, 1, 2])
        nf0, nf1, nc = (rng.choice([0, 1, 1, 2, 3]) for _ in range(3))
        ns0 = rng.choice([1, 2]) if solo and rng.random() < 0.15 else 0
        n = nb + nf0 + nf1 + nc + ns0
        if n == 0 or n > 7:
            continue
        it = iter(rng.sample(LETTERS, n))
        bat = [next(it) for _ in range(nb)]
        f0 = [next(it) for _ in range(nf0)]
        f1 = [next(it) for _ in range(nf1)]
        con = [next(it) for _ in range(nc)]
        s0 = [next(it) for _ in range(ns0)]
        in0, in1, out = bat + f0 + con + s0, bat + f1 + con, bat + f0 + f1
        if not in0 or not in1 or not out:
            continue
        rng.shuffle(in0)
        rng.shuffle(in1)
        rng.shuffle(out)
        size = {a: rng.choice(sizes) for a in in0 + in1}
        n0, n1, no = (prod(size[a] for a in t) for t in (in0, in1, out))
        work = no * prod(size[a] for a in con) * prod(size[a] for a in s0)
        if max(n0, n1) > max_elems or no > max_elems or work > max_work:
            continue
        eq = "".join(in0) + "," + "".join(in1) + "->" + "".join(out)
        return eq, tuple(size[a] for a in in0), tuple(size[a] for a in in1), bool(s0)
