"""CPU restatements of pe_reduce_axes' documented summation order, for the
bit-exact checks of the reduction kernel (test infrastructure only).

The order, with (V, L, C) as pe_reduce_order reports them: the nterm terms of
an output, row-major over the reduced index, form G = ceil(nterm / V) groups of
V consecutive terms; the groups are cut into C contiguous chunks, the first
G % C one group longer; in a chunk, lane l of L sums groups l, l + L, ... term
by term from +0; the L lane sums, then the C chunk sums, are combined by a
pairwise tree (for s = 1, 2, 4, ...: p[i] = p[i] + p[i + s] for every i that
is a multiple of 2s with i + s in range; the result is p[0]).

Two independent statements: `scalar_ordered_sum` follows the text loop by
loop in Python scalars (small inputs only); `ordered_sum` vectorises it over
outputs, chunks and lanes with numpy for the GPU test sizes.  The CPU tests
check them against each other, against the plain sequential loop (V = L = C
= 1) and against exact integer sums."""
import numpy as np


def _flat(x: np.ndarray, axes):
    keep = [i for i in range(x.ndim) if i not in axes]
    xt = np.transpose(x, keep + list(axes)).astype(np.float32)
    nout = int(np.prod([x.shape[i] for i in keep], dtype=np.int64))
    nterm = int(np.prod([x.shape[i] for i in axes], dtype=np.int64))
    return xt.reshape(nout, nterm), [x.shape[i] for i in keep]


def _chunks(G: int, C: int):
    q, r = divmod(G, C)
    b = np.array([c * q + min(c, r) for c in range(C)], dtype=np.int64)
    e = b + q + (np.arange(C) < r)
    return b, e


def _tree(p: np.ndarray) -> np.ndarray:
    """Pairwise tree over the last axis (float32)."""
    p = p.copy()
    n = p.shape[-1]
    s = 1
    while s < n:
        i = np.arange(0, n - s, 2 * s)
        p[..., i] = p[..., i] + p[..., i + s]
        s *= 2
    return p[..., 0]


def ordered_sum(x: np.ndarray, axes, V: int, L: int, C: int) -> np.ndarray:
    flat, keep_shape = _flat(x, tuple(axes))
    nout, nterm = flat.shape
    if nterm == 0:
        return np.zeros(keep_shape, dtype=np.float32)
    G = -(-nterm // V)
    groups = np.zeros((nout, G * V), dtype=np.float32)
    groups[:, :nterm] = flat          # the padding adds +0: exact
    groups = groups.reshape(nout, G, V)
    b, e = _chunks(G, C)
    lanes = np.zeros((nout, C, L), dtype=np.float32)
    steps = -(-int((e - b).max()) // L)
    for k in range(steps):
        gidx = b[:, None] + np.arange(L)[None, :] + k * L   # (C, L)
        valid = gidx < e[:, None]
        gi = np.where(valid, gidx, 0)
        for v in range(V):
            terms = np.where(valid[None], groups[:, gi, v], np.float32(0.0))
            lanes = lanes + terms
    return _tree(_tree(lanes)).reshape(keep_shape)


def scalar_ordered_sum(x: np.ndarray, axes, V: int, L: int, C: int) -> np.ndarray:
    flat, keep_shape = _flat(x, tuple(axes))
    nout, nterm = flat.shape
    G = -(-nterm // V) if nterm else 0
    q, r = divmod(G, C)
    out = np.zeros(nout, dtype=np.float32)
    for o in range(nout):
        chunk_sums = []
        for c in range(C):
            g0 = c * q + min(c, r)
            g1 = g0 + q + (1 if c < r else 0)
            lane_sums = []
            for lane in range(L):
                acc = np.float32(0.0)
                for g in range(g0 + lane, g1, L):
                    for t in range(g * V, min(g * V + V, nterm)):
                        acc = np.float32(acc + flat[o, t])
                lane_sums.append(acc)
            chunk_sums.append(_scalar_tree(lane_sums))
        out[o] = _scalar_tree(chunk_sums)
    return out.reshape(keep_shape)


def _scalar_tree(p):
    p = list(p)
    s = 1
    while s < len(p):
        for i in range(0, len(p), 2 * s):
            if i + s < len(p):
                p[i] = np.float32(p[i] + p[i + s])
        s *= 2
    return p[0]


def reduce_desc(x, axes):
    """pe_reduce_desc for summing torch tensor x over `axes` (dims kept in order)."""
    from pto_einsum import abi

    keep = [i for i in range(x.dim()) if i not in axes]
    d = abi.ReduceDesc()
    d.dtype = 1 if str(x.dtype) == "torch.float16" else 0
    d.nkeep, d.nred, d.reserved = len(keep), len(axes), 0
    for j, i in enumerate(keep):
        d.keep_shape[j], d.keep_stride[j] = x.shape[i], x.stride(i)
    for j, i in enumerate(axes):
        d.red_shape[j], d.red_stride[j] = x.shape[i], x.stride(i)
    d.src_numel = x.untyped_storage().nbytes() // x.element_size() - x.storage_offset()
    return d
