"""pto_einsum for AMD Instinct MI355X (gfx950).

Public API, unchanged from the reference (src/pto_einsum/__init__.py:12-15):

    einsum(equation, a, b, device="cuda")   -> float32 result tensor
    EinsumBuilder(equation, shapes, dtype)  -> reusable compiled runner
    INCLUDE_DIR                             -> headers the JIT sources compile against

Beyond the reference's surface:

    einsum(eq, a, b, reduce_solo_axes=True) -> also sums indices found in one operand
                                               only (e.g. "ij,jk->k"), which the
                                               reference rejects
    linear_attention(q, k, v, m)            -> fused einsum("tn,sn,sp,ts->tp"), float32
    StageGraph(fn)                          -> fn's launches captured into one HIP graph

Example:
    >>> from pto_einsum import einsum
    >>> c = einsum("ij, jk -> ik", a, b)    # a, b are tensors on the GPU
"""

from .builder import EinsumBuilder, INCLUDE_DIR, einsum
from .graph import StageGraph
from .linattn import linear_attention

__all__ = ["einsum", "EinsumBuilder", "INCLUDE_DIR", "linear_attention", "StageGraph"]
__version__ = "0.2.0"
