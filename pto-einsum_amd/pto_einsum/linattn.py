"""Fused linear-attention chain on the GPU.

``linear_attention(q, k, v, m)`` computes

    out[t, p] = sum_s ((sum_n q[t, n] * k[s, n]) * m[t, s]) * v[s, p]

in one kernel launch.  The reference runs the same chain as three two-operand
einsums with float32 intermediates (tests/test_llm_ops.py:81-107,
benchmarks/complex/bench_linear_attention.py:62-94)::

    A = einsum("tn,sn->ts", q, k)
    A = einsum("ts,ts->ts", A, m)
    out = einsum("ts,sp->tp", A, v)

which writes and re-reads two T x S float32 intermediates; the fused kernel
keeps them in registers.  Results follow that chain's float32 arithmetic (every
operand up-cast exactly, the inner sum and the mask product rounded to
float32); sums are taken in a different order, so agreement is to contraction
tolerance, not bit for bit.

The last product P.V (P = the masked scores) runs by default on bfloat16
matrix cores at float32 accuracy: P is split into three bfloat16 terms and V
into two (float16, exact) or three (float32), each term the bfloat16 nearest
to what the previous ones left (round to nearest even; the remainders are
exact in float32), and P.V is the sum of the term products Pi.Vj with
i + j <= 2 -- products exact, sums float32.  What is left out is below
2^-22 |P||V| per product, the scale of float32's own rounding.
``precise=True`` runs P.V on float32 matrix cores instead (about three times
the MFMA time of that product).
"""
from __future__ import annotations

import ctypes

import torch

from . import abi, launch, runtime

_DT = {torch.float32: launch.DT_F32, torch.float16: launch.DT_F16}


def _extent(t: torch.Tensor) -> int:
    """Elements addressable from t's first element to the end of its storage."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def _rows(t: torch.Tensor) -> torch.Tensor:
    """Rows contiguous from a 16-byte aligned base (what the workspace size
    query assumes); strided rows are fine."""
    ok = t.stride(1) == 1 and t.stride(0) >= t.shape[1] and t.data_ptr() % 16 == 0
    return t if ok or t.numel() == 0 else t.contiguous()


def linear_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, m: torch.Tensor,
                     *, split: int = 0, precise: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused ``einsum("tn,sn,sp,ts->tp", q, k, v, m)``; returns a float32
    [T, P] tensor on the operands' GPU.

    q [T, N] and k [S, N] share a dtype (float16 or float32; N <= 256 for
    float16, N <= 128 for float32); v [S, P] and m [T, S] are float16 or
    float32.  ``split`` forces the number of s splits (0 = choose);
    ``precise`` computes P.V on float32 matrix cores instead of the split
    bfloat16 terms.  ``out``: a contiguous float32 [T, P] tensor on the same
    GPU to write into (else a new one is returned)."""
    for name, t in (("q", q), ("k", k), ("v", v), ("m", m)):
        if t.dim() != 2:
            raise ValueError(f"linear_attention: {name} must be 2-D, got shape {tuple(t.shape)}")
        if t.dtype not in _DT:
            raise TypeError(f"linear_attention: unsupported dtype {t.dtype} for {name}")
    if q.dtype != k.dtype:
        raise TypeError(f"linear_attention: q and k must share a dtype, got {q.dtype} and {k.dtype}")
    T, N = q.shape
    S, P = v.shape
    if tuple(k.shape) != (S, N) or tuple(m.shape) != (T, S):
        raise ValueError(f"linear_attention: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} "
                         f"m{tuple(m.shape)} do not form tn,sn,sp,ts->tp")
    dev = q.device
    if dev.type != "cuda" or any(t.device != dev for t in (k, v, m)):
        raise ValueError("linear_attention: operands must all live on one GPU")
    q, k, v, m = (_rows(t) for t in (q, k, v, m))
    if out is not None and (out.dtype != torch.float32 or tuple(out.shape) != (T, P) or out.device != dev
                            or not out.is_contiguous()):
        raise ValueError(f"linear_attention: out must be a contiguous float32 tensor of shape {(T, P)} on {dev}")

    d = abi.LinAttnDesc()
    d.qk_dtype, d.v_dtype, d.m_dtype, d.split = _DT[q.dtype], _DT[v.dtype], _DT[m.dtype], int(split)
    d.precise = 1 if precise else 0
    d.T, d.S, d.N, d.P = T, S, N, P
    d.q_ts, d.k_ss, d.v_ss, d.m_ts = q.stride(0), k.stride(0), v.stride(0), m.stride(0)
    d.q_numel, d.k_numel, d.v_numel, d.m_numel = (_extent(t) for t in (q, k, v, m))
    lib = abi.bind()
    with torch.cuda.device(dev):
        if out is None:
            out = torch.empty((T, P), dtype=torch.float32, device=dev)
        ws_bytes = lib.pe_linear_attention_workspace_bytes(ctypes.byref(d))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        rc = lib.pe_linear_attention(ctypes.byref(d), ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()),
                                     ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(m.data_ptr()),
                                     ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ws_bytes,
                                     runtime.current_stream_ptr(dev))
        runtime.check(rc, "pe_linear_attention")
    return out
