"""ctypes mirrors of the core library's C structs (include/pto_einsum_hip.h).

Lets Python callers (and the component tests) drive the core launchers
directly: ``pe_product``, ``pe_permute``, ``pe_gemm``, ``pe_linear_attention``,
``pe_reduce_axes`` and the plan executor.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

from . import launch, runtime

MAX_DIMS = 8
_I64x8 = ctypes.c_int64 * MAX_DIMS


class ProductDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("add_zero", ctypes.c_int32),
                ("ndims", ctypes.c_int32), ("_pad", ctypes.c_int32),
                ("shape", _I64x8), ("a_stride", _I64x8), ("b_stride", _I64x8),
                ("a_numel", ctypes.c_int64), ("b_numel", ctypes.c_int64)]


class PermuteDesc(ctypes.Structure):
    _fields_ = [("elem_bytes", ctypes.c_int32), ("ndims", ctypes.c_int32),
                ("shape", _I64x8), ("src_stride", _I64x8), ("src_numel", ctypes.c_int64)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("nbatch", ctypes.c_int32),
                ("split_k", ctypes.c_int32), ("tile", ctypes.c_int32),
                ("batch_shape", _I64x8), ("a_bstride", _I64x8), ("b_bstride", _I64x8),
                ("c_bstride", _I64x8),
                ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("a_ms", ctypes.c_int64), ("a_ks", ctypes.c_int64), ("b_ks", ctypes.c_int64),
                ("b_ns", ctypes.c_int64), ("c_ms", ctypes.c_int64), ("c_ns", ctypes.c_int64),
                ("a_numel", ctypes.c_int64), ("b_numel", ctypes.c_int64), ("c_numel", ctypes.c_int64)]


class EinsumPlan(ctypes.Structure):
    _fields_ = [("route", ctypes.c_int32), ("gather0", ctypes.c_int32), ("gather1", ctypes.c_int32),
                ("scatter_out", ctypes.c_int32),
                ("product", ProductDesc), ("perm0", PermuteDesc), ("perm1", PermuteDesc),
                ("perm_out", PermuteDesc), ("gemm", GemmDesc),
                ("ws0_off", ctypes.c_int64), ("ws1_off", ctypes.c_int64),
                ("wsout_off", ctypes.c_int64), ("wsgemm_off", ctypes.c_int64),
                ("ws_bytes", ctypes.c_int64), ("skip_phases", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class LinAttnDesc(ctypes.Structure):
    _fields_ = [("qk_dtype", ctypes.c_int32), ("v_dtype", ctypes.c_int32), ("m_dtype", ctypes.c_int32),
                ("split", ctypes.c_int32),
                ("T", ctypes.c_int64), ("S", ctypes.c_int64), ("N", ctypes.c_int64), ("P", ctypes.c_int64),
                ("q_ts", ctypes.c_int64), ("k_ss", ctypes.c_int64), ("v_ss", ctypes.c_int64),
                ("m_ts", ctypes.c_int64),
                ("q_numel", ctypes.c_int64), ("k_numel", ctypes.c_int64), ("v_numel", ctypes.c_int64),
                ("m_numel", ctypes.c_int64), ("precise", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class ReduceDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("nkeep", ctypes.c_int32), ("nred", ctypes.c_int32),
                ("reserved", ctypes.c_int32),
                ("keep_shape", _I64x8), ("keep_stride", _I64x8), ("red_shape", _I64x8), ("red_stride", _I64x8),
                ("src_numel", ctypes.c_int64)]


def _set(arr, values: Sequence[int]):
    for i, v in enumerate(values):
        arr[i] = int(v)


def permute_desc(d: launch.PermuteDesc) -> PermuteDesc:
    c = PermuteDesc()
    c.elem_bytes, c.ndims, c.src_numel = d.elem_bytes, len(d.shape), d.src_numel
    _set(c.shape, d.shape)
    _set(c.src_stride, d.src_stride)
    return c


def gemm_desc(d: launch.GemmDesc) -> GemmDesc:
    c = GemmDesc()
    c.dtype, c.nbatch, c.split_k, c.tile = d.dtype, len(d.batch_shape), d.split_k, d.tile
    _set(c.batch_shape, d.batch_shape)
    _set(c.a_bstride, d.a_bstride)
    _set(c.b_bstride, d.b_bstride)
    _set(c.c_bstride, d.c_bstride)
    for f in ("M", "N", "K", "a_ms", "a_ks", "b_ks", "b_ns", "c_ms", "c_ns", "a_numel", "b_numel", "c_numel"):
        setattr(c, f, int(getattr(d, f)))
    return c


def product_desc(d: launch.ProductDesc) -> ProductDesc:
    c = ProductDesc()
    c.dtype, c.add_zero, c.ndims = d.dtype, d.add_zero, len(d.shape)
    _set(c.shape, d.shape)
    _set(c.a_stride, d.a_stride)
    _set(c.b_stride, d.b_stride)
    c.a_numel, c.b_numel = d.a_numel, d.b_numel
    return c


def einsum_plan(p: launch.LaunchPlan) -> EinsumPlan:
    """The ``pe_einsum_plan`` of a launch plan (the struct the generated
    per-shape sources fill in, built here for direct calls)."""
    c = EinsumPlan()
    c.route = p.route
    if p.route == launch.ROUTE_PRODUCT:
        c.product = product_desc(p.product)
        return c
    c.gather0, c.gather1, c.scatter_out = int(p.gather0), int(p.gather1), int(p.scatter_out)
    c.gemm = gemm_desc(p.gemm)
    if p.gather0:
        c.perm0 = permute_desc(p.perm0)
    if p.gather1:
        c.perm1 = permute_desc(p.perm1)
    if p.scatter_out:
        c.perm_out = permute_desc(p.perm_out)
    c.ws0_off, c.ws1_off, c.wsout_off, c.ws_bytes = p.ws0_off, p.ws1_off, p.wsout_off, p.ws_bytes
    return c


def bind(lib=None):
    """Set argtypes/restypes of the core launchers on the loaded core library."""
    lib = lib or runtime.core()
    vp = ctypes.c_void_p
    lib.pe_product.argtypes = [ctypes.POINTER(ProductDesc), vp, vp, vp, vp]
    lib.pe_permute.argtypes = [ctypes.POINTER(PermuteDesc), vp, vp, vp]
    lib.pe_gemm.argtypes = [ctypes.POINTER(GemmDesc), vp, vp, vp, vp, ctypes.c_int64, vp]
    lib.pe_gemm_workspace_bytes.argtypes = [ctypes.POINTER(GemmDesc)]
    lib.pe_gemm_workspace_bytes.restype = ctypes.c_int64
    lib.pe_gemm_choice.argtypes = [ctypes.POINTER(GemmDesc), ctypes.POINTER(ctypes.c_int64)]
    lib.pe_einsum_exec.argtypes = [ctypes.POINTER(EinsumPlan), vp, vp, vp, vp, vp]
    lib.pe_einsum_workspace_bytes.argtypes = [ctypes.POINTER(EinsumPlan)]
    lib.pe_einsum_workspace_bytes.restype = ctypes.c_int64
    lib.pe_einsum_setup.argtypes = [ctypes.POINTER(EinsumPlan), vp]
    lib.pe_einsum_setup.restype = vp
    lib.pe_einsum_teardown.argtypes = [vp]
    lib.pe_einsum_run.argtypes = [ctypes.POINTER(EinsumPlan), vp, vp, vp, vp]
    lib.pe_einsum_exec_noalloc.argtypes = [ctypes.POINTER(EinsumPlan), vp, vp, vp, vp]
    lib.pe_linear_attention.argtypes = [ctypes.POINTER(LinAttnDesc), vp, vp, vp, vp, vp, vp, ctypes.c_int64, vp]
    lib.pe_linear_attention_workspace_bytes.argtypes = [ctypes.POINTER(LinAttnDesc)]
    lib.pe_linear_attention_workspace_bytes.restype = ctypes.c_int64
    lib.pe_reduce_axes.argtypes = [ctypes.POINTER(ReduceDesc), vp, vp, vp, ctypes.c_int64, vp]
    lib.pe_reduce_workspace_bytes.argtypes = [ctypes.POINTER(ReduceDesc)]
    lib.pe_reduce_workspace_bytes.restype = ctypes.c_int64
    lib.pe_reduce_order.argtypes = [ctypes.POINTER(ReduceDesc), vp, ctypes.POINTER(ctypes.c_int64)]
    lib.pe_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, vp, ctypes.c_int64, vp]
    lib.pe_probe_mfma_flops.argtypes = [ctypes.c_int, ctypes.c_int64]
    lib.pe_probe_mfma_flops.restype = ctypes.c_int64
    lib.pe_probe_out_len.restype = ctypes.c_int64
    lib.pe_probe_launch.argtypes = [vp, vp]
    for f in ("pe_product", "pe_permute", "pe_gemm", "pe_einsum_exec", "pe_einsum_teardown", "pe_einsum_run", "pe_probe_mfma", "pe_probe_launch", "pe_gemm_choice",
              "pe_einsum_exec_noalloc", "pe_linear_attention", "pe_reduce_axes", "pe_reduce_order"):
        getattr(lib, f).restype = ctypes.c_int
    return lib
