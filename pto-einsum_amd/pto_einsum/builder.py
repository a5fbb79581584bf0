"""``EinsumBuilder`` and ``einsum``: the reference's public API on MI355X.

Reference: src/pto_einsum/builder.py:112-902.  Same constructor, staged
methods (``parse_equation`` / ``generate_code`` / ``compile`` /
``load_library`` / ``build``), attributes (``recipe``, ``cpp_code``,
``cpp_filename``, ``so_filename``, ``target_dir``, ``lib``), runner checks,
error types and messages, and ``cleanup``.

Devices: ``"cuda"`` (default; ``"npu"``, ``"gpu"`` and ``"hip"`` are aliases,
so code written for the reference runs unchanged) selects the gfx950 path;
``"cpu"`` selects the reference's single-threaded CPU route.  The GPU path
has no CPU fallback: without the built core library or a visible GPU it
raises.
"""
from __future__ import annotations

import collections
import ctypes
import os
import shutil
import threading
from typing import Dict, Optional, Sequence

import torch

from . import codegen, jit, launch, planner, runtime

INCLUDE_DIR = runtime.include_dir()

_GPU_ALIASES = ("cuda", "npu", "gpu", "hip")


def _normalise_device(device) -> str:
    d = str(device)
    if d == "cpu":
        return "cpu"
    base = d.split(":")[0]
    if base in _GPU_ALIASES:
        return "cuda"
    raise ValueError(f"Unsupported device '{device}': use 'cuda' (MI355X) or 'cpu'")


class EinsumBuilder:
    def __init__(self, equation: str, input_shapes: Sequence[Sequence[int]], dtype: torch.dtype,
                 device: str = "cuda"):
        self.equation = equation
        self.input_shapes = input_shapes
        self.dtype = dtype
        self.device = device
        self._route_device = _normalise_device(device)

        self.include_dir = INCLUDE_DIR
        base = os.getenv("EINSUM_BUILD_DIR")
        self.build_base = os.path.abspath(base) if base else os.path.join(os.getcwd(), "build")

        self.recipe: Optional[Dict] = None
        self.cpp_code: Optional[str] = None
        self.cpp_filename: Optional[str] = None
        self.so_filename: Optional[str] = None
        self.lib = None
        self.c_type = None
        self.code_hash: Optional[str] = None
        self.target_dir: Optional[str] = None
        self.launch_plan: Optional[launch.LaunchPlan] = None
        self._workspaces: Dict[int, tuple] = {}   # device -> (workspace tensor, its allocation stream)
        self._swap_operands = False
        self._exec_shapes = tuple(tuple(s) for s in input_shapes)
        self._exec_equation: Optional[str] = None

    # --- planner (builder.py:148-461) -------------------------------------
    def _validate_einsum_expr(self, fn: str, shape0, shape1):
        return planner.validate_expr(fn, shape0, shape1)

    def parse_recipe(self, fn: str, input_shape0, input_shape1) -> Dict:
        return planner.parse_recipe(fn, input_shape0, input_shape1, self._route_device)

    def _try_broadcast(self, in0, in1, out, shape0, shape1, out_shape):
        return planner.try_broadcast(in0, in1, out, shape0, shape1, out_shape, self._route_device)

    def transpose_config_gen(self, name: str, shape, perm) -> Dict:
        return planner.transpose_config(name, shape, perm)

    def parse_equation(self):
        if len(self.input_shapes) != 2:
            raise ValueError("Only exactly two input shapes are supported.")
        shape0, shape1 = (tuple(int(x) for x in s) for s in self.input_shapes)
        recipe, swapped, exec_shapes, exec_eq = planner.plan_operand_order(
            self.equation, shape0, shape1, self._route_device)
        self.recipe = recipe
        self._swap_operands = swapped
        self._exec_shapes = exec_shapes
        self._exec_equation = exec_eq

    # --- codegen / JIT (builder.py:606-736) -------------------------------
    def _dtype_code(self) -> int:
        if self.dtype == torch.float32:
            self.c_type = ctypes.c_float
            return launch.DT_F32
        if self.dtype == torch.float16:
            if self._route_device == "cpu":
                raise TypeError("float16 is not supported on CPU")
            self.c_type = ctypes.c_uint16
            return launch.DT_F16
        raise TypeError(f"Unsupported torch dtype: {self.dtype}")

    def generate_code(self):
        if self.recipe is None:
            self.parse_equation()
        dtype_code = self._dtype_code()
        shapes = [tuple(int(x) for x in s) for s in self.input_shapes]
        if self._route_device == "cpu":
            self.cpp_code = codegen.cpu_source(self.equation, shapes, self.recipe, self._exec_shapes)
        else:
            self.launch_plan = launch.plan_launch(self.recipe, self._exec_equation,
                                                  self._exec_shapes[0], self._exec_shapes[1],
                                                  dtype_code)
            self.cpp_code = codegen.gpu_source(
                self.equation, shapes, "float32" if dtype_code == launch.DT_F32 else "float16",
                self.recipe, self._exec_shapes, self.launch_plan, self._swap_operands)
        self.code_hash = jit.cache_key(self._route_device, self.cpp_code)
        self.target_dir, self.cpp_filename, self.so_filename = jit.paths(self.build_base, self.code_hash)

    def compile(self):
        jit.compile_library(self._route_device, self.cpp_code, self.cpp_filename, self.so_filename)

    def load_library(self):
        if self._route_device != "cpu":
            runtime.core()  # binds the kernels' library (and torch's HIP runtime) first
        self.lib = ctypes.CDLL(self.so_filename)
        cT = ctypes.POINTER(self.c_type)
        cF = ctypes.POINTER(ctypes.c_float)
        vp = ctypes.c_void_p
        if self._route_device == "cpu":
            self.lib.run_einsum.argtypes = [cT, cT, cF, vp]
            self.lib.run_einsum.restype = None
            return
        is_matmul = not self.recipe["elementwise"] and not self.recipe["broadcast"]
        if is_matmul:
            for name in ("run_transpose_inp0", "run_transpose_inp1"):
                fn = getattr(self.lib, name)
                fn.argtypes = [cT, cT, vp]
                fn.restype = ctypes.c_int
            self.lib.run_transpose_out.argtypes = [cF, cF, vp]
            self.lib.run_transpose_out.restype = ctypes.c_int
            self.lib.run_batched_matmul.argtypes = [cT, cT, cF, vp]
            self.lib.run_batched_matmul.restype = ctypes.c_int
        self.lib.run_einsum.argtypes = [cT, cT, cF, vp]
        self.lib.run_einsum.restype = ctypes.c_int
        self.lib.run_einsum_setup.argtypes = [vp]
        self.lib.run_einsum_setup.restype = vp
        self.lib.run_einsum_exec.argtypes = [cT, cT, cF, vp, vp]
        self.lib.run_einsum_exec.restype = ctypes.c_int
        self.lib.run_einsum_teardown.argtypes = [vp]
        self.lib.run_einsum_teardown.restype = None

    # --- lifecycle (builder.py:738-759) ----------------------------------
    def _free_workspaces(self):
        # The runner's workspaces are torch allocations: dropping them returns
        # the memory to torch's stream-ordered caching allocator, which hands
        # it out again only behind the work already queued on the streams
        # that used it (recorded in run()).  No device synchronisation.
        self._workspaces = {}

    def cleanup(self):
        self._free_workspaces()
        self.lib = None
        if self.target_dir and os.path.exists(self.target_dir):
            shutil.rmtree(self.target_dir)

    # --- runner (builder.py:817-884) -------------------------------------
    def _ptr(self, t: torch.Tensor, ctype):
        return ctypes.cast(t.data_ptr(), ctypes.POINTER(ctype))

    def build(self):
        self.parse_equation()
        self.generate_code()
        self.compile()
        self.load_library()
        gpu = self._route_device != "cpu"
        if gpu:
            from . import abi

            self._ws_bytes = int(abi.bind().pe_einsum_workspace_bytes(ctypes.byref(abi.einsum_plan(self.launch_plan))))

        def run(*operands):
            if len(operands) != 2:
                raise ValueError("Expected exactly two operands.")
            inp0, inp1 = operands
            if tuple(inp0.shape) != tuple(self.input_shapes[0]) or \
                    tuple(inp1.shape) != tuple(self.input_shapes[1]):
                raise ValueError(
                    f"Input shapes {inp0.shape} and {inp1.shape} do not match built shapes {self.input_shapes}.")
            if inp0.dtype != self.dtype or inp1.dtype != self.dtype:
                raise TypeError(
                    f"Input datatypes {inp0.dtype} and {inp1.dtype} do not match built datatype {self.dtype}.")
            if gpu:
                if inp0.device.type != "cuda" or inp1.device != inp0.device:
                    raise ValueError(
                        f"Operands must both live on one GPU for device '{self.device}', "
                        f"got {inp0.device} and {inp1.device}.")
            elif inp0.device.type != "cpu" or inp1.device.type != "cpu":
                raise ValueError("Operands must be CPU tensors for device 'cpu'.")
            if not inp0.is_contiguous():
                inp0 = inp0.contiguous()
            if not inp1.is_contiguous():
                inp1 = inp1.contiguous()
            if self._swap_operands:
                inp0, inp1 = inp1, inp0
            out_shape = self.recipe["out_shape"]
            if not gpu:
                out = torch.zeros(out_shape, dtype=torch.float32, device="cpu")
                self.lib.run_einsum(self._ptr(inp0, self.c_type), self._ptr(inp1, self.c_type),
                                    self._ptr(out, ctypes.c_float), None)
                return out
            dev = inp0.device
            with torch.cuda.device(dev):
                out = torch.empty(out_shape, dtype=torch.float32, device=dev)
                stream = runtime.current_stream_ptr(dev)
                idx = dev.index if dev.index is not None else torch.cuda.current_device()
                # Workspace (split-K partials, staged operands): a torch
                # allocation per device, so creating it is stream-ordered and
                # allowed under graph capture, and dropping it needs no
                # synchronisation.  A use on another stream than the one it
                # was allocated on is recorded, so the allocator does not
                # reuse the memory before that stream's work is done.
                entry = self._workspaces.get(idx)
                if entry is None:
                    entry = (torch.empty(self._ws_bytes, dtype=torch.uint8, device=dev), stream)
                    self._workspaces[idx] = entry
                elif entry[1] != stream:
                    entry[0].record_stream(torch.cuda.current_stream(dev))
                rc = self.lib.run_einsum_exec(self._ptr(inp0, self.c_type), self._ptr(inp1, self.c_type),
                                              self._ptr(out, ctypes.c_float), ctypes.c_void_p(entry[0].data_ptr()),
                                              stream)
                runtime.check(rc, "run_einsum_exec")
            return out

        return run


_RUNNER_CACHE_SIZE = 64
_runners: "collections.OrderedDict" = collections.OrderedDict()
_runners_lock = threading.Lock()
# Runners handed out while a StageGraph captures: the graph keeps them (and so
# their workspaces, which its replays read and write) alive after the cache
# evicts them.  None outside a capture.
_capture_pins: Optional[list] = None


def _reduce_operand(x: torch.Tensor, subs: str, solo: str) -> torch.Tensor:
    """Sum x over the axes named in `solo` (pe_reduce_axes): a contiguous
    float32 tensor over the other axes, in their order in `subs`.  With no
    solo axis, x converted to float32."""
    from . import abi

    keep = [i for i, a in enumerate(subs) if a not in solo]
    red = [i for i, a in enumerate(subs) if a in solo]
    d = abi.ReduceDesc()
    d.dtype = 1 if x.dtype == torch.float16 else 0
    d.nkeep, d.nred, d.reserved = len(keep), len(red), 0
    for j, i in enumerate(keep):
        d.keep_shape[j], d.keep_stride[j] = x.shape[i], x.stride(i)
    for j, i in enumerate(red):
        d.red_shape[j], d.red_stride[j] = x.shape[i], x.stride(i)
    d.src_numel = x.untyped_storage().nbytes() // x.element_size() - x.storage_offset()
    out = torch.empty([x.shape[i] for i in keep], dtype=torch.float32, device=x.device)
    lib = abi.bind()
    ws_bytes = int(lib.pe_reduce_workspace_bytes(ctypes.byref(d)))
    # Chunk sums of the two-pass order: stream-ordered, freed with the tensor.
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    with torch.cuda.device(x.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        rc = lib.pe_reduce_axes(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                ctypes.c_void_p(ws.data_ptr() if ws is not None else None), ws_bytes, stream)
    runtime.check(rc, "pe_reduce_axes")
    return out


def _reduce_solo_axes(equation: str, inp0: torch.Tensor, inp1: torch.Tensor):
    """Sums every single-operand reduction axis (an index in one operand only
    and not in the output, e.g. i in ``ij,jk->k``) out of its operand, as
    torch.einsum does, and returns the remaining two-operand equation with
    its operands.  The reference rejects such equations (builder.py:218-229);
    this is the reduction stage its roadmap describes (IMPLEMENTATION.md:
    812-821).  The reduced operand is float32; a float16 partner is converted
    to float32 too, since both operands of the contraction share a dtype."""
    reduced, in0, in1, solo0, solo1 = planner.solo_split(equation, inp0.shape, inp1.shape)
    if not solo0 and not solo1:
        return equation, inp0, inp1
    if not (inp0.is_cuda and inp1.is_cuda):
        raise ValueError("einsum: reduce_solo_axes needs both operands on the GPU")
    if inp0.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"Unsupported torch dtype {inp0.dtype}")
    r0 = _reduce_operand(inp0, in0, solo0) if solo0 or inp0.dtype != torch.float32 else inp0
    r1 = _reduce_operand(inp1, in1, solo1) if solo1 or inp1.dtype != torch.float32 else inp1
    return reduced, r0, r1


def einsum(equation: str, *operands, device: str = "cuda", reduce_solo_axes: bool = False):
    """One-shot einsum of two operands; returns a float32 tensor.

    Reference: builder.py:887-902.  Runners are cached in-process by
    (equation, shapes, dtype, device), so a repeated call reuses the loaded
    library and workspace instead of re-planning and re-loading.

    ``reduce_solo_axes`` (keyword only, off by default, no counterpart in the
    reference): an index found in one operand only and not in the output is
    summed out of that operand on the GPU first, as torch.einsum does
    (e.g. ``ij,jk->k``); the result is computed in float32.  Off, such
    equations raise the reference's ValueError.
    """
    if len(operands) != 2:
        raise ValueError("Only exactly two operands are supported.")
    inp0, inp1 = operands
    if inp0.dtype != inp1.dtype:
        raise ValueError("Operands must have the same datatype.")
    if reduce_solo_axes:
        equation, inp0, inp1 = _reduce_solo_axes(equation, inp0, inp1)
    key = (equation, tuple(inp0.shape), tuple(inp1.shape), inp0.dtype, _normalise_device(device),
           os.getenv("EINSUM_BUILD_DIR", ""), os.getenv("EINSUM_EXTRA_DEFINES", ""))
    with _runners_lock:
        entry = _runners.get(key)
        if entry is not None:
            _runners.move_to_end(key)
    if entry is None:
        builder = EinsumBuilder(equation, [inp0.shape, inp1.shape], inp0.dtype, device=device)
        entry = (builder, builder.build())
        with _runners_lock:
            _runners[key] = entry
    with _runners_lock:
        # No eviction while a graph is being captured: a runner used earlier
        # in the capture must keep its workspace, which the graph reads at
        # every replay.  The cache shrinks back at the first call after it.
        if len(_runners) > _RUNNER_CACHE_SIZE and not _capturing():
            while len(_runners) > _RUNNER_CACHE_SIZE:
                _runners.popitem(last=False)
        if _capture_pins is not None:
            _capture_pins.append(entry)
    return entry[1](inp0, inp1)


def _capturing() -> bool:
    try:
        return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    except Exception:
        return False


def clear_runner_cache():
    """Drop every cached one-shot runner (and with it their workspaces)."""
    with _runners_lock:
        _runners.clear()
