"""Source generation for the per-shape JIT libraries.

Reference counterparts: the config-struct and wrapper templates of
templates.py:1-191 filled by generate_code (builder.py:606-683).

A generated source holds

* the reference's configuration structs -- ``config_tpose_inp0/inp1/out``
  (templates.py:1-9) and ``config_einsum`` with the recipe fields of
  templates.py:11-62, so callers that inspect ``cpp_code`` for a path gate
  (``in_nt = 1``, ``out_fusible = 1``) see what the reference would emit;
* the MI355X launch plan as a ``pe_einsum_plan`` built from those values;
* the ``extern "C"`` entry points of the reference ABI, which hand the plan to
  the core library (libpto_einsum_hip.so) where the gfx950 kernels live.

The GPU source includes only the plain-C header ``pto_einsum_hip.h`` and is
compiled as host code: the device code of every kernel is built once for
gfx950 by the core library build, so a new shape costs a sub-second host
compile instead of a device compile.

The CPU route (``device="cpu"``) generates the reference's CPU wrapper shape
(templates.py:131-156) around ``pto_einsum_cpu.h``.
"""
from __future__ import annotations

from math import prod
from typing import Dict, Sequence

from . import launch as L
from .planner import transpose_config

CTYPE = {L.DT_F32: "float", L.DT_F16: "uint16_t"}


def _arr(xs: Sequence[int]) -> str:
    xs = list(xs) or [0]
    return ", ".join(str(int(x)) for x in xs)


def tconfig_struct(cfg: Dict) -> str:
    dims = max(1, cfg["dims"])
    return (
        f"struct {cfg['config_name']} {{\n"
        f"    static constexpr unsigned dims = {cfg['dims']};\n"
        f"    static constexpr unsigned long long N = {cfg['N']};\n"
        f"    static constexpr unsigned long long from_shape[{dims}] = {{{_arr(cfg['from_shape'])}}};\n"
        f"    static constexpr unsigned long long to_shape[{dims}] = {{{_arr(cfg['to_shape'])}}};\n"
        f"    static constexpr unsigned perm[{dims}] = {{{_arr(cfg['perm'])}}};\n"
        f"    static constexpr unsigned long long perm_strides[{dims}] = {{{_arr(cfg['perm_strides'])}}};\n"
        f"}};\n")


def einsum_struct(r: Dict) -> str:
    nb = max(1, len(r["out_batch_sizes"]))
    nib = max(1, len(r["in_batch_sizes"]))
    return (
        "struct config_einsum {\n"
        "    typedef config_tpose_inp0 tpose_inp0_config;\n"
        "    typedef config_tpose_inp1 tpose_inp1_config;\n"
        "    typedef config_tpose_out tpose_out_conf;\n"
        f"    static const unsigned long long n_free0 = {r['L0']};\n"
        f"    static const unsigned long long n_free1 = {r['L1']};\n"
        f"    static const unsigned long long n_contract = {r['C']};\n"
        f"    static const unsigned long long n_inplace = {r['I']};\n"
        f"    static constexpr unsigned out_fusible = {r['out_fusible']};\n"
        f"    static constexpr unsigned long long out_row_stride = {r['out_row_stride']};\n"
        f"    static constexpr unsigned out_n_batch = {r['out_n_batch']};\n"
        f"    static constexpr unsigned long long out_batch_sizes[{nb}] = {{{_arr(r['out_batch_sizes'])}}};\n"
        f"    static constexpr unsigned long long out_batch_strides[{nb}] = {{{_arr(r['out_batch_strides'])}}};\n"
        f"    static constexpr unsigned in_nt = {r['in_nt']};\n"
        f"    static constexpr unsigned in_n_batch = {r['in_n_batch']};\n"
        f"    static constexpr unsigned long long in0_row_stride = {r['in0_row_stride']};\n"
        f"    static constexpr unsigned long long in0_k_stride = {r['in0_k_stride']};\n"
        f"    static constexpr unsigned long long in1_col_stride = {r['in1_col_stride']};\n"
        f"    static constexpr unsigned long long in1_k_stride = {r['in1_k_stride']};\n"
        f"    static constexpr unsigned long long in_batch_sizes[{nib}] = {{{_arr(r['in_batch_sizes'])}}};\n"
        f"    static constexpr unsigned long long in0_batch_strides[{nib}] = {{{_arr(r['in0_batch_strides'])}}};\n"
        f"    static constexpr unsigned long long in1_batch_strides[{nib}] = {{{_arr(r['in1_batch_strides'])}}};\n"
        "};\n")


def _fill(var: str, obj, fields: Sequence[str]) -> str:
    lines = []
    for f in fields:
        v = getattr(obj, f)
        if isinstance(v, (list, tuple)):
            for i, x in enumerate(v):
                lines.append(f"    {var}.{f}[{i}] = {int(x)}LL;")
        else:
            lines.append(f"    {var}.{f} = {int(v)}LL;")
    return "\n".join(lines)


def _permute_fill(var: str, d: L.PermuteDesc) -> str:
    return "\n".join([
        f"    {var}.elem_bytes = {d.elem_bytes};",
        f"    {var}.ndims = {len(d.shape)};",
        _fill(var, d, ("shape", "src_stride", "src_numel")),
    ])


def _gemm_fill(var: str, d: L.GemmDesc) -> str:
    return "\n".join([
        f"    {var}.dtype = {d.dtype};",
        f"    {var}.nbatch = {len(d.batch_shape)};",
        f"    {var}.split_k = {d.split_k};",
        f"    {var}.tile = {d.tile};",
        _fill(var, d, ("batch_shape", "a_bstride", "b_bstride", "c_bstride", "M", "N", "K",
                       "a_ms", "a_ks", "b_ks", "b_ns", "c_ms", "c_ns", "a_numel", "b_numel",
                       "c_numel")),
    ])


def _product_fill(var: str, d: L.ProductDesc) -> str:
    return "\n".join([
        f"    {var}.dtype = {d.dtype};",
        f"    {var}.add_zero = {d.add_zero};",
        f"    {var}.ndims = {len(d.shape)};",
        _fill(var, d, ("shape", "a_stride", "b_stride", "a_numel", "b_numel")),
    ])


def plan_function(plan: L.LaunchPlan) -> str:
    body = ["static pe_einsum_plan make_plan() {", "    pe_einsum_plan p;",
            "    memset(&p, 0, sizeof(p));", f"    p.route = {plan.route};"]
    if plan.route == L.ROUTE_PRODUCT:
        body.append(_product_fill("p.product", plan.product))
    else:
        body += [f"    p.gather0 = {int(plan.gather0)};", f"    p.gather1 = {int(plan.gather1)};",
                 f"    p.scatter_out = {int(plan.scatter_out)};",
                 _gemm_fill("p.gemm", plan.gemm)]
        if plan.gather0:
            body.append(_permute_fill("p.perm0", plan.perm0))
        if plan.gather1:
            body.append(_permute_fill("p.perm1", plan.perm1))
        if plan.scatter_out:
            body.append(_permute_fill("p.perm_out", plan.perm_out))
        body += [f"    p.ws0_off = {plan.ws0_off}LL;", f"    p.ws1_off = {plan.ws1_off}LL;",
                 f"    p.wsout_off = {plan.wsout_off}LL;", f"    p.ws_bytes = {plan.ws_bytes}LL;"]
    body += ["    p.skip_phases = (EINSUM_PHASE_STOP < 1 ? 1 : 0) | (EINSUM_PHASE_STOP < 2 ? 2 : 0) |",
             "                    (EINSUM_PHASE_STOP < 3 ? 4 : 0);",
             "    return p;", "}", "static const pe_einsum_plan kPlan = make_plan();", ""]
    return "\n".join(body)


def component_functions(plan: L.LaunchPlan) -> str:
    out = []
    for name, d in (("kPerm0", plan.comp_perm0), ("kPerm1", plan.comp_perm1),
                    ("kPermOut", plan.comp_perm_out)):
        out += [f"static pe_permute_desc make_{name}() {{", "    pe_permute_desc d;",
                "    memset(&d, 0, sizeof(d));", _permute_fill("d", d), "    return d;", "}",
                f"static const pe_permute_desc {name} = make_{name}();", ""]
    out += ["static pe_gemm_desc make_kCanonGemm() {", "    pe_gemm_desc d;",
            "    memset(&d, 0, sizeof(d));", _gemm_fill("d", plan.comp_gemm), "    return d;", "}",
            "static const pe_gemm_desc kCanonGemm = make_kCanonGemm();", ""]
    return "\n".join(out)


def gpu_source(equation: str, shapes, dtype_name: str, recipe: Dict, exec_shapes,
               plan: L.LaunchPlan, swapped: bool) -> str:
    """The per-shape GPU wrapper source (reference: templates.py:74-92,
    111-129, 158-191)."""
    T = CTYPE[L.DT_F32 if dtype_name == "float32" else L.DT_F16]
    head = [
        f"// pto_einsum JIT source: {equation} {tuple(shapes[0])} x {tuple(shapes[1])} {dtype_name}",
        f"// execution order: {'swapped' if swapped else 'natural'} operands {tuple(exec_shapes[0])} x {tuple(exec_shapes[1])}",
        "#define PE_NO_PER_SHAPE_DECLS",
        '#include "pto_einsum_hip.h"',
        "#include <string.h>",
        "",
        "// Phase ablation (EINSUM_EXTRA_DEFINES=-DEINSUM_PHASE_STOP=N): phases after",
        "// the N-th launch nothing (0: none, 1: operand gathers, 2: + GEMM, 3: all).",
        "#ifndef EINSUM_PHASE_STOP",
        "#define EINSUM_PHASE_STOP 3",
        "#endif",
        "",
    ]
    configs = []
    if recipe["elementwise"]:
        configs.append(f"struct config_elementwise {{\n    static const unsigned long long N = {recipe['n_elem']};\n}};\n")
    elif recipe["broadcast"]:
        r = recipe
        od = r["bc_outer_dims"] or (1,)
        ob = r["bc_outer_bstride"] or (0,)
        nor = max(1, len(r["bc_outer_dims"]))
        configs.append(
            "struct config_broadcast {\n"
            f"    static constexpr int mode = {r['bc_mode']};\n"
            f"    static constexpr unsigned long long N = {r['n_elem']};\n"
            f"    static constexpr unsigned long long Cc = {r['bc_Cc']};\n"
            f"    static constexpr unsigned long long Rr = {r['bc_Rr']};\n"
            f"    static constexpr unsigned long long Inner = {r['bc_Inner']};\n"
            f"    static constexpr unsigned long long Outer = {r['bc_Outer']};\n"
            f"    static constexpr unsigned long long sizeB = {r['bc_sizeB']};\n"
            f"    static constexpr unsigned outer_rank = {len(r['bc_outer_dims'])};\n"
            f"    static constexpr unsigned long long outer_dims[{nor}] = {{{_arr(od)}}};\n"
            f"    static constexpr unsigned long long outer_bstride[{nor}] = {{{_arr(ob)}}};\n"
            f"    static constexpr bool full_is_input0 = {'true' if r['bc_full_is_in0'] else 'false'};\n"
            "};\n")
    else:
        s0, s1 = exec_shapes
        p0, p1 = recipe["in_transpose_idxs"]
        configs += [tconfig_struct(transpose_config("config_tpose_inp0", s0, p0)),
                    tconfig_struct(transpose_config("config_tpose_inp1", s1, p1)),
                    tconfig_struct(transpose_config("config_tpose_out", recipe["out_interpret_shape"],
                                                    recipe["out_transpose_idxs"])),
                    einsum_struct(recipe)]
    parts = head + configs + ["// MI355X launch plan", plan_function(plan)]
    is_matmul = not recipe["elementwise"] and not recipe["broadcast"]
    if is_matmul:
        parts.append(component_functions(plan))
    ep = [
        'extern "C" {',
        f"int run_einsum(const {T}* input0, const {T}* input1, float* output, void* stream) {{",
        "    return pe_einsum_run(&kPlan, input0, input1, output, stream);",
        "}",
        "void* run_einsum_setup(void* stream) {",
        "    return pe_einsum_setup(&kPlan, stream);",
        "}",
        f"int run_einsum_exec(const {T}* input0, const {T}* input1, float* output, void* workspace, void* stream) {{",
        "    return pe_einsum_exec(&kPlan, input0, input1, output, workspace, stream);",
        "}",
        "void run_einsum_teardown(void* workspace) {",
        "    pe_einsum_teardown(workspace);",
        "}",
    ]
    if is_matmul:
        ep += [
            f"int run_transpose_inp0(const {T}* input, {T}* output, void* stream) {{",
            "    return pe_permute(&kPerm0, input, output, stream);",
            "}",
            f"int run_transpose_inp1(const {T}* input, {T}* output, void* stream) {{",
            "    return pe_permute(&kPerm1, input, output, stream);",
            "}",
            "int run_transpose_out(const float* input, float* output, void* stream) {",
            "    return pe_permute(&kPermOut, input, output, stream);",
            "}",
            f"int run_batched_matmul(const {T}* ws0, const {T}* ws1, float* ws_res, void* stream) {{",
            "    return pe_gemm(&kCanonGemm, ws0, ws1, ws_res, 0, 0, stream);",
            "}",
        ]
    ep += ["}  // extern \"C\"", ""]
    return "\n".join(parts + ep)


def cpu_source(equation: str, shapes, recipe: Dict, exec_shapes) -> str:
    """The per-shape CPU-route source (reference: templates.py:131-156)."""
    head = [f"// pto_einsum JIT source (CPU route): {equation} {tuple(shapes[0])} x {tuple(shapes[1])} float32",
            '#include "pto_einsum_cpu.h"', ""]
    if recipe["elementwise"]:
        body = [f"struct config_elementwise {{\n    static const unsigned long long N = {recipe['n_elem']};\n}};\n",
                'extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {',
                "    pto_einsum_cpu::hadamard<float, config_elementwise>(input0, input1, output);",
                "}", ""]
        return "\n".join(head + body)
    s0, s1 = exec_shapes
    p0, p1 = recipe["in_transpose_idxs"]
    body = [tconfig_struct(transpose_config("config_tpose_inp0", s0, p0)),
            tconfig_struct(transpose_config("config_tpose_inp1", s1, p1)),
            tconfig_struct(transpose_config("config_tpose_out", recipe["out_interpret_shape"],
                                            recipe["out_transpose_idxs"])),
            einsum_struct(recipe),
            'extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {',
            "    pto_einsum_cpu::einsum<float, config_einsum>(input0, input1, output);",
            "}", ""]
    return "\n".join(head + body)
