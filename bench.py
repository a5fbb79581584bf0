"""Benchmark of the MI355X einsum path (one JSON line on stdout).

Headline workload: benchmark config 2, the transposing batched contraction
``bji,bjk->bik`` in float32 with b=16, i=1000, j=777, k=1536 (standard-normal
inputs from a seed).  A step is one ``run_einsum_exec`` over that batch with
operands and output resident in HBM.  ``value`` is TFLOP/s over the timed
steps (2*b*i*j*k flops per step).  ``roofline`` relates the GEMM kernel's
average launch time (HIP events recorded around each launch on the launch
stream) to the float32 MFMA peak.  ``cpu_baseline`` times the reference CPU
route (cpu_einsum.h compiled by oracle/ref_build.py; the C restatement in
oracle/ when that build is absent) on the whole of config 2, one thread, and
every ``per_config`` row carries the same route's time on that config
(``cpu_s``, one thread, same seeded inputs up-cast to float32).

Cache: MI355X has a 256 MB Infinity Cache in front of HBM.  Every timed case
therefore rotates through enough copies of its operands and output (at least
1 GiB in total, four times the cache) that each call reads operands and
writes an output no call has touched for over 768 MB of traffic: the figures
are HBM figures, not cache figures.  Einsum cases call the per-shape
library's run_einsum_exec with an explicit output per operand set; the
headline steps rotate the same way.

Clocks: after an idle gap (host-side setup between cases) the GPU's clock
ramps back up over about 25 ms of sustained work: config 2's launches take
346 us right after a 1 s pause and settle at 292 us (128x256 tiles) or 278 us
(128x128) after about 80 launches.  Every figure here is taken at the
settled clock: the headline does ``--warmup`` untimed steps first (default
200, about 60 ms), and each graph-replayed case replays its graph back to
back for at least 50 ms before the timed replays, which also run back to
back (one event pair per replay, one synchronisation after the last).

``per_config`` adds every other benchmark equation at full size with its own
binding roof (HBM bytes or MFMA flops).  Those kernels run for tens of
microseconds, less than one Python-level call costs, so the rotation's calls
are captured once in a HIP graph and the graph is replayed between two
events: the figure is the GPU time per einsum.

``large_f16`` times 8192^3 float16 contractions (float32 output) in the
NN and NT layouts on the dense float16 MFMA roof, with torch.matmul (the
vendor library, float16 output) beside them; ``vendor_thin`` times
torch.matmul on config 5's two thin contractions (5.1, 5.3) with the same
operand rotation as the ``per_config`` rows.

``gdn`` times the GDN contraction set at the reference's sizes the same way,
and ``gdn_stages`` two of its stage sequences issued eagerly (one Python call
per launch) and replayed as one HIP graph (``pto_einsum.StageGraph``).

``launch_floor`` replays the launch probe (one wave, one store) in a graph
of as many launches as config 1's rotation: the fixed cost of a launch that
config 1's 256^3 GEMM is read against.  ``cold_call`` gives the host cost of
the one-shot ``einsum()``: the first call on a new shape (plan, host-code
compile, load), the first after the in-process runner cache is cleared, and
a cached call's host time.

``roofline.traffic`` (HBM bytes per launch of the headline GEMM) is read from
profiles/gemm_f32_config2_traffic.json, written from two rocprofv3 --pmc runs
(FETCH_SIZE, WRITE_SIZE) of ``bench.py --profile 2``, scaled by the same
counters on ``--copy-probe`` (a plain copy of known size); the file names
the kernel it was measured on, and the line carries that name beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-configs]
       python bench.py --profile CASE   # one case, eager calls (after ~50 ms of warm-up calls), for rocprofv3
       python bench.py --list-cases
       python bench.py --copy-probe     # counter calibration: one 1 GiB copy
"""
import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pto-einsum_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"f32": 157.3, "f16": 2516.6}
ROTATE_BYTES = 1 << 30          # rotated working set per timed case (4x the Infinity Cache)
MAX_SETS = 2048


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-configs", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-time budget of the CPU baseline (at least one whole call)")
    ap.add_argument("--profile", metavar="CASE",
                    help="run one case (see --list-cases) as eager rotated calls and exit")
    ap.add_argument("--list-cases", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run a plain 1 GiB device copy (counter calibration) and exit")
    return ap.parse_args()


# ------------------------------------------------------------------ timing --

def n_sets(set_bytes):
    """Copies of a case's operands + output that make a >= 1 GiB rotation."""
    if set_bytes >= ROTATE_BYTES:
        return 1
    return int(min(MAX_SETS, max(2, math.ceil(ROTATE_BYTES / max(1, set_bytes)))))


def replicate(tensors, n):
    """n copies (the first the originals) of every tensor, on the GPU."""
    sets = [tuple(tensors)]
    for _ in range(n - 1):
        sets.append(tuple(t.clone() for t in tensors))
    return sets


def time_runner(run, sets, steps, warmup):
    """Headline timing: per-launch HIP-event times (ms) and the wall time of
    the timed region; step i runs on operand set i % len(sets)."""
    import torch

    for i in range(warmup):
        run(*sets[i % len(sets)])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i, (s, e) in enumerate(ev):
        s.record(stream)
        run(*sets[(warmup + i) % len(sets)])
        e.record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in ev]
    return per, t0.elapsed_time(t1)


def time_graph(call, sets, reps=5, warm_ms=50.0):
    """GPU time (ms) per call: one call per operand set captured in one HIP
    graph; the graph is replayed back to back for at least `warm_ms` (the
    clock's ramp after an idle gap), then `reps` more times back to back,
    each between its own pair of events; the median replay time divided by
    the number of calls."""
    import torch

    for s in sets[:2]:
        call(*s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s in sets:
            call(*s)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    once = max(e0.elapsed_time(e1), 1e-3)
    for _ in range(min(100000, int(math.ceil(warm_ms / once)))):
        g.replay()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) / len(sets) for a, b in ev]
    del g
    return statistics.median(per)


def run_eager(call, sets, calls, warm_ms=50.0):
    """Profiling mode: eager calls rotating over the sets, first for at least
    `warm_ms` of GPU time (the clock's ramp), then `calls` more (the ones a
    profile summary averages); returns the number of warm-up calls."""
    import torch

    it = iter(range(1 << 30))
    warm = settle(lambda: call(*sets[next(it) % len(sets)]), warm_ms)
    for i in range(calls):
        call(*sets[i % len(sets)])
    torch.cuda.synchronize()
    return warm


def settle(fn, warm_ms=50.0):
    """Calls fn() for at least `warm_ms` of GPU time (the clock's ramp after
    an idle gap; see the module docstring); returns the number of calls."""
    import torch

    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    warm = min(5000, int(math.ceil(warm_ms / max(e0.elapsed_time(e1), 1e-3))))
    for _ in range(warm):
        fn()
    return warm + 2


def time_rotated(fn, sets, calls, warm_ms=50.0):
    """GPU time (ms) per call of `calls` eager calls rotating over the sets,
    between two events, after settle()."""
    import torch

    it = iter(range(1 << 30))
    settle(lambda: fn(*sets[next(it) % len(sets)]), warm_ms)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(calls):
        fn(*sets[i % len(sets)])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / calls


def copy_probe():
    """A 1 GiB float32 copy through the core library's permutation launcher
    (identity permutation = plain copy): reads and writes exactly 1 GiB."""
    import torch

    from pto_einsum import abi, launch

    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    lib = abi.bind()
    d = abi.permute_desc(launch.PermuteDesc(4, [n], [1], n))
    for _ in range(5):
        rc = lib.pe_permute(ctypes.byref(d), ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "launches": 5}))


def attainable(dev):
    """Attainable peaks on this device, measured with kernels of this build:
    a 1 GiB float32 copy (the permutation launcher with the identity; cold,
    as 1 GiB exceeds the Infinity Cache) and the MFMA probe (no memory
    traffic; float16 on random and on constant operands, float32 on random
    ones -- the clock follows the operands' bit activity)."""
    import torch

    from pto_einsum import abi, launch

    lib = abi.bind()
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def timed(fn, reps=5):
        settle(fn)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # seconds per call

    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    d = abi.permute_desc(launch.PermuteDesc(4, [n], [1], n))

    def copy():
        rc = lib.pe_permute(ctypes.byref(d), ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), st)
        if rc != 0:
            raise RuntimeError("copy probe failed")

    out = {"copy_gbs": round(2 * n * 4 / timed(copy) / 1e9, 1)}
    del src, dst
    buf = torch.empty(int(lib.pe_probe_out_len()), dtype=torch.float32, device=dev)
    for name, dt, rnd, iters in (("mfma_f16_random_tflops", 1, 1, 2000), ("mfma_f16_constant_tflops", 1, 0, 2000),
                                 ("mfma_f32_random_tflops", 0, 1, 2000)):
        def probe():
            rc = lib.pe_probe_mfma(dt, rnd, iters, ctypes.c_void_p(buf.data_ptr()), buf.numel(), st)
            if rc != 0:
                raise RuntimeError("mfma probe failed")
        out[name] = round(int(lib.pe_probe_mfma_flops(dt, iters)) / timed(probe) / 1e12, 1)
    log(f"bench: attainable {out}")
    return out


def traffic_from_profile():
    path = os.path.join(ROOT, "profiles", "gemm_f32_config2_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None, None
    src = f"profiles/gemm_f32_config2_traffic.json ({d.get('kernel', '?')}, commit {d.get('commit', '?')})"
    return d.get("hbm_bytes_per_launch"), src


# ------------------------------------------------------------------- cases --

def rope_table(s, d):
    import torch

    pos = torch.arange(s, dtype=torch.float64)[:, None]
    i = torch.arange(d, dtype=torch.float64)[None, :] % (d // 2)
    theta = 10000.0 ** (-2.0 * i / d)
    return torch.cos(pos * theta).to(torch.float16)


def decay(t, gamma):
    import torch

    i = torch.arange(t, dtype=torch.float64)
    d = (i[:, None] - i[None, :])
    return torch.where(d >= 0, gamma ** d.clamp(min=0), torch.zeros(())).float()


def config_list():
    """benchmark configs other than the headline: (name, equation, operand
    generator, roof dtype)."""
    import torch

    def randn(shape, g, scale=1.0, dtype=torch.float32):
        return (torch.randn(shape, generator=g) * scale).to(dtype)

    f16 = torch.float16
    return [
        ("1", "ij,jk->ik", lambda g: (torch.rand(256, 256, generator=g), torch.rand(256, 256, generator=g)), "f32"),
        ("3", "bshd,bthd->bsht", lambda g: (randn((4, 2048, 32, 128), g, 128 ** -0.5, f16),
                                            randn((4, 2048, 32, 128), g, 128 ** -0.5, f16)), "f16"),
        ("4a", "ts,ts->ts", lambda g: (torch.rand(8192, 8192, generator=g), decay(8192, 0.99)), "f32"),
        ("4b", "bsd,d->bsd", lambda g: (randn((8, 4096, 4096), g, 1.0, f16),
                                        (torch.rand(4096, generator=g) + 0.5).to(f16)), "f16"),
        ("5.1", "tn,sn->ts", lambda g: (randn((4096, 128), g, 128 ** -0.5, f16),
                                        randn((4096, 128), g, 128 ** -0.5, f16)), "f16"),
        ("5.2", "ts,ts->ts", lambda g: (torch.rand(4096, 4096, generator=g), decay(4096, 0.995)), "f32"),
        ("5.3", "ts,sp->tp", lambda g: (torch.rand(4096, 4096, generator=g), randn((4096, 128), g)), "f32"),
        ("5.R", "bshd,sd->bshd", lambda g: (randn((2, 4096, 32, 128), g, 1.0, f16), rope_table(4096, 128)), "f16"),
    ]


def transpose_list():
    """The reference recipe's standalone operand / output transposes (Phase A
    and Phase C of pto_einsum.h:52-177) for the benchmark contractions that
    have them, run through the per-shape library's run_transpose_* entry
    points: (label, equation, operand shapes, dtype, entry point)."""
    import torch

    f16 = torch.float16
    s3 = (4, 2048, 32, 128)
    return [
        ("2 in0 (0,2,1)", "bji,bjk->bik", ((16, 777, 1000), (16, 777, 1536)), torch.float32, "run_transpose_inp0"),
        ("3 in0 (0,2,1,3)", "bshd,bthd->bsht", (s3, s3), f16, "run_transpose_inp0"),
        ("3 in1 (0,2,3,1)", "bshd,bthd->bsht", (s3, s3), f16, "run_transpose_inp1"),
        ("3 out (0,2,1,3)", "bshd,bthd->bsht", (s3, s3), f16, "run_transpose_out"),
        ("5.1 in1 (1,0)", "tn,sn->ts", ((4096, 128), (4096, 128)), f16, "run_transpose_inp1"),
    ]


GDN_EQS = (("kkt", "bihd,bjhd->bihj"), ("wy_fast", "bihj,bjhd->bihd"),
           ("chunk_h kv", "bvhd,bvhe->bhde"), ("chunk_o inter", "bvhd,bhde->bvhe"))


def gdn_list():
    """The GDN contraction set (float32, chunk = d = 128) at the sizes the
    reference measures it on (IMPLEMENTATION.md:700-782: b x H = 16x16, 64x16,
    16x48; b = folded chunks): (label, equation, shape0, shape1)."""
    rows = []
    for b, H in ((16, 16), (64, 16), (16, 48)):
        for name, eq in GDN_EQS:
            s1 = (b, H, 128, 128) if eq == "bvhd,bhde->bvhe" else (b, 128, H, 128)
            rows.append((f"{name} {b}x{H}", eq, (b, 128, H, 128), s1))
    return rows


def work(eq, a, b):
    """(flops, compulsory bytes) of one einsum: 2*I*L0*L1*C (or N for a
    product) and inputs read once plus the float32 output written once."""
    from math import prod

    t0, rest = eq.split(",")
    t1, to = rest.split("->")
    size = dict(zip(t0, a.shape))
    size.update(zip(t1, b.shape))
    out = prod(size[x] for x in to)
    C = prod(size[x] for x in (set(t0) & set(t1)) - set(to))
    flops = 2 * out * C if C > 1 else out
    nbytes = a.numel() * a.element_size() + b.numel() * b.element_size() + out * 4
    return flops, nbytes


def roofline(flops, nbytes, t_ms, dtype):
    tflops = flops / (t_ms * 1e-3) / 1e12
    gbs = nbytes / (t_ms * 1e-3) / 1e9
    t_mfma = flops / (PEAK_TFLOPS[dtype] * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    if t_mfma >= t_hbm:
        return dict(bound="mfma", achieved=round(tflops, 3), peak=PEAK_TFLOPS[dtype], unit="TFLOP/s",
                    frac=round(tflops / PEAK_TFLOPS[dtype], 4)), tflops, gbs
    return dict(bound="hbm", achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                frac=round(gbs / PEAK_HBM_GBS, 4)), tflops, gbs


class Case:
    """One timed workload: `prepare(dev)` returns (call, operand tuple,
    set bytes); `call(*operands)` enqueues it once."""

    def __init__(self, name, prepare, finish):
        self.name, self.prepare, self.finish = name, prepare, finish


def exec_call(builder, dev):
    """call(x, y, out): one run_einsum_exec of the built per-shape library
    (the C ABI the reference's runner calls, builder.py:877-881) on the
    current stream, writing into `out`, with one workspace kept with the
    call.  Every rotated operand set carries its own output, so no
    two calls in a row write the same output buffer."""
    import torch

    lib, ct = builder.lib, builder.c_type
    ws = torch.zeros(max(int(builder._ws_bytes), 256), dtype=torch.uint8, device=dev)
    swap = builder._swap_operands

    def call(x, y, out):
        a, b = (y, x) if swap else (x, y)
        rc = lib.run_einsum_exec(ctypes.cast(a.data_ptr(), ctypes.POINTER(ct)),
                                 ctypes.cast(b.data_ptr(), ctypes.POINTER(ct)),
                                 ctypes.cast(out.data_ptr(), ctypes.POINTER(ctypes.c_float)),
                                 ctypes.c_void_p(ws.data_ptr()),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"run_einsum_exec failed ({rc})")

    call.workspace = ws
    return call


def einsum_case(name, eq, gen, dt, seed, label=None):
    import torch

    from pto_einsum import EinsumBuilder

    def prepare(dev):
        g = torch.Generator().manual_seed(seed)
        x, y = gen(g)
        x, y = x.to(dev), y.to(dev)
        builder = EinsumBuilder(eq, [tuple(x.shape), tuple(y.shape)], x.dtype)
        builder.build()
        out = torch.empty(builder.recipe["out_shape"], dtype=torch.float32, device=dev)
        call = exec_call(builder, dev)
        call.builder = builder
        return call, (x, y, out), (x.numel() * x.element_size() + y.numel() * y.element_size()
                                    + out.numel() * 4)

    def finish(ms, operands, nsets):
        x, y = operands[:2]
        f, nb = work(eq, x, y)
        rf, tf, gb = roofline(f, nb, ms, dt)
        row = dict(config=name, equation=eq, dtype=dt, us=round(ms * 1e3, 2), tflops=round(tf, 3),
                   gbs=round(gb, 1), roof=rf["bound"], frac=rf["frac"], sets=nsets)
        if label:
            row = dict(label, **row)
        log(f"bench: {name} {eq} {ms * 1e3:.1f} us  {tf:.2f} TFLOP/s  {gb:.0f} GB/s  "
            f"{rf['bound']} {rf['frac'] * 100:.1f}%  ({nsets} rotated sets)")
        return row

    case = Case(name, prepare, finish)
    case.seed, case.gen, case.eq = seed, gen, eq
    return case


def transpose_case(label, eq, shapes, dtype, entry):
    import torch

    from pto_einsum import EinsumBuilder

    info = {}

    def prepare(dev):
        builder = EinsumBuilder(eq, [tuple(x) for x in shapes], dtype)
        builder.build()
        rec = builder.recipe
        if entry == "run_transpose_out":
            src_shape = tuple(rec["out_interpret_shape"])
            perm = tuple(rec["out_transpose_idxs"])
            src_dtype = torch.float32
        else:
            k = 0 if entry == "run_transpose_inp0" else 1
            src_shape = tuple(builder._exec_shapes[k])
            perm = tuple(rec["in_transpose_idxs"][k])
            src_dtype = dtype
        g = torch.Generator().manual_seed(7)
        x = torch.randn(src_shape, generator=g).to(src_dtype).to(dev)
        y = torch.empty([src_shape[p] for p in perm], dtype=src_dtype, device=dev)
        fn = getattr(builder.lib, entry)
        info.update(builder=builder, src_shape=src_shape, perm=perm, src_dtype=src_dtype)

        def call(x, y):
            rc = fn(ctypes.cast(x.data_ptr(), fn.argtypes[0]), ctypes.cast(y.data_ptr(), fn.argtypes[1]),
                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if rc != 0:
                raise RuntimeError(f"{entry} failed ({rc})")

        return call, (x, y), 2 * x.numel() * x.element_size()

    def finish(ms, operands, nsets):
        x, _ = operands
        nbytes = 2 * x.numel() * x.element_size()
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"bench: transpose {label} of {eq} {info['src_shape']} {ms * 1e3:.1f} us  {gbs:.0f} GB/s  "
            f"hbm {gbs / PEAK_HBM_GBS * 100:.1f}%  ({nsets} rotated sets)")
        return dict(transpose=label, equation=eq, dtype=str(info["src_dtype"]).replace("torch.", ""),
                    shape=list(info["src_shape"]), perm=list(info["perm"]), us=round(ms * 1e3, 2),
                    gbs=round(gbs, 1), roof="hbm", frac=round(gbs / PEAK_HBM_GBS, 4), sets=nsets)

    return Case("T" + ".".join(label.split()[:2]), prepare, finish)


T5, N5 = 4096, 128


def chain_case(precise):
    """benchmark config 5's linear-attention chain in one fused launch
    (pto_einsum.linear_attention): q, k float16 normal(0, 1/sqrt(128)), v
    float16 normal(0, 1), the causal decay mask gamma^(t-s), gamma = 0.995,
    in float32; t = s = 4096, n = p = 128.  The default launch computes P.V
    at float32 accuracy on bfloat16 MFMAs (P in three terms, the float16 V in
    two: five products per k step); ``precise`` puts P.V on float32 MFMAs.
    The roof is the larger of the compulsory HBM bytes (q, k, v, m read once,
    out written once) at 8 TB/s and the MFMAs the launch issues for the dense
    chain (2*T*S*N float16 flops plus, for the default, 5 * 2*T*S*P bfloat16
    flops at the 16-bit peak, for precise 2*T*S*P at the float32 peak); zero
    mask blocks are skipped, so the causal case does less."""
    import torch

    from pto_einsum import linear_attention

    T = S = T5
    N = P = N5

    def prepare(dev):
        g = torch.Generator().manual_seed(105)
        q = (torch.randn(T, N, generator=g) * N ** -0.5).half().to(dev)
        k = (torch.randn(S, N, generator=g) * N ** -0.5).half().to(dev)
        v = torch.randn(S, P, generator=g).half().to(dev)
        m = decay(T, 0.995).to(dev)
        out = torch.empty((T, P), dtype=torch.float32, device=dev)
        nbytes = (q.numel() + k.numel() + v.numel()) * 2 + m.numel() * 4 + T * P * 4

        def call(q, k, v, m, out):
            linear_attention(q, k, v, m, precise=precise, out=out)

        return call, (q, k, v, m, out), nbytes

    def finish(ms, operands, nsets):
        flops = 2 * T * S * N + T * S + 2 * T * S * P
        nbytes = T * N * 2 * 2 + S * P * 2 + T * S * 4 + T * P * 4
        hbm_ms = nbytes / (PEAK_HBM_GBS * 1e9) * 1e3
        if precise:
            mfma_ms = (2 * T * S * N / PEAK_TFLOPS["f16"] + 2 * T * S * P / PEAK_TFLOPS["f32"]) / 1e12 * 1e3
        else:
            mfma_ms = (2 * T * S * N + 5 * 2 * T * S * P) / (PEAK_TFLOPS["f16"] * 1e12) * 1e3
        floor_ms = max(hbm_ms, mfma_ms)
        row = dict(config="5.F" + (" precise" if precise else ""), equation="tn,sn,sp,ts->tp (fused)",
                   dtype="f16 q/k, f32 chain, P.V " + ("f32 MFMA" if precise else "f32-accurate bf16x3"),
                   us=round(ms * 1e3, 2), tflops=round(flops / (ms * 1e-3) / 1e12, 3),
                   gbs=round(nbytes / (ms * 1e-3) / 1e9, 1), roof="hbm" if hbm_ms >= mfma_ms else "mfma",
                   frac=round(floor_ms / ms, 4), floor_us=round(floor_ms * 1e3, 2), sets=nsets)
        log(f"bench: config {row['config']} tn,sn,sp,ts->tp {ms * 1e3:.1f} us (floor {floor_ms * 1e3:.1f} us, "
            f"{row['roof']} {row['frac'] * 100:.1f}%)  ({nsets} rotated sets)")
        return row

    return Case("5.Fp" if precise else "5.F", prepare, finish)


def large_f16_cases():
    import torch

    n = 8192

    def gen(g):
        return ((torch.randn(n, n, generator=g) / 64).half(), (torch.randn(n, n, generator=g) / 64).half())

    return [einsum_case(f"f16{lab}", eq, gen, "f16", 77, dict(shape=f"{n}^3 {lab}"))
            for eq, lab in (("ij,jk->ik", "NN"), ("ik,jk->ij", "NT"))]


# Opt-in solo-axis reduction (pe_reduce_axes): (label, shape, reduced axes, dtype); the
# operands are 0.5-1 GiB, so every call reads cold data.
SOLO_REDUCE = (
    ("f32 [64,4000000] sum(1)", (64, 4_000_000), (1,), "f32"),
    ("f32 [1024,250000] sum(1)", (1024, 250_000), (1,), "f32"),
    ("f16 [1024,250000] sum(1)", (1024, 250_000), (1,), "f16"),
    ("f32 [16384,16000] sum(1)", (16384, 16_000), (1,), "f32"),
    ("f32 [262144,1024] sum(1)", (262144, 1024), (1,), "f32"),
    ("f32 [1000000,256] sum(1)", (1_000_000, 256), (1,), "f32"),
    ("f32 [8000000,32] sum(1)", (8_000_000, 32), (1,), "f32"),
    ("f32 [4000000,64] sum(0)", (4_000_000, 64), (0,), "f32"),
)


def solo_reduce_case(label, shape, axes, dt):
    """builder._reduce_operand (the reduction stage of einsum(...,
    reduce_solo_axes=True)) on one operand; roof = bytes read at 8 TB/s."""
    import torch

    info = {}

    def prepare(dev):
        from pto_einsum.builder import _reduce_operand

        subs = "ab"
        solo = "".join(subs[i] for i in axes)
        g = torch.Generator().manual_seed(17)
        x = torch.randn(shape, generator=g).to(torch.float16 if dt == "f16" else torch.float32).to(dev)
        info["bytes"] = x.numel() * x.element_size()

        def call(x):
            _reduce_operand(x, subs, solo)

        return call, (x,), info["bytes"]

    def finish(ms, operands, nsets):
        gbs = info["bytes"] / (ms * 1e-3) / 1e9
        log(f"bench: solo reduce {label} {ms * 1e3:.1f} us  {gbs:.0f} GB/s  hbm {gbs / PEAK_HBM_GBS * 100:.1f}%")
        return dict(reduce=label, dtype=dt, us=round(ms * 1e3, 2), gbs=round(gbs, 1), roof="hbm",
                    frac=round(gbs / PEAK_HBM_GBS, 4), sets=nsets)

    name = "R." + "x".join(str(n) for n in shape) + ".sum" + "".join(str(a) for a in axes) + "." + dt
    return Case(name, prepare, finish)


def gdn_cases():
    import torch

    out = []
    for i, (label, eq, s0, s1) in enumerate(gdn_list()):
        def gen(g, s0=s0, s1=s1):
            return (torch.randn(s0, generator=g) * 128 ** -0.5, torch.randn(s1, generator=g) * 128 ** -0.5)

        out.append(einsum_case("gdn." + label.replace(" ", "."), eq, gen, "f32", 200 + i,
                               dict(gdn=label, shapes=[list(s0), list(s1)])))
    return out


HEADLINE_SEED = 2


def headline_gen(g):
    """Config 2's operands: standard normal, b=16, j=777, i=1000, k=1536."""
    import torch

    return torch.randn((16, 777, 1000), generator=g), torch.randn((16, 777, 1536), generator=g)


def all_cases():
    import torch

    head = einsum_case("2", "bji,bjk->bik", headline_gen, "f32", HEADLINE_SEED)
    groups = {"headline": [head],
              "per_config": [einsum_case(n, e, gen, d, 100 + i) for i, (n, e, gen, d) in enumerate(config_list())]
              + [chain_case(False), chain_case(True)],
              "transposes": [transpose_case(*t) for t in transpose_list()],
              "large_f16": large_f16_cases(),
              "gdn": gdn_cases(),
              "solo_reduce": [solo_reduce_case(*r) for r in SOLO_REDUCE]}
    return groups


def measure(case, dev, steps, warmup, profile_calls=0):
    """Rotated timing of one case: returns its row (or runs it eagerly for a
    profiler when profile_calls > 0)."""
    import torch

    call, operands, set_bytes = case.prepare(dev)
    nsets = n_sets(set_bytes)
    sets = replicate(operands, nsets)
    if profile_calls:
        warm = run_eager(call, sets, profile_calls)
        log(f"bench: profiling {case.name}: {warm} warm-up and {profile_calls} counted eager calls over {nsets} "
            f"rotated sets")
        return warm
    ms = time_graph(call, sets, reps=max(3, steps // 6))
    row = case.finish(ms, operands, nsets)
    del sets, operands, call
    torch.cuda.empty_cache()
    return row


# ------------------------------------------------------------ stage graphs --

def time_eager(fn, iters):
    """GPU-side time (ms) per call of `fn` issued back to back from Python:
    events around the whole loop, so host gaps between launches count."""
    import torch

    settle(fn)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def time_stage_graph(fn, iters):
    import torch

    from pto_einsum import StageGraph

    graph = StageGraph(fn)
    settle(graph.replay)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / iters


def time_gdn_stages(dev, steps):
    """Two GDN stage sequences issued eagerly (one Python call per launch)
    and as one StageGraph replay: the seven folded-batch contractions of one
    GDN forward (b = 16, H = 16) and the chunk_h recurrence (B = 1, T = 1024,
    H = 32: per chunk two contractions and four elementwise ops, eight chunks
    in sequence).  These measure launch overhead, so they run on one set of
    operands (their working sets are cache-sized by construction)."""
    import torch

    from pto_einsum import einsum

    g = torch.Generator().manual_seed(300)
    shape = (16, 128, 16, 128)
    q, k, v = ((torch.randn(shape, generator=g) * 128 ** -0.5).to(dev) for _ in range(3))

    def stages():
        A = einsum("bihd,bjhd->bihj", k, k)
        return (A, einsum("bihj,bjhd->bihd", A, v), einsum("bihj,bjhd->bihd", A, k),
                einsum("bvhd,bhde->bvhe", q, einsum("bvhd,bvhe->bhde", k, v)),
                einsum("bihj,bjhd->bihd", einsum("bihd,bjhd->bihj", q, k), v))

    B, T, H, D = 1, 1024, 32, 128
    w = (torch.randn(B, T, H, D, generator=g) * D ** -0.5).to(dev)
    u = torch.randn(B, T, H, D, generator=g).to(dev)
    kk = (torch.randn(B, T, H, D, generator=g) * D ** -0.5).to(dev)
    gexp = (0.5 + 0.5 * torch.rand(B, T, H, 1, generator=g)).to(dev)
    gdecay = (0.5 + 0.5 * torch.rand(T // 128, B, H, 1, 1, generator=g)).to(dev)
    S0 = torch.zeros(B, H, D, D, device=dev)

    def chunk_h():
        S = S0
        vs = []
        for c in range(T // 128):
            rows_ = slice(c * 128, (c + 1) * 128)
            vc = u[:, rows_] - einsum("bvhd,bhde->bvhe", w[:, rows_], S)
            vs.append(vc)
            S = gdecay[c] * S + einsum("bvhd,bvhe->bhde", kk[:, rows_], vc * gexp[:, rows_])
        return torch.cat(vs, dim=1), S

    seqs = []
    for label, fn, launches in (("gdn forward contractions b=16 H=16 (7 einsums)", stages, 7),
                                ("chunk_h recurrence B=1 T=1024 H=32 (16 einsums + 32 elementwise)", chunk_h, 48)):
        eager = time_eager(fn, max(10, steps))
        replay = time_stage_graph(fn, max(10, steps))
        seqs.append(dict(stages=label, launches=launches, eager_us=round(eager * 1e3, 2),
                         graph_us=round(replay * 1e3, 2), speedup=round(eager / replay, 2)))
        log(f"bench: {label}: eager {eager * 1e3:.1f} us, graph replay {replay * 1e3:.1f} us "
            f"({eager / replay:.2f}x)")
    torch.cuda.empty_cache()
    return seqs


def time_torch_matmul(dev):
    """torch.matmul (hipBLASLt, float16 output) at 8192^3 NN / NT beside the
    large float16 contractions, rotating two operand sets."""
    import torch

    n = 8192
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(n, n, generator=g) / 64).half().to(dev)
    y = (torch.randn(n, n, generator=g) / 64).half().to(dev)
    out = []
    for label in ("NN", "NT"):
        yy = y if label == "NN" else y.t().contiguous()
        sets = replicate((x, yy), 2)
        fn = (lambda a, b: torch.matmul(a, b)) if label == "NN" else (lambda a, b: torch.matmul(a, b.t()))
        t = time_rotated(fn, sets, 10)
        tf = 2 * n ** 3 / t / 1e9
        out.append(dict(shape=f"{n}^3 {label}", equation="torch.matmul (float16 output)", dtype="f16",
                        us=round(t * 1e3, 1), tflops=round(tf, 1), roof="mfma",
                        frac=round(tf / PEAK_TFLOPS["f16"], 4)))
        log(f"bench: torch.matmul f16 {label} {t * 1e3:.1f} us {tf:.1f} TFLOP/s")
        del sets
    del x, y
    torch.cuda.empty_cache()
    return out


def time_torch_thin(dev, calls=50):
    """The vendor library (torch.matmul / torch.bmm -> hipBLASLt) on config 5's
    two thin contractions and on the headline, with the operand rotation of
    the per-config rows: 5.1 tn,sn->ts in float16 (float16 output, half the
    bytes this path's float32 output writes), 5.3 ts,sp->tp and config 2
    bji,bjk->bik (A read transposed, as here) in float32 with TF32 off (this
    path's precision)."""
    import torch

    g = torch.Generator().manual_seed(51)
    f16 = torch.float16
    cases = (("5.1", "tn,sn->ts", (torch.randn(4096, 128, generator=g) * 128 ** -0.5).to(f16),
              (torch.randn(4096, 128, generator=g) * 128 ** -0.5).to(f16), lambda a, b: torch.matmul(a, b.t()),
              4096 * 4096 * 2),
             ("5.3", "ts,sp->tp", torch.rand(4096, 4096, generator=g), torch.randn(4096, 128, generator=g),
              torch.matmul, 4096 * 128 * 4),
             # the headline contraction in its own layout: A read transposed
             # (a [b, j, i] view as [b, i, j]), float32 in and out
             ("2", "bji,bjk->bik", torch.randn(16, 777, 1000, generator=g), torch.randn(16, 777, 1536, generator=g),
              lambda a, b: torch.bmm(a.transpose(1, 2), b), 16 * 1000 * 1536 * 4))
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    out = []
    try:
        for cfg, eq, a, b, fn, out_bytes in cases:
            a, b = a.to(dev), b.to(dev)
            sets = replicate((a, b), n_sets(a.nbytes + b.nbytes + out_bytes))
            t = time_rotated(fn, sets, calls)
            tf = (2 * 16 * 1000 * 1536 * 777 if cfg == "2" else 2 * 4096 * 4096 * 128) / (t * 1e-3) / 1e12
            out.append(dict(config=cfg, equation=f"torch.{'bmm' if cfg == '2' else 'matmul'} {eq} ({a.dtype} in and out)",
                            us=round(t * 1e3, 2), tflops=round(tf, 2), operand_sets=len(sets)))
            log(f"bench: torch.matmul {cfg} {eq} {t * 1e3:.1f} us")
            del sets, a, b
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------ CPU baseline --

def cpu_baseline(budget_s=10.0):
    """Reference CPU route on the whole of config 2 (all 16 batches) with the
    headline's own inputs (same generator and seed), one thread: called
    until `budget_s` is spent (at least once); best call."""
    import torch

    eq, s0, s1 = "bji,bjk->bik", (16, 777, 1000), (16, 777, 1536)
    g = torch.Generator().manual_seed(HEADLINE_SEED)
    a, b = (t.numpy() for t in headline_gen(g))
    fn, kind = _cpu_route(eq, a, b)
    times = []
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start) + statistics.median(times) < budget_s:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    dt = min(times)
    flops = 2.0 * 16 * 1000 * 1536 * 777
    return dict(value=round(flops / dt / 1e12, 6), unit="TFLOP/s", cores=1, kind=kind,
                sample=(f"the whole of config 2 (bji,bjk->bik float32, b=16, j=777, i=1000, k=1536; the "
                        f"headline's seeded inputs), {flops / 1e9:.1f} GFLOP per call, {len(times)} call(s) in "
                        f"{sum(times):.1f} s; best call {dt:.2f} s on 1 thread of {os.cpu_count()}"),
                seconds=round(sum(times), 3))


def _cpu_route(eq, a, b):
    """(callable, kind) running the reference CPU route on float32 arrays:
    the reference's own cpu_einsum.h build (oracle/_ref) when it was built
    for these shapes, else the C restatement in oracle/."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import ref_build

    if os.path.exists(ref_build.so_path(eq, a.shape, b.shape)):
        return (lambda: ref_build.run(eq, a, b)), "reference"
    return (lambda: oracle.einsum(eq, a, b)), "port"


def _cpu_time(fn):
    """Median wall time (s) of one synchronous call: three calls when one
    takes under 3 s, else the single call."""
    t = time.perf_counter()
    fn()
    first = time.perf_counter() - t
    if first >= 3.0:
        return first, 1
    times = [first]
    for _ in range(2):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), 3


def cpu_per_config(per_config_rows, cases):
    """The reference CPU route (device="cpu": float32, one thread) on every
    per-config workload at full size, with the inputs the GPU row used (same
    generator and seed; float16 inputs up-cast to float32, as that route is
    float32-only, builder.py:612-613).  Adds cpu_s, cpu_cores, cpu_kind and
    cpu_calls to each row; the fused chain's row gets the three reference
    einsums it replaces run in sequence on its own inputs."""
    import torch

    host = os.cpu_count()
    by_name = {c.name: c for c in cases}
    for row in per_config_rows:
        name = row["config"]
        if name.startswith("5.F"):
            continue
        case = by_name[name]
        g = torch.Generator().manual_seed(case.seed)
        x, y = case.gen(g)
        a, b = x.float().numpy(), y.float().numpy()
        fn, kind = _cpu_route(case.eq, a, b)
        dt, calls = _cpu_time(fn)
        row.update(cpu_s=round(dt, 4), cpu_cores=f"1 of {host}", cpu_kind=kind, cpu_calls=calls)
        log(f"bench: cpu {name} {case.eq} {dt:.3f} s ({kind}, {calls} call(s), 1 thread of {host})")
    chain = [r for r in per_config_rows if r["config"].startswith("5.F")]
    if chain:
        g = torch.Generator().manual_seed(105)
        T = S = T5
        q = (torch.randn(T, N5, generator=g) * N5 ** -0.5).half().float().numpy()
        k = (torch.randn(S, N5, generator=g) * N5 ** -0.5).half().float().numpy()
        v = torch.randn(S, N5, generator=g).half().float().numpy()
        m = decay(T, 0.995).numpy()
        f1, kind = _cpu_route("tn,sn->ts", q, k)

        def steps():
            A = f1()
            A2 = _cpu_route("ts,ts->ts", A, m)[0]()
            return _cpu_route("ts,sp->tp", A2, v)[0]()

        dt, calls = _cpu_time(steps)
        for r in chain:
            r.update(cpu_s=round(dt, 4), cpu_cores=f"1 of {host}", cpu_kind=kind, cpu_calls=calls,
                     cpu_note="the three reference einsums tn,sn->ts, ts,ts->ts, ts,sp->tp in sequence")
        log(f"bench: cpu 5.F (three einsums) {dt:.3f} s ({kind}, {calls} call(s))")


def cold_call(dev):
    """Host cost of the one-shot einsum() (builder.py:887-902 re-plans and
    re-loads per call): the first call on a new shape with an empty build
    directory (plan, host-code generation and compile, library load,
    workspace), the first call after the in-process runner cache is cleared
    (plan and load from the on-disk cache), and the steady-state host time
    of a cached call (Python checks, output allocation, ctypes launch),
    measured without synchronising, beside the GPU time of the same call."""
    import shutil
    import tempfile

    import torch

    from pto_einsum import builder as pb
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(99)
    a = torch.rand(256, 257, generator=g).to(dev)
    b = torch.rand(257, 255, generator=g).to(dev)
    eq = "ij,jk->ik"
    tmp = tempfile.mkdtemp(prefix="pe_cold_")
    old = os.environ.get("EINSUM_BUILD_DIR")
    os.environ["EINSUM_BUILD_DIR"] = tmp
    try:
        pb.clear_runner_cache()
        torch.cuda.synchronize()
        t = time.perf_counter()
        einsum(eq, a, b)
        torch.cuda.synchronize()
        first = time.perf_counter() - t
        pb.clear_runner_cache()
        t = time.perf_counter()
        einsum(eq, a, b)
        torch.cuda.synchronize()
        reload = time.perf_counter() - t
        for _ in range(20):
            einsum(eq, a, b)
        torch.cuda.synchronize()
        n = 200
        t = time.perf_counter()
        for _ in range(n):
            einsum(eq, a, b)
        host = (time.perf_counter() - t) / n
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            einsum(eq, a, b)
        e1.record()
        torch.cuda.synchronize()
        loop = e0.elapsed_time(e1) / n
    finally:
        if old is None:
            os.environ.pop("EINSUM_BUILD_DIR", None)
        else:
            os.environ["EINSUM_BUILD_DIR"] = old
        pb.clear_runner_cache()
        shutil.rmtree(tmp, ignore_errors=True)
    row = dict(equation=f"{eq} float32 (256, 257) x (257, 255)", first_call_ms=round(first * 1e3, 2),
               reload_call_ms=round(reload * 1e3, 2), cached_call_host_us=round(host * 1e6, 1),
               cached_call_loop_us=round(loop * 1e3, 1))
    log(f"bench: einsum() first call {first * 1e3:.1f} ms (plan + compile + load), after a runner-cache clear "
        f"{reload * 1e3:.1f} ms, cached call {host * 1e6:.1f} us host, {loop * 1e3:.1f} us per call back to back")
    return row


def launch_floor(dev, config1_row):
    """Per-launch time of the launch probe (one wave storing one float)
    replayed in a graph with as many launches as config 1's rotation, the
    floor config 1's 256^3 GEMM is read against."""
    import torch

    from pto_einsum import abi

    lib = abi.bind()
    nsets = config1_row["sets"] if config1_row else 1024
    bufs = [(torch.empty(64, dtype=torch.float32, device=dev),) for _ in range(nsets)]

    def call(buf):
        rc = lib.pe_probe_launch(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError("launch probe failed")

    ms = time_graph(call, bufs)
    row = dict(kernel="launch probe (one wave, one store)", us=round(ms * 1e3, 2), launches_per_replay=nsets)
    if config1_row:
        row["config1_us"] = config1_row["us"]
        row["config1_over_floor_us"] = round(config1_row["us"] - ms * 1e3, 2)
    log(f"bench: launch floor {ms * 1e3:.2f} us per launch in a graph of {nsets}")
    return row


# -------------------------------------------------------------------- main --

def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the contraction would shard on its batch axes with no exchange between GPUs).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    groups = all_cases()
    if args.list_cases:
        for grp, cases in groups.items():
            for c in cases:
                print(f"{grp}: {c.name}")
        return
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_probe:
        copy_probe()
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.profile:
        found = [c for cs in groups.values() for c in cs if c.name == args.profile]
        if not found:
            sys.exit(f"bench.py: no case {args.profile!r} (see --list-cases)")
        warm = measure(found[0], dev, args.steps, args.warmup, profile_calls=max(1, args.steps))
        print(json.dumps({"profiled": args.profile, "calls": max(1, args.steps), "warm_calls": warm}))
        return

    # ---- headline: config 2, rotated operand sets ----
    head = groups["headline"][0]
    call, operands, set_bytes = head.prepare(dev)
    nsets = n_sets(set_bytes)
    sets = replicate(operands, nsets)
    a, b = operands[:2]
    eq = "bji,bjk->bik"
    log(f"bench: config 2 {eq} {tuple(a.shape)} x {tuple(b.shape)} float32, {nsets} rotated operand sets")
    per, total_ms = time_runner(call, sets, args.steps, args.warmup)
    flops, nbytes = work(eq, a, b)
    ms_per_step = total_ms / args.steps
    kernel_ms = statistics.mean(per)
    roof, _, _ = roofline(flops, nbytes, kernel_ms, "f32")
    roof["traffic"], roof["traffic_source"] = traffic_from_profile()
    roof["kernel_us"] = round(kernel_ms * 1e3, 2)
    value = flops / (ms_per_step * 1e-3) / 1e12
    log(f"bench: config 2 {ms_per_step * 1e3:.1f} us/step, kernel {kernel_ms * 1e3:.1f} us, {value:.2f} TFLOP/s")
    del sets, operands, call
    torch.cuda.empty_cache()

    rows = {k: [] for k in groups if k != "headline"}
    rows["attainable"] = attainable(dev)
    if not args.no_configs:
        for grp in ("per_config", "transposes", "large_f16", "gdn", "solo_reduce"):
            for case in groups[grp]:
                rows[grp].append(measure(case, dev, args.steps, args.warmup))
        pc = rows["per_config"]
        chain = sum(c["us"] for c in pc if c["config"] in ("5.1", "5.2", "5.3"))
        for c in pc:
            if c["config"].startswith("5.F"):
                c["three_einsums_us"] = round(chain, 2)
        rows["large_f16"] += time_torch_matmul(dev)
        rows["vendor_thin"] = time_torch_thin(dev)
        rows["gdn_stages"] = time_gdn_stages(dev, args.steps)
        rows["launch_floor"] = launch_floor(dev, next((r for r in pc if r["config"] == "1"), None))
        rows["cold_call"] = cold_call(dev)

    cpu = None
    if not args.no_cpu:
        log("bench: timing the CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"bench: cpu baseline {cpu}")
        if not args.no_configs:
            cpu_per_config(rows["per_config"], groups["per_config"])

    line = {
        "metric": "einsum TFLOP/s & HBM GB/s as % of MI355X roofline, per equation",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": (f"synthetic (seeded standard-normal operands, resident in HBM; {nsets} operand sets "
                 f"rotated per step, >= 1 GiB, so no step reads the Infinity Cache's copy)"),
        "config": {"workload": "config 2: bji,bjk->bik float32 b=16 i=1000 j=777 k=1536",
                   "equation": eq, "shapes": [list(a.shape), list(b.shape)], "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    line.update(rows)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
