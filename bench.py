"""Benchmark of the MI355X einsum path (one JSON line on stdout).

Headline workload: BASELINE config 2, the transposing batched contraction
``bji,bjk->bik`` in float32 with b=16, i=1000, j=777, k=1536 (standard-normal
inputs from a seed).  A step is one ``run_einsum_exec`` over that batch with
operands and output resident in HBM.  ``value`` is TFLOP/s over the timed
steps (2*b*i*j*k flops per step).  ``roofline`` relates the GEMM kernel's
average launch time (HIP events recorded around each launch on the launch
stream) to the float32 MFMA peak.  ``cpu_baseline`` times the reference CPU
route (cpu_einsum.h compiled by oracle/ref_build.py; the C restatement in
oracle/ when that build is absent) on one of the 16 batches.

``per_config`` adds every other BASELINE equation at full size with its own
binding roof (HBM bytes or MFMA flops).  Those kernels run for tens of
microseconds, less than one Python-level call costs, so each is captured once
in a HIP graph and the graph is replayed between two events: the figure is the
GPU time of the einsum's launches.

``large_f16`` times 8192^3 float16 contractions (float32 output) in the
NN and NT layouts on the dense float16 MFMA roof, with torch.matmul (the
vendor library, float16 output) beside them.

``gdn`` times the GDN contraction set at the reference's sizes the same way,
and ``gdn_stages`` two of its stage sequences issued eagerly (one Python call
per launch) and replayed as one HIP graph (``pto_einsum.StageGraph``).

``roofline.traffic`` (HBM bytes per launch of the headline GEMM) is read from
profiles/gemm_f32_config2_traffic.json, written from two rocprofv3 --pmc runs
(FETCH_SIZE, WRITE_SIZE) of this script, scaled by the same counters on
``--copy-probe`` (a plain copy of known size).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-configs]
       python bench.py --copy-probe     # counter calibration: one 1 GiB copy
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pto-einsum_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"f32": 157.3, "f16": 2516.6}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-configs", action="store_true", help="headline workload only")
    ap.add_argument("--cpu-sample-batches", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-time budget of the CPU-baseline sample")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run a plain 1 GiB device copy (counter calibration) and exit")
    return ap.parse_args()


def time_runner(run, a, b, steps, warmup):
    """Per-launch HIP-event times (ms) and wall time of the timed region."""
    import torch

    for _ in range(warmup):
        run(a, b)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for s, e in ev:
        s.record(stream)
        run(a, b)
        e.record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in ev]
    return per, t0.elapsed_time(t1)


def time_graph(run, a, b, steps, warmup, out_bytes):
    """GPU time (ms) of one einsum: `reps` calls are captured in one HIP graph
    (graph launch overhead paid once per replay), the graph is replayed
    `steps` times between events, and the median per-call time is returned."""
    import torch

    reps = int(max(1, min(20, (8 << 30) // max(1, out_bytes))))
    for _ in range(max(2, warmup)):
        run(a, b)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            run(a, b)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(max(3, steps // 4)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / reps)
    del g
    torch.cuda.empty_cache()
    return statistics.median(per)


def copy_probe():
    """A 1 GiB float32 copy through the core library's permutation launcher
    (identity permutation = plain copy): reads and writes exactly 1 GiB."""
    import ctypes

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


def traffic_from_profile():
    path = os.path.join(ROOT, "profiles", "gemm_f32_config2_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def config_list():
    import torch

    def randn(shape, g, scale=1.0, dtype=torch.float32):
        return (torch.randn(shape, generator=g) * scale).to(dtype)

    def decay(t, gamma):
        i = torch.arange(t, dtype=torch.float64)
        d = (i[:, None] - i[None, :])
        return torch.where(d >= 0, gamma ** d.clamp(min=0), torch.zeros(())).float()

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
    and Phase C of pto_einsum.h:52-177) for the BASELINE contractions that
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


def time_transposes(dev, steps, warmup):
    """GPU time of each standalone transpose (HIP graph replay, as for the
    per-config figures) with its HBM roof: one read and one write of every
    element."""
    import torch

    from pto_einsum import EinsumBuilder

    rows = []
    for label, eq, shapes, dtype, entry in transpose_list():
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

        def run(a, b, fn=fn, x=x, y=y):
            rc = fn(ctypes.cast(x.data_ptr(), fn.argtypes[0]), ctypes.cast(y.data_ptr(), fn.argtypes[1]),
                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if rc != 0:
                raise RuntimeError(f"{entry} failed ({rc})")

        km = time_graph(run, None, None, max(10, steps), max(3, warmup // 2), y.numel() * y.element_size())
        nbytes = 2 * x.numel() * x.element_size()
        gbs = nbytes / (km * 1e-3) / 1e9
        rows.append(dict(transpose=label, equation=eq, dtype=str(src_dtype).replace("torch.", ""),
                         shape=list(src_shape), perm=list(perm), us=round(km * 1e3, 2), gbs=round(gbs, 1),
                         roof="hbm", frac=round(gbs / PEAK_HBM_GBS, 4)))
        log(f"bench: transpose {label} of {eq} {src_shape} {km * 1e3:.1f} us  {gbs:.0f} GB/s  "
            f"hbm {gbs / PEAK_HBM_GBS * 100:.1f}%")
        del x, y, builder
        torch.cuda.empty_cache()
    return rows


def time_fused_chain(dev, steps, warmup):
    """BASELINE config 5's linear-attention chain in one fused launch
    (pto_einsum.linear_attention): q, k float16 normal(0, 1/sqrt(128)), v
    float16 normal(0, 1), the causal decay mask gamma^(t-s), gamma = 0.995,
    in float32; t = s = 4096, n = p = 128.  The default launch computes P.V
    as three bfloat16 MFMA terms of the split P and V; ``precise_us`` is the
    same chain with P.V on float32 MFMAs.  The roof is the larger of the
    compulsory HBM bytes (q, k, v, m read once, out written once) at 8 TB/s
    and the MFMAs the default launch issues for the dense chain (2*T*S*N
    float16 flops plus 3 * 2*T*S*P bfloat16 flops at the 16-bit peak); masked
    blocks that are zero are skipped, so the causal case does less."""
    import torch

    from pto_einsum import linear_attention

    T = S = 4096
    N = P = 128
    g = torch.Generator().manual_seed(105)
    q = (torch.randn(T, N, generator=g) * N ** -0.5).half().to(dev)
    k = (torch.randn(S, N, generator=g) * N ** -0.5).half().to(dev)
    v = torch.randn(S, P, generator=g).half().to(dev)
    i = torch.arange(T, dtype=torch.float64)
    d = i[:, None] - i[None, :]
    m = torch.where(d >= 0, 0.995 ** d.clamp(min=0), torch.zeros(())).float().to(dev)
    km = time_graph(lambda a, b: linear_attention(q, k, v, m), None, None, max(10, steps), max(3, warmup // 2),
                    T * P * 4)
    kp = time_graph(lambda a, b: linear_attention(q, k, v, m, precise=True), None, None, max(10, steps),
                    max(3, warmup // 2), T * P * 4)
    flops = 2 * T * S * N + T * S + 2 * T * S * P
    nbytes = (q.numel() + k.numel() + v.numel()) * 2 + m.numel() * 4 + T * P * 4
    hbm_ms = nbytes / (PEAK_HBM_GBS * 1e9) * 1e3
    mfma_ms = (2 * T * S * N + 3 * 2 * T * S * P) / (PEAK_TFLOPS["f16"] * 1e12) * 1e3
    floor_ms = max(hbm_ms, mfma_ms)
    return dict(config="5.F", equation="tn,sn,sp,ts->tp (fused)", dtype="f16 q/k, f32 chain (P.V as 3 bf16 terms)",
                us=round(km * 1e3, 2), tflops=round(flops / (km * 1e-3) / 1e12, 3),
                gbs=round(nbytes / (km * 1e-3) / 1e9, 1), roof="hbm" if hbm_ms >= mfma_ms else "mfma",
                frac=round(floor_ms / km, 4), precise_us=round(kp * 1e3, 2))


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


def time_eager(fn, iters):
    """GPU-side time (ms) per call of `fn` issued back to back from Python:
    events around the whole loop, so host gaps between launches count."""
    import torch

    for _ in range(2):
        fn()
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
    graph.replay()
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


def time_gdn(dev, steps, warmup):
    """Per-contraction GPU times of the GDN set, then two stage sequences
    issued eagerly (one Python call per launch) and as one StageGraph replay:
    the seven folded-batch contractions of one GDN forward (b = 16, H = 16)
    and the chunk_h recurrence (B = 1, T = 1024, H = 32: per chunk two
    contractions and four elementwise ops, eight chunks in sequence)."""
    import torch

    from pto_einsum import EinsumBuilder, einsum

    rows = []
    for label, eq, s0, s1 in gdn_list():
        g = torch.Generator().manual_seed(200 + len(rows))
        x = (torch.randn(s0, generator=g) * 128 ** -0.5).to(dev)
        y = (torch.randn(s1, generator=g) * 128 ** -0.5).to(dev)
        r = EinsumBuilder(eq, [s0, s1], torch.float32).build()
        f, nb = work(eq, x, y)
        km = time_graph(r, x, y, max(10, steps), max(3, warmup // 2), r(x, y).numel() * 4)
        rf, tf, gb = roofline(f, nb, km, "f32")
        rows.append(dict(gdn=label, equation=eq, dtype="f32", shapes=[list(s0), list(s1)], us=round(km * 1e3, 2),
                         tflops=round(tf, 3), gbs=round(gb, 1), roof=rf["bound"], frac=rf["frac"]))
        log(f"bench: gdn {label} {eq} {km * 1e3:.1f} us  {tf:.2f} TFLOP/s  {gb:.0f} GB/s  "
            f"{rf['bound']} {rf['frac'] * 100:.1f}%")
        del x, y, r

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
    return rows, seqs


def rope_table(s, d):
    import torch

    pos = torch.arange(s, dtype=torch.float64)[:, None]
    i = torch.arange(d, dtype=torch.float64)[None, :] % (d // 2)
    theta = 10000.0 ** (-2.0 * i / d)
    return torch.cos(pos * theta).to(torch.float16)


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


def time_large_f16(dev, steps, warmup):
    """Large float16 contractions (float32 output): the north star's
    "large fp16 contractions" on the dense float16 MFMA roof, with torch's
    matmul (the vendor library, float16 output) timed beside them."""
    import torch

    from pto_einsum import EinsumBuilder

    out = []
    n = 8192
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(n, n, generator=g) / 64).half().to(dev)
    y = (torch.randn(n, n, generator=g) / 64).half().to(dev)
    for eq, label in (("ij,jk->ik", "NN"), ("ik,jk->ij", "NT")):
        r = EinsumBuilder(eq, [tuple(x.shape), tuple(y.shape)], torch.float16).build()
        f, nb = work(eq, x, y)
        km = time_graph(r, x, y, max(5, steps // 2), max(2, warmup // 2), r(x, y).numel() * 4)
        rf, tf, gb = roofline(f, nb, km, "f16")
        out.append(dict(shape=f"{n}^3 {label}", equation=eq, dtype="f16", us=round(km * 1e3, 1),
                        tflops=round(tf, 1), roof=rf["bound"], frac=rf["frac"]))
        log(f"bench: large f16 {eq} {km * 1e3:.1f} us {tf:.1f} TFLOP/s ({rf['frac'] * 100:.1f}% of fp16 MFMA)")
        del r
        torch.cuda.empty_cache()
    yt = y.t().contiguous()
    for label, fn in (("NN", lambda: torch.matmul(x, y)), ("NT", lambda: torch.matmul(x, yt.t()))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / 10
        tf = 2 * n ** 3 / t / 1e9
        out.append(dict(shape=f"{n}^3 {label}", equation="torch.matmul (float16 output)", dtype="f16",
                        us=round(t * 1e3, 1), tflops=round(tf, 1), roof="mfma",
                        frac=round(tf / PEAK_TFLOPS["f16"], 4)))
        log(f"bench: torch.matmul f16 {label} {t * 1e3:.1f} us {tf:.1f} TFLOP/s")
    del x, y, yt
    torch.cuda.empty_cache()
    return out


def cpu_baseline(nbatch, budget_s=10.0, max_reps=30):
    """Reference CPU route on `nbatch` of config 2's 16 batches, 1 thread,
    called repeatedly for about `budget_s` seconds (median call time)."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import ref_build

    eq, s0, s1 = "bji,bjk->bik", (nbatch, 777, 1000), (nbatch, 777, 1536)
    g = torch.Generator().manual_seed(1)
    a = torch.randn(s0, generator=g).numpy()
    b = torch.randn(s1, generator=g).numpy()
    if os.path.exists(ref_build.so_path(eq, s0, s1)):
        kind = "reference"
        fn = lambda: ref_build.run(eq, a, b)  # noqa: E731
    else:
        kind = "port"
        fn = lambda: oracle.einsum(eq, a, b)  # noqa: E731
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start) < budget_s:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    dt = statistics.median(times)
    flops = 2.0 * nbatch * 1000 * 1536 * 777
    return dict(value=round(flops / dt / 1e12, 6), unit="TFLOP/s", cores=1, kind=kind,
                sample=(f"{nbatch} of 16 batches of config 2 (bji,bjk->bik float32, j=777, i=1000, "
                        f"k=1536), {flops / 1e9:.2f} GFLOP per call, called {len(times)} times "
                        f"({sum(times):.1f} s); median call {dt:.3f} s on 1 thread of {os.cpu_count()}"),
                seconds=round(sum(times), 3))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the contraction would shard on its batch axes with no exchange between GPUs).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from pto_einsum import EinsumBuilder

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_probe:
        copy_probe()
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---- headline: config 2 ----
    eq, s0, s1 = "bji,bjk->bik", (16, 777, 1000), (16, 777, 1536)
    g = torch.Generator().manual_seed(2)
    a = torch.randn(s0, generator=g).to(dev)
    b = torch.randn(s1, generator=g).to(dev)
    log(f"bench: building {eq} {s0} x {s1} float32")
    builder = EinsumBuilder(eq, [s0, s1], torch.float32)
    run = builder.build()
    log(f"bench: plan {builder.launch_plan.gemm} staged={builder.launch_plan.gather0 or builder.launch_plan.gather1 or builder.launch_plan.scatter_out}")
    per, total_ms = time_runner(run, a, b, args.steps, args.warmup)
    flops, nbytes = work(eq, a, b)
    ms_per_step = total_ms / args.steps
    kernel_ms = statistics.mean(per)
    roof, _, _ = roofline(flops, nbytes, kernel_ms, "f32")
    roof["traffic"] = traffic_from_profile()
    value = flops / (ms_per_step * 1e-3) / 1e12
    log(f"bench: config 2 {ms_per_step * 1e3:.1f} us/step, kernel {kernel_ms * 1e3:.1f} us, {value:.2f} TFLOP/s")

    per_config = []
    if not args.no_configs:
        for name, ceq, gen, dt in config_list():
            gg = torch.Generator().manual_seed(100 + len(per_config))
            x, y = gen(gg)
            x, y = x.to(dev), y.to(dev)
            r = EinsumBuilder(ceq, [tuple(x.shape), tuple(y.shape)], x.dtype).build()
            f, nb = work(ceq, x, y)
            km = time_graph(r, x, y, max(10, args.steps), max(3, args.warmup // 2),
                            r(x, y).numel() * 4)
            rf, tf, gb = roofline(f, nb, km, dt)
            per_config.append(dict(config=name, equation=ceq, dtype=dt, us=round(km * 1e3, 2),
                                   tflops=round(tf, 3), gbs=round(gb, 1), roof=rf["bound"],
                                   frac=rf["frac"]))
            log(f"bench: config {name} {ceq} {km * 1e3:.1f} us  {tf:.2f} TFLOP/s  {gb:.0f} GB/s  "
                f"{rf['bound']} {rf['frac'] * 100:.1f}%")
            del x, y, r
            torch.cuda.empty_cache()

    if not args.no_configs:
        fused = time_fused_chain(dev, args.steps, args.warmup)
        chain_us = sum(c["us"] for c in per_config if c["config"] in ("5.1", "5.2", "5.3"))
        fused["three_einsums_us"] = round(chain_us, 2)
        per_config.append(fused)
        log(f"bench: config 5 fused tn,sn,sp,ts->tp {fused['us']:.1f} us ({fused['tflops']:.1f} TFLOP/s "
            f"dense-equivalent, {fused['roof']} {fused['frac'] * 100:.1f}%; float32 P.V {fused['precise_us']:.1f} us); "
            f"the three einsums take {chain_us:.1f} us")

    transposes = [] if args.no_configs else time_transposes(dev, args.steps, args.warmup)
    large_f16 = [] if args.no_configs else time_large_f16(dev, args.steps, args.warmup)
    gdn, gdn_stages = ([], []) if args.no_configs else time_gdn(dev, args.steps, args.warmup)

    log("bench: timing the CPU baseline")
    cpu = cpu_baseline(args.cpu_sample_batches, args.cpu_seconds)
    log(f"bench: cpu baseline {cpu}")

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
        "data": "synthetic (seeded standard-normal operands, resident in HBM)",
        "config": {"workload": "config 2: bji,bjk->bik float32 b=16 i=1000 j=777 k=1536",
                   "equation": eq, "shapes": [list(s0), list(s1)], "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_config": per_config,
        "transposes": transposes,
        "large_f16": large_f16,
        "gdn": gdn,
        "gdn_stages": gdn_stages,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
