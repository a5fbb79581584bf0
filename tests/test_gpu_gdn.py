"""The GDN contraction set on the GPU, and graph capture of its stages.

The four contractions of the reference's chunked GDN forward
(benchmarks/complex/gdn/einsum_gdn.py:94,197,221-222,266,276,327-336):

    kkt / chunk_o qk     bihd,bjhd->bihj   (NT read: contraction innermost in both)
    wy_fast / intra      bihj,bjhd->bihd   (NN read with a strided k row)
    chunk_h kv           bvhd,bvhe->bhde   (TN read: A transposed)
    chunk_h ws / inter   bvhd,bhde->bvhe   (NN read, batch axes split around the rows)

at the reference's base-benchmark shapes (benchmarks/base/bench_einsum.py:129-157:
b folded chunks in {8, 16, 32, 64}, chunk = d = 128, H = 16) and its
IMPLEMENTATION.md:700-782 sizes (b x H = 16x16, 64x16, 16x48); determinism as
the reference's test_*_strided_input_deterministic (8 runs, torch.equal); and
the stage sequences captured with ``StageGraph`` and replayed, each replay
bit-identical to eager calls on the same inputs."""
import numpy as np
import pytest
import torch

import oracle
from parity_util import RTOL, check, ref64_gpu

pytestmark = pytest.mark.gpu

GDN_EQS = ["bihd,bjhd->bihj", "bihj,bjhd->bihd", "bvhd,bvhe->bhde", "bvhd,bhde->bvhe"]


def _shapes(eq, b, H, C=128, D=128):
    if eq == "bvhd,bhde->bvhe":
        return (b, C, H, D), (b, H, D, D)
    return (b, C, H, D), (b, C, H, D)


def _inputs(eq, b, H, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    s0, s1 = _shapes(eq, b, H)
    return ((torch.randn(s0, generator=g) * 128 ** -0.5).to(dtype),
            (torch.randn(s1, generator=g) * 128 ** -0.5).to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq", GDN_EQS)
def test_gdn_contraction_full_oracle(eq, dtype):
    """b = 8 folded chunks, H = 16: every element against the oracle."""
    from pto_einsum import einsum

    a, b = _inputs(eq, 8, 16, dtype, seed=GDN_EQS.index(eq))
    print(f"gdn {eq} {tuple(a.shape)} x {tuple(b.shape)} {dtype}", flush=True)
    got = einsum(eq, a.cuda(), b.cuda()).cpu().numpy()
    check(got, oracle.einsum(eq, a.float().numpy(), b.float().numpy()), False, RTOL[dtype], eq)


@pytest.mark.parametrize("b,H", [(64, 16), (16, 48), (32, 16)])
@pytest.mark.parametrize("eq", GDN_EQS)
def test_gdn_contraction_reference_sizes(eq, b, H):
    """The reference's benchmark sizes in float32: every element against a
    float64 GPU evaluation, sampled elements against the oracle's exact sums."""
    from pto_einsum import einsum

    a, bb = _inputs(eq, b, H, torch.float32, seed=b * 100 + H)
    print(f"gdn {eq} {tuple(a.shape)} x {tuple(bb.shape)}", flush=True)
    got = einsum(eq, a.cuda(), bb.cuda())
    ref = ref64_gpu(eq, a.cuda(), bb.cuda())
    err = float((got.double() - ref).abs().max())
    assert err <= 1e-4 * float(ref.abs().max())
    idx = np.random.default_rng(b + H).integers(0, got.numel(), 2048)
    want = oracle.sampled(eq, a.numpy(), bb.numpy(), idx)
    check(got.flatten()[torch.from_numpy(idx).cuda()].cpu().numpy(), want, False, 1e-4, eq)


@pytest.mark.parametrize("eq", GDN_EQS)
def test_gdn_contraction_deterministic(eq):
    from pto_einsum import EinsumBuilder

    a, b = _inputs(eq, 16, 16, torch.float32, seed=7)
    run = EinsumBuilder(eq, [tuple(a.shape), tuple(b.shape)], torch.float32).build()
    a, b = a.cuda(), b.cuda()
    first = run(a, b)
    for _ in range(7):
        assert torch.equal(run(a, b), first)


def _stages(q, k, v):
    """The folded-batch contraction stages of one GDN forward, in dependency
    order (the gating and masking between them left out)."""
    from pto_einsum import einsum

    A = einsum("bihd,bjhd->bihj", k, k)          # kkt
    u = einsum("bihj,bjhd->bihd", A, v)          # wy_fast u
    w = einsum("bihj,bjhd->bihd", A, k)          # wy_fast w
    kv = einsum("bvhd,bvhe->bhde", k, v)         # chunk_h kv
    qh = einsum("bvhd,bhde->bvhe", q, kv)        # chunk_o inter
    qk = einsum("bihd,bjhd->bihj", q, k)         # chunk_o qk
    intra = einsum("bihj,bjhd->bihd", qk, v)     # chunk_o intra
    return A, u, w, kv, qh, qk, intra


def test_stage_graph_replays_match_eager():
    from pto_einsum import StageGraph, einsum

    g = torch.Generator().manual_seed(21)
    shape = (16, 128, 16, 128)
    q, k, v = ((torch.randn(shape, generator=g) * 128 ** -0.5).cuda() for _ in range(3))
    graph = StageGraph(lambda: _stages(q, k, v))
    for rep in range(3):
        # new inputs in place, then eager work of its own between replays
        for t in (q, k, v):
            t.copy_(torch.randn(shape, generator=g) * 128 ** -0.5)
        other = einsum("bihd,bjhd->bihj", v, q)
        torch.cuda.synchronize()
        eager = _stages(q, k, v)
        got = graph.replay()
        torch.cuda.synchronize()
        print(f"stage graph replay {rep}", flush=True)
        for name, x, y in zip(("A", "u", "w", "kv", "qh", "qk", "intra"), got, eager):
            assert torch.equal(x, y), f"replay {rep}: stage {name} differs from eager"
        assert torch.isfinite(other).all()
    # and the first stage against the oracle
    check(got[0].cpu().numpy(), oracle.einsum("bihd,bjhd->bihj", k.cpu().numpy(), k.cpu().numpy()),
          False, 1e-4, "kkt")


def _chunk_h(w, u, k, gexp, gdecay, S0, C=128):
    """The chunk_h recurrence (einsum_gdn.py:255-280) with the gates given as
    tensors: per chunk, ws = w_c . S; v_c = u_c - ws; kv = k_c^T . (v_c * gexp_c);
    S = gdecay_c * S + kv.  Returns the new values and the final state."""
    from pto_einsum import einsum

    S = S0
    vs = []
    for c in range(w.shape[1] // C):
        rows = slice(c * C, (c + 1) * C)
        ws = einsum("bvhd,bhde->bvhe", w[:, rows], S)
        vc = u[:, rows] - ws
        vs.append(vc)
        kv = einsum("bvhd,bvhe->bhde", k[:, rows], vc * gexp[:, rows])
        S = gdecay[c] * S + kv
    return torch.cat(vs, dim=1), S


def _chunk_h_ref64(w, u, k, gexp, gdecay, S0, C=128):
    S = S0.double()
    vs = []
    for c in range(w.shape[1] // C):
        rows = slice(c * C, (c + 1) * C)
        wc, kc = w[:, rows].double(), k[:, rows].double()
        ws = (wc.permute(0, 2, 1, 3) @ S).permute(0, 2, 1, 3)
        vc = u[:, rows].double() - ws
        vs.append(vc)
        vsc = (vc * gexp[:, rows].double()).permute(0, 2, 1, 3).contiguous()
        kv = kc.permute(0, 2, 3, 1).contiguous() @ vsc
        S = gdecay[c].double() * S + kv
    return torch.cat(vs, dim=1), S


@pytest.mark.parametrize("B", [1, 2])
def test_chunk_h_recurrence_graph(B):
    """A launch-bound sequential stage: 2 contractions and 4 elementwise ops
    per chunk, 8 chunks, captured as one graph; replays equal eager calls and
    agree with a float64 evaluation."""
    from pto_einsum import StageGraph

    g = torch.Generator().manual_seed(30 + B)
    T, H, D = 1024, 32, 128
    w = (torch.randn(B, T, H, D, generator=g) * D ** -0.5).cuda()
    u = torch.randn(B, T, H, D, generator=g).cuda()
    k = (torch.randn(B, T, H, D, generator=g) * D ** -0.5).cuda()
    gexp = (0.5 + 0.5 * torch.rand(B, T, H, 1, generator=g)).cuda()
    gdecay = (0.5 + 0.5 * torch.rand(T // 128, B, H, 1, 1, generator=g)).cuda()
    S0 = torch.zeros(B, H, D, D, device="cuda")
    print(f"chunk_h recurrence B={B} T={T} H={H}", flush=True)
    graph = StageGraph(lambda: _chunk_h(w, u, k, gexp, gdecay, S0))
    for rep in range(3):
        u.copy_(torch.randn(B, T, H, D, generator=g))
        torch.cuda.synchronize()
        eager = _chunk_h(w, u, k, gexp, gdecay, S0)
        got = graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got[0], eager[0]) and torch.equal(got[1], eager[1]), f"replay {rep} differs"
    vref, Sref = _chunk_h_ref64(w, u, k, gexp, gdecay, S0)
    for x, r in ((got[0], vref), (got[1], Sref)):
        err = float((x.double() - r).abs().max())
        assert err <= 1e-4 * float(r.abs().max()), err


def test_linear_attention_graph():
    from pto_einsum import StageGraph, linear_attention

    g = torch.Generator().manual_seed(40)
    T, S, N, P = 500, 700, 128, 128
    q = (torch.randn(T, N, generator=g) * N ** -0.5).half().cuda()
    k = (torch.randn(S, N, generator=g) * N ** -0.5).half().cuda()
    v = torch.randn(S, P, generator=g).cuda()
    m = torch.tril(torch.rand(T, S, generator=g)).cuda()
    graph = StageGraph(lambda: linear_attention(q, k, v, m))
    for rep in range(3):
        v.copy_(torch.randn(S, P, generator=g))
        torch.cuda.synchronize()
        eager = linear_attention(q, k, v, m)
        got = graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {rep} differs"


def test_random_einsum_sequences_replay_bit_identical():
    """30 seeded random sequences of two to five einsums (tests/random_einsum.py:
    product, direct, staged and split-K GEMM routes, single-operand reduction
    axes, both dtypes) captured by StageGraph and replayed three times with
    new inputs written in place: every output of every replay equals an
    eager call on the same inputs bit for bit."""
    import random

    from pto_einsum import StageGraph, einsum
    from random_einsum import random_case

    rng = random.Random(5)
    for it in range(30):
        cases = []
        for _ in range(rng.choice([2, 3, 5])):
            eq, s0, s1, solo = random_case(rng, solo=True, max_elems=3e5, max_work=2e7)
            cases.append((eq, s0, s1, solo, rng.choice([torch.float32, torch.float16])))
        print(f"graph sequence {it}: " + "; ".join(c[0] for c in cases), flush=True)
        ins = [(torch.rand(c[1], device="cuda").to(c[4]), torch.rand(c[2], device="cuda").to(c[4])) for c in cases]

        def fn():
            return [einsum(c[0], a, b, reduce_solo_axes=c[3]) for c, (a, b) in zip(cases, ins)]

        graph = StageGraph(fn)
        for rep in range(3):
            for a, b in ins:
                a.copy_(torch.rand(a.shape, device="cuda").to(a.dtype))
                b.copy_(torch.rand(b.shape, device="cuda").to(b.dtype))
            graph.replay()
            torch.cuda.synchronize()
            eager = fn()
            torch.cuda.synchronize()
            for k, (got, want) in enumerate(zip(graph.outputs, eager)):
                assert torch.equal(got, want), f"sequence {it} replay {rep} output {k}"
