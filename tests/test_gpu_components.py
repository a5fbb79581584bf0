"""Component entry points on the GPU: the per-shape run_transpose_* /
run_batched_matmul / run_einsum symbols (test_matmul.py:24-147 of the
reference) and the core permutation launcher on the reference's transpose
matrix (test_transpose.py:108-161), all through the C ABI."""
import ctypes
import itertools

import numpy as np
import pytest
import torch

import oracle
from parity_util import check
from pto_einsum import EinsumBuilder, abi, launch, runtime
from test_launch import EXTRA
from test_oracle import TRANSPOSE_CASES

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", [("ij,jk->ik", (32, 64), (64, 128)),
                                      ("bji,bjk->bik", (3, 37, 50), (3, 37, 41)),
                                      ("bshd,bthd->bsht", (2, 24, 3, 16), (2, 20, 3, 16)),
                                      ("ij,jk->ki", (33, 20), (20, 47))])
def test_staged_components(eq, s0, s1, dtype, build_dir):
    builder = EinsumBuilder(eq, [s0, s1], dtype)
    builder.build()
    lib = builder.lib
    r = builder.recipe
    g = torch.Generator().manual_seed(1)
    x, y = torch.rand(s0, generator=g).to(dtype), torch.rand(s1, generator=g).to(dtype)
    if builder._swap_operands:
        x, y = y, x
    p0, p1 = r["in_transpose_idxs"]
    t0 = torch.empty([x.shape[i] for i in p0], dtype=dtype, device="cuda")
    t1 = torch.empty([y.shape[i] for i in p1], dtype=dtype, device="cuda")
    xc, yc = x.cuda(), y.cuda()
    assert lib.run_transpose_inp0(ctypes.cast(_ptr(xc), ctypes.POINTER(builder.c_type)),
                                  ctypes.cast(_ptr(t0), ctypes.POINTER(builder.c_type)), _stream()) == 0
    assert lib.run_transpose_inp1(ctypes.cast(_ptr(yc), ctypes.POINTER(builder.c_type)),
                                  ctypes.cast(_ptr(t1), ctypes.POINTER(builder.c_type)), _stream()) == 0
    assert torch.equal(t0.cpu(), x.permute(p0).contiguous())
    assert torch.equal(t1.cpu(), y.permute(p1).contiguous())
    I, L0, L1, C = r["I"], r["L0"], r["L1"], r["C"]
    res = torch.empty(I * L0 * L1, dtype=torch.float32, device="cuda")
    rc = lib.run_batched_matmul(ctypes.cast(_ptr(t0), ctypes.POINTER(builder.c_type)),
                                ctypes.cast(_ptr(t1), ctypes.POINTER(builder.c_type)),
                                ctypes.cast(_ptr(res), ctypes.POINTER(ctypes.c_float)), _stream())
    assert rc == 0
    want = oracle.bmm(t0.float().cpu().numpy().reshape(I, L0, C), t1.float().cpu().numpy().reshape(I, C, L1))
    check(res.cpu().numpy().reshape(I, L0, L1), want, False, 1e-4 if dtype == torch.float32 else 2e-3, "bmm")
    out = torch.empty(r["out_shape"], dtype=torch.float32, device="cuda")
    rc = lib.run_transpose_out(ctypes.cast(_ptr(res), ctypes.POINTER(ctypes.c_float)),
                               ctypes.cast(_ptr(out), ctypes.POINTER(ctypes.c_float)), _stream())
    assert rc == 0
    assert torch.equal(out.cpu(), res.cpu().reshape(r["out_interpret_shape"]).permute(r["out_transpose_idxs"]))
    # One-shot entry point (setup + exec + sync + teardown).
    out2 = torch.empty(r["out_shape"], dtype=torch.float32, device="cuda")
    assert lib.run_einsum(ctypes.cast(_ptr(xc), ctypes.POINTER(builder.c_type)),
                          ctypes.cast(_ptr(yc), ctypes.POINTER(builder.c_type)),
                          ctypes.cast(_ptr(out2), ctypes.POINTER(ctypes.c_float)), _stream()) == 0
    user0, user1 = (y, x) if builder._swap_operands else (x, y)
    want_full = oracle.einsum(eq, user0.float().numpy(), user1.float().numpy())
    check(out2.cpu().numpy(), want_full, False, 1e-4 if dtype == torch.float32 else 2e-3, "run_einsum")
    builder.cleanup()


def _permute_gpu(x: torch.Tensor, perm):
    lib = abi.bind()
    d = abi.permute_desc(launch._permute_desc(tuple(x.shape), perm, x.element_size()))
    xc = x.cuda()
    out = torch.empty([x.shape[p] for p in perm], dtype=x.dtype, device="cuda")
    rc = lib.pe_permute(ctypes.byref(d), _ptr(xc), _ptr(out), _stream())
    assert rc == 0, runtime.last_error()
    return out.cpu()


ND = [((2, 3, 4, 5), p) for p in itertools.permutations(range(4))] + [
    ((64, 3, 130), (2, 1, 0)), ((7, 65, 66, 3), (0, 2, 1, 3)), ((5, 129, 2, 67), (3, 1, 2, 0)),
    ((1, 1, 1), (2, 0, 1)), ((4096, 33), (1, 0))]


@pytest.mark.parametrize("shape,perm,dt", TRANSPOSE_CASES + [(s, p, np.float32) for s, p in ND]
                         + [(s, p, np.float16) for s, p in ND[-5:]])
def test_permute_bit_exact(shape, perm, dt):
    x = torch.from_numpy(np.random.default_rng(42).random(shape).astype(dt))
    got = _permute_gpu(x, perm)
    assert torch.equal(got.view(torch.int16 if dt == np.float16 else torch.int32),
                       x.permute(perm).contiguous().view(torch.int16 if dt == np.float16 else torch.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", EXTRA)
def test_staged_plans_on_gpu(eq, s0, s1, dtype, build_dir):
    """Equations whose axis groups force operand gathers / an output
    permutation through the workspace."""
    from parity_util import RTOL, contraction_size, make_inputs
    from pto_einsum import einsum

    a, b = make_inputs(eq, s0, s1, dtype)
    got = einsum(eq, a.cuda(), b.cuda()).cpu().numpy()
    want = oracle.einsum(eq, a.float().numpy(), b.float().numpy())
    check(got, want, contraction_size(eq, s0, s1) <= 1, RTOL[dtype], eq)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("eq,s0,s1", [("abc,cd->adb", (64, 48, 96), (96, 80)),
                                      ("acb,cd->abd", (48, 64, 40), (64, 72)),
                                      ("abcd,de->aebc", (4, 5, 40, 8), (8, 24)),
                                      ("bac,cdb->adb", (3, 40, 72), (72, 20, 3))])
def test_free_axes_made_batch_on_gpu(eq, s0, s1, dtype, build_dir):
    """Free groups that collapse in neither tensor run as one batched GEMM
    storing straight into the output (no workspace), against the oracle."""
    from parity_util import RTOL, make_inputs
    from pto_einsum import einsum

    b = EinsumBuilder(eq, [s0, s1], dtype)
    b.parse_equation()
    b.generate_code()
    lp = b.launch_plan
    assert not (lp.gather0 or lp.gather1 or lp.scatter_out) and lp.ws_bytes == 0
    x, y = make_inputs(eq, s0, s1, dtype)
    got = einsum(eq, x.cuda(), y.cuda()).cpu().numpy()
    want = oracle.einsum(eq, x.float().numpy(), y.float().numpy())
    check(got, want, False, RTOL[dtype], eq)


@pytest.mark.parametrize("eq,s0,s1", [("acb,cd->abd", (48, 64, 6), (64, 72)),    # gathers in0
                                      ("abc,cd->adb", (64, 6, 96), (96, 80)),    # stages the result
                                      ("bsd,d->bsd", (2, 16, 64), (64,))])       # one product launch
def test_phase_skip_leaves_skipped_outputs_unwritten(eq, s0, s1):
    """pe_einsum_exec with skip_phases (the EINSUM_PHASE_STOP ablation): the
    whole plan (0) gives the einsum, and a skipped phase that would write the
    output leaves it as it was (NaN sentinel); skipping only a phase the plan
    does not have changes nothing."""
    from parity_util import make_inputs

    lib = abi.bind()
    b = EinsumBuilder(eq, [s0, s1], torch.float32)
    b.parse_equation()
    b.generate_code()
    lp = b.launch_plan
    plan = abi.einsum_plan(lp)
    x, y = make_inputs(eq, s0, s1, torch.float32)
    x, y = x.cuda(), y.cuda()
    if b._swap_operands:
        x, y = y, x
    ws = lib.pe_einsum_setup(ctypes.byref(plan), _stream())
    assert ws or plan.ws_bytes == 0, runtime.last_error()

    def run(skip):
        plan.skip_phases = skip
        out = torch.full(b.recipe["out_shape"], float("nan"), device="cuda")
        print(f"phase skip {skip}: {eq} {s0} {s1}", flush=True)
        rc = lib.pe_einsum_exec(ctypes.byref(plan), _ptr(x), _ptr(y), _ptr(out), ctypes.c_void_p(ws), _stream())
        assert rc == 0, runtime.last_error()
        torch.cuda.synchronize()
        return out

    full = run(0)
    want = oracle.einsum(eq, *(t.float().cpu().numpy() for t in ((y, x) if b._swap_operands else (x, y))))
    check(full.cpu().numpy(), want, False, 1e-4, eq)
    assert bool(run(7).isnan().all())
    if lp.route == launch.ROUTE_PRODUCT or not lp.scatter_out:
        assert bool(run(2).isnan().all())          # the GEMM / product writes the output
        assert torch.equal(run(4), full)           # no output permutation to skip
    else:
        assert bool(run(4).isnan().all())          # the output permutation writes it
    if lp.route != launch.ROUTE_PRODUCT and not (lp.gather0 or lp.gather1):
        assert torch.equal(run(1), full)           # no gather to skip
    plan.skip_phases = 8
    assert lib.pe_einsum_exec(ctypes.byref(plan), _ptr(x), _ptr(y), _ptr(full), ctypes.c_void_p(ws), _stream()) != 0
    if ws:
        assert lib.pe_einsum_teardown(ctypes.c_void_p(ws)) == 0


def test_operand_row_strides_beyond_32_bit_slab_offsets():
    """A float16 batched GEMM whose A rows are 8.4M elements apart: a 256-row
    slab of A spans more than 2^32 bytes, past the 32-bit per-lane load
    offsets of the 256x256 kernel, so it must run on the 64-bit-addressed
    direct-load kernel.  mbk,bkn->bmn with m = n = 1024, b = 2064, k = 4096
    (17 GB per operand, 8.6 GB out); sampled outputs against float64."""
    from pto_einsum import einsum

    m, b, k, n = 1024, 2064, 4096, 1024
    assert (255 * b * k + 31 + 8) * 2 >= 2 ** 32
    g = torch.Generator(device="cuda").manual_seed(3)
    A = torch.randn(m, b, k, device="cuda", dtype=torch.float16, generator=g)
    B = torch.randn(b, k, n, device="cuda", dtype=torch.float16, generator=g)
    print("einsum mbk,bkn->bmn", (m, b, k), (b, k, n), flush=True)
    out = einsum("mbk,bkn->bmn", A, B)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    for _ in range(48):
        bi, mi, ni = int(rng.integers(b)), int(rng.integers(m)), int(rng.integers(n))
        a_row, b_col = A[mi, bi].double(), B[bi, :, ni].double()
        want = float((a_row * b_col).sum())
        bound = float((a_row.abs() * b_col.abs()).sum())
        assert abs(float(out[bi, mi, ni]) - want) <= 2e-3 * bound, (bi, mi, ni)
    del A, B, out
    torch.cuda.empty_cache()


def _gemm_direct(a, b, M, N, K, a_ms, a_ks, b_ks, b_ns, dtype_code, tile=0, split_k=0, nbatch=2):
    """C[bt] = A[bt] @ B[bt] through pe_gemm with explicit strides; A and B are
    flat device buffers holding `nbatch` operands each."""
    lib = abi.bind()
    a_bs = (M - 1) * a_ms + (K - 1) * a_ks + 1
    b_bs = (N - 1) * b_ns + (K - 1) * b_ks + 1
    d = launch.GemmDesc(dtype=dtype_code, batch_shape=[nbatch], a_bstride=[a_bs], b_bstride=[b_bs],
                        c_bstride=[M * N], M=M, N=N, K=K, a_ms=a_ms, a_ks=a_ks, b_ks=b_ks, b_ns=b_ns,
                        c_ms=N, c_ns=1, a_numel=a.numel(), b_numel=b.numel(), c_numel=nbatch * M * N,
                        split_k=split_k, tile=tile)
    cd = abi.gemm_desc(d)
    ws_bytes = lib.pe_gemm_workspace_bytes(ctypes.byref(cd))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    c = torch.empty(nbatch * M * N, dtype=torch.float32, device="cuda")
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), ctypes.c_void_p(c.data_ptr()), _ptr(ws),
                     ws_bytes, _stream())
    assert rc == 0, runtime.last_error()
    return c.cpu().reshape(nbatch, M, N)


@pytest.mark.parametrize("tile,dtype", [(64, torch.float32), (128, torch.float32), (192, torch.float32),
                                        (256, torch.float32), (64, torch.float16), (128, torch.float16),
                                        (256, torch.float16)])
@pytest.mark.parametrize("M,N,K", [(300, 200, 77), (200, 300, 77), (390, 390, 33),
                                   (264, 136, 40), (136, 264, 40)])
@pytest.mark.parametrize("layout", ["mn", "k"])
@pytest.mark.parametrize("split_k", [0, 3])
def test_gemm_tiles_direct(tile, dtype, M, N, K, layout, split_k):
    """Every tile shape in both orientations (M >= N picks the tall variant),
    both vector loaders (rows contiguous / k contiguous), partial tiles in M,
    N and K, with and without split-K, against a float64 reference."""
    nbatch = 2
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(nbatch, M, K, generator=g).to(dtype)
    B = torch.randn(nbatch, K, N, generator=g).to(dtype)
    if layout == "mn":    # A stored [K][M] (m contiguous), B stored [K][N] (n contiguous)
        a_buf, a_ms, a_ks = A.transpose(1, 2).contiguous(), 1, M
        b_buf, b_ks, b_ns = B.contiguous(), N, 1
    else:                 # A stored [M][K], B stored [N][K] (k contiguous)
        a_buf, a_ms, a_ks = A.contiguous(), K, 1
        b_buf, b_ks, b_ns = B.transpose(1, 2).contiguous(), 1, K
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    got = _gemm_direct(a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda(), M, N, K, a_ms, a_ks, b_ks, b_ns,
                       code, tile=tile, split_k=split_k, nbatch=nbatch)
    want = torch.bmm(A.double(), B.double()).numpy()
    scale = float(np.abs(want).max())
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    assert float(np.abs(got.numpy() - want).max()) <= rtol * scale


def _gemm_out_strides(A, B, a, b, a_ms, a_ks, b_ks, b_ns, dtype_code, tile, out, split_k=0):
    """pe_gemm with the output stored column-major ("cols": c_ms = 1, c_ns =
    M) or row-major with a row pitch past N ("pitch": c_ms = N + 5, whose
    rows are not whole 16-byte vectors); returns the product as [b][M][N]
    and the elements between the rows, which must stay untouched (NaN)."""
    nb, M, K = A.shape
    N = B.shape[2]
    c_ms, c_ns, c_bs = (1, M, M * N) if out == "cols" else (N + 5, 1, M * (N + 5))
    c_numel = nb * c_bs
    d = launch.GemmDesc(dtype=dtype_code, batch_shape=[nb], a_bstride=[a.numel() // nb],
                        b_bstride=[b.numel() // nb], c_bstride=[c_bs], M=M, N=N, K=K, a_ms=a_ms, a_ks=a_ks,
                        b_ks=b_ks, b_ns=b_ns, c_ms=c_ms, c_ns=c_ns, a_numel=a.numel(), b_numel=b.numel(),
                        c_numel=c_numel, split_k=split_k, tile=tile)
    lib = abi.bind()
    cd = abi.gemm_desc(d)
    ws_bytes = lib.pe_gemm_workspace_bytes(ctypes.byref(cd))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    c = torch.full((c_numel,), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), _ptr(c), _ptr(ws), ws_bytes, _stream())
    assert rc == 0, runtime.last_error()
    got = torch.as_strided(c, (nb, M, N), (c_bs, c_ms, c_ns)).cpu()
    gaps = None if out == "cols" else torch.as_strided(c, (nb, M, 5), (c_bs, c_ms, 1), N).cpu()
    return got, gaps


@pytest.mark.parametrize("out", ["cols", "pitch"])
@pytest.mark.parametrize("tile,dtype", [(64, torch.float32), (128, torch.float32), (256, torch.float32),
                                        (128, torch.float16), (256, torch.float16)])
@pytest.mark.parametrize("split_k", [0, 3])
def test_gemm_tiles_output_strides(tile, dtype, split_k, out):
    """Tile shapes with the output column-major or with a row pitch that is
    not a whole number of 16-byte vectors (gaps between rows untouched),
    partial tiles in M and N, with and without split-K."""
    nbatch, M, N, K = 2, 304, 200, 80
    g = torch.Generator().manual_seed(tile + split_k + len(out))
    A = torch.randn(nbatch, M, K, generator=g).to(dtype)
    B = torch.randn(nbatch, K, N, generator=g).to(dtype)
    a_buf, b_buf = A.contiguous(), B.transpose(1, 2).contiguous()
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    got, gaps = _gemm_out_strides(A, B, a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda(), K, 1, 1, K, code,
                                  tile, out, split_k=split_k)
    want = torch.bmm(A.double(), B.double())
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    assert float((got.double() - want).abs().max()) <= rtol * float(want.abs().max())
    if gaps is not None:
        assert bool(torch.isnan(gaps).all())


@pytest.mark.parametrize("c_ms", [2_000_003, 2_200_001], ids=["dl-near-limit", "staged-beyond-limit"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_gemm_large_output_row_stride(c_ms, dtype):
    """Output rows ~8 MB apart: just under the direct-load kernel's limit
    (every element of a 256 x 256 tile within 2^31 bytes of its corner, so
    in-tile store offsets reach ~500 MB) and just over it (the staged kernel
    takes the call), with partial tiles in M and N."""
    M, N, K = 130, 70, 40
    g = torch.Generator().manual_seed(c_ms % 1000)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(K, N, generator=g).to(dtype)
    lib = abi.bind()
    c_numel = (M - 1) * c_ms + N
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[1], a_bstride=[M * K], b_bstride=[K * N], c_bstride=[c_numel],
                        M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=N, b_ns=1, c_ms=c_ms, c_ns=1, a_numel=M * K,
                        b_numel=K * N, c_numel=c_numel)
    cd = abi.gemm_desc(d)
    ws_bytes = lib.pe_gemm_workspace_bytes(ctypes.byref(cd))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    c = torch.full((c_numel,), float("nan"), dtype=torch.float32, device="cuda")
    a, b = A.contiguous().cuda(), B.contiguous().cuda()
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), ctypes.c_void_p(c.data_ptr()), _ptr(ws), ws_bytes,
                     _stream())
    assert rc == 0, runtime.last_error()
    got = torch.as_strided(c, (M, N), (c_ms, 1)).cpu().double()
    gaps = torch.as_strided(c, (M - 1, 16), (c_ms, 1), N).cpu()
    want = A.double() @ B.double()
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    assert float((got - want).abs().max()) <= rtol * float(want.abs().max())
    assert bool(torch.isnan(gaps).all())  # nothing stored between the rows


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 128), (1024, 8192, 1024), (1000, 6000, 300)])
def test_long_k_split_grids(dtype, M, K, N):
    """Long-K products that the tile choice runs as 128x128 tiles split over
    K at about two blocks per CU (partial tiles and a K tail in the last
    case), through the public einsum against a float64 GPU reference."""
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(M + K + N)
    a = (torch.randn(M, K, generator=g) * 0.1).to(dtype).cuda()
    b = (torch.randn(K, N, generator=g) * 0.1).to(dtype).cuda()
    got = einsum("ij,jk->ik", a, b).double()
    want = a.double() @ b.double()
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    assert float((got - want).abs().max()) <= rtol * float(want.abs().max())
    assert torch.equal(einsum("ij,jk->ik", a, b), einsum("ij,jk->ik", a, b))  # deterministic split order


def test_gemm_rejects_bad_tile():
    lib = abi.bind()
    d = launch.GemmDesc(dtype=launch.DT_F16, batch_shape=[1], a_bstride=[0], b_bstride=[0], c_bstride=[0],
                        M=4, N=4, K=4, a_ms=4, a_ks=1, b_ks=4, b_ns=1, c_ms=4, c_ns=1, a_numel=16,
                        b_numel=16, c_numel=16, tile=192)
    x = torch.zeros(16, device="cuda")
    rc = lib.pe_gemm(ctypes.byref(abi.gemm_desc(d)), _ptr(x), _ptr(x), _ptr(x), None, 0, _stream())
    assert rc == -3 and "192" in runtime.last_error()
    d.tile, d.dtype = 96, launch.DT_F32
    rc = lib.pe_gemm(ctypes.byref(abi.gemm_desc(d)), _ptr(x), _ptr(x), _ptr(x), None, 0, _stream())
    assert rc == -1 and "tile" in runtime.last_error()


@pytest.mark.parametrize("layout_a,layout_b", [("mn", "mn"), ("k", "k"), ("mn", "k"), ("k", "mn")])
@pytest.mark.parametrize("dtype,nbatch,M,N,K", [(torch.float32, 96, 512, 512, 40), (torch.float32, 64, 512, 512, 36),
                                                (torch.float32, 48, 520, 264, 100),
                                                (torch.float16, 96, 512, 512, 40), (torch.float16, 64, 512, 512, 72),
                                                (torch.float16, 48, 520, 264, 104), (torch.float16, 2, 1024, 1024, 512)],
                         ids=["f32-768t-k40", "f32-512t-k36", "f32-partial", "f16-768t-k40", "f16-512t-k72",
                              "f16-partial", "f16-compute"])
def test_gemm_grids_of_wide_tiles(layout_a, layout_b, dtype, nbatch, M, N, K):
    """Grids large enough for the tile choice to consider the 256-wide tiles
    at both register budgets (768 tiles fill one round at three blocks per
    CU, 512 one round at two), with every operand layout pairing (float16
    k-major operands go through the transposing LDS read), K tails inside the
    last slab, partial tiles in M and N, and (last case) a compute-bound
    float16 grid that runs persistent."""
    g = torch.Generator().manual_seed(nbatch + M + K)
    A = torch.randn(nbatch, M, K, generator=g).to(dtype)
    B = torch.randn(nbatch, K, N, generator=g).to(dtype)
    if layout_a == "mn":
        a_buf, a_ms, a_ks = A.transpose(1, 2).contiguous(), 1, M
    else:
        a_buf, a_ms, a_ks = A.contiguous(), K, 1
    if layout_b == "mn":
        b_buf, b_ks, b_ns = B.contiguous(), N, 1
    else:
        b_buf, b_ks, b_ns = B.transpose(1, 2).contiguous(), 1, K
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    got = _gemm_direct(a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda(), M, N, K, a_ms, a_ks, b_ks, b_ns,
                       code, nbatch=nbatch)
    want = torch.bmm(A.double().cuda(), B.double().cuda()).cpu()
    scale = float(want.abs().max())
    rtol = 1e-4 if dtype == torch.float32 else 2e-3
    assert float((got.double() - want).abs().max()) <= rtol * scale


def test_mfma_probe_runs_and_validates():
    """The attainable-peak probe: finite per-lane sums, positive flops, and
    the argument checks of its C entry point."""
    import ctypes

    from pto_einsum import abi, runtime

    lib = abi.bind()
    n = int(lib.pe_probe_out_len())
    out = torch.full((n,), float("nan"), device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for dt in (0, 1):
        for rnd in (0, 1):
            rc = lib.pe_probe_mfma(dt, rnd, 3, ctypes.c_void_p(out.data_ptr()), n, st)
            assert rc == 0, runtime.last_error()
            torch.cuda.synchronize()
            assert bool(torch.isfinite(out).all())
        assert int(lib.pe_probe_mfma_flops(dt, 3)) > 0
    assert lib.pe_probe_mfma(7, 0, 3, ctypes.c_void_p(out.data_ptr()), n, st) == -3
    assert lib.pe_probe_mfma(1, 0, 0, ctypes.c_void_p(out.data_ptr()), n, st) == -1
    assert lib.pe_probe_mfma(1, 0, 3, ctypes.c_void_p(out.data_ptr()), n - 1, st) == -2


@pytest.mark.parametrize("split_k", [7, 9, 13, 15])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_tile_walk_with_block_counts_not_a_multiple_of_eight(split_k, dtype):
    """36 tiles of 128x128 times an odd split count: grids of 252-540 blocks,
    which the XCD-aware walk deals to the 8 XCDs in unequal shares; every
    tile of every split is computed exactly once (the output starts as NaN)."""
    M = N = 768
    K = 4096 if dtype == torch.float32 else 8192
    g = torch.Generator().manual_seed(split_k)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(K, N, generator=g).to(dtype)
    lib = abi.bind()
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[1], a_bstride=[0], b_bstride=[0], c_bstride=[0],
                        M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=N, b_ns=1, c_ms=N, c_ns=1, a_numel=M * K,
                        b_numel=K * N, c_numel=M * N, tile=128, split_k=split_k)
    cd = abi.gemm_desc(d)
    ws_bytes = lib.pe_gemm_workspace_bytes(ctypes.byref(cd))
    assert ws_bytes == split_k * M * N * 4
    ws = torch.full((ws_bytes // 4,), float("nan"), device="cuda")
    c = torch.full((M, N), float("nan"), device="cuda")
    a, b = A.cuda(), B.cuda()
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), ctypes.c_void_p(c.data_ptr()), _ptr(ws), ws_bytes, _stream())
    assert rc == 0, runtime.last_error()
    got = c.cpu().double()
    want = A.double() @ B.double()
    bound = A.double().abs() @ B.double().abs()
    assert not torch.isnan(got).any()
    assert bool(((got - want).abs() <= 1e-5 * bound + 1e-6).all())


# pe_product stride patterns: operand A laid out as the output (its offset is
# the flat index) with B broadcast over outer axes in every position, and A
# transposed or broadcast itself (the general per-axis decode).
PRODUCT_STRIDES = [
    # out shape, a strides, b strides
    ((3, 40, 5, 64), (12800, 320, 64, 1), (0, 64, 0, 1)),        # bshd,sd->bshd: B's outermost axis broadcast
    ((3, 40, 5, 64), (12800, 320, 64, 1), (320, 0, 64, 1)),      # B broadcast over the second axis only
    ((3, 40, 5, 64), (12800, 320, 64, 1), (0, 0, 0, 1)),         # B a row, every outer axis broadcast
    ((3, 40, 5, 64), (12800, 320, 64, 1), (12800, 320, 64, 0)),  # B broadcast along the vector axis
    ((3, 40, 5, 64), (12800, 320, 64, 1), (0, 5, 1, 200)),       # B transposed: scalar path
    ((6, 40, 64), (64, 384, 1), (0, 64, 1)),                      # A with permuted outer axes
    ((6, 40, 64), (0, 64, 1), (2560, 64, 1)),                     # A broadcast, B laid out as the output
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("add_zero", [0, 1])
@pytest.mark.parametrize("shape,sa,sb", PRODUCT_STRIDES)
def test_product_stride_patterns_bit_exact(shape, sa, sb, add_zero, dtype):
    g = torch.Generator().manual_seed(len(shape) * 7 + sum(sb) + add_zero)
    na = 1 + sum((n - 1) * s for n, s in zip(shape, sa))
    nb = 1 + sum((n - 1) * s for n, s in zip(shape, sb))
    a = torch.randn(na, generator=g).to(dtype)
    b = torch.randn(nb, generator=g).to(dtype)
    a[::7] = -0.0
    nout = int(np.prod(shape))
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    d = abi.product_desc(launch.ProductDesc(code, add_zero, list(shape), list(sa), list(sb), na, nb))
    ga, gb = a.cuda(), b.cuda()
    out = torch.full((nout,), float("nan"), device="cuda")
    rc = abi.bind().pe_product(ctypes.byref(d), _ptr(ga), _ptr(gb), _ptr(out), _stream())
    assert rc == 0, runtime.last_error()
    av = torch.as_strided(a, shape, sa).float()
    bv = torch.as_strided(b, shape, sb).float()
    want = av * bv
    if add_zero:
        want = 0.0 + want
    got = out.cpu().view(shape)
    assert torch.equal(got.view(torch.int32), want.contiguous().view(torch.int32))


@pytest.mark.parametrize("shape,perm", [((16, 777, 1000), (0, 2, 1)),   # config 2 in0: 32-element float32 tiles
                                        ((3, 37, 45), (0, 2, 1)),       # partial tiles on both axes
                                        ((2, 5, 33, 7), (0, 3, 2, 1)),  # odd rows, batch axes
                                        ((65, 31), (1, 0)),
                                        ((64, 37, 400), (0, 2, 1)),     # q = 37: one 32 x 64 tile spans it
                                        ((5, 50, 70), (0, 2, 1))])
def test_float32_transposes_with_unaligned_destination_rows(shape, perm):
    """Destination rows that are not whole 16-byte vectors take the
    32-element float32 tile (32 x 64 where q is 33 to 64); bit-exact against torch.permute (NaN payloads
    included, the data being arbitrary 32-bit patterns)."""
    n = int(np.prod(shape))
    src = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device="cuda")
    dst = torch.zeros(n, dtype=torch.int32, device="cuda")
    from pto_einsum.planner import transpose_config
    cfg = transpose_config("p", shape, perm)
    d = abi.permute_desc(launch.PermuteDesc(4, list(cfg["to_shape"]), list(cfg["perm_strides"]), n))
    rc = abi.bind().pe_permute(ctypes.byref(d), _ptr(src), _ptr(dst), _stream())
    assert rc == 0, runtime.last_error()
    assert torch.equal(dst.cpu(), src.cpu().view(shape).permute(perm).contiguous().view(-1))
