"""The k-split GEMM (pe_gemm_ks.h): float32 products with a K of at most
1024 whose tile choice splits K over blocks, or leaves at most two 64x64 tiles
per CU, and split ones with a K of at most 2048 whose 32x32 tiles give every
CU one, and float16 split grids whose 64x64 tiles give every CU (K <= 8192) or
a quarter of the CUs (K <= 2048) one, run as one block per 32x32 or 64x64
output tile, the block's four waves splitting K, with no workspace traffic.  Every operand
layout pairing (rows or k contiguous), batches, partial tiles, K tails that
end inside a stage's first, middle or last sub-slab, and transposed output
strides, against a float64 reference with a bound of 1e-5 sum |a||b| (float32
sums of at most 2048 terms); repeated calls are bit-identical."""
import ctypes

import pytest
import torch

from pto_einsum import abi, launch, runtime

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _run(M, N, K, nb, al, bl, ct, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(nb, M, K, generator=g).to(dtype)
    B = torch.randn(nb, K, N, generator=g).to(dtype)
    # A: "mn" stored [b][K][M] (m contiguous), "k" stored [b][M][K]
    if al == "mn":
        a_buf, a_ms, a_ks = A.transpose(1, 2).contiguous(), 1, M
    else:
        a_buf, a_ms, a_ks = A.contiguous(), K, 1
    # B: "mn" stored [b][K][N] (n contiguous), "k" stored [b][N][K]
    if bl == "mn":
        b_buf, b_ks, b_ns = B.contiguous(), N, 1
    else:
        b_buf, b_ks, b_ns = B.transpose(1, 2).contiguous(), 1, K
    c_ms, c_ns = (N, 1) if ct == "rows" else (1, M)
    code = launch.DT_F32 if dtype == torch.float32 else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[nb], a_bstride=[M * K], b_bstride=[K * N],
                        c_bstride=[M * N], M=M, N=N, K=K, a_ms=a_ms, a_ks=a_ks, b_ks=b_ks, b_ns=b_ns,
                        c_ms=c_ms, c_ns=c_ns, a_numel=nb * M * K, b_numel=nb * K * N, c_numel=nb * M * N)
    cd = abi.gemm_desc(d)
    lib = abi.bind()
    ws_bytes = int(lib.pe_gemm_workspace_bytes(ctypes.byref(cd)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    a, b = a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda()
    outs = []
    for _ in range(2):
        c = torch.full((nb * M * N,), float("nan"), device="cuda")
        rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), _ptr(c), _ptr(ws), ws_bytes, _stream())
        assert rc == 0, runtime.last_error()
        outs.append(torch.as_strided(c, (nb, M, N), (M * N, c_ms, c_ns)).cpu())
    want = torch.bmm(A.double(), B.double())
    bound = torch.bmm(A.double().abs(), B.double().abs())
    return outs, want, bound, ws_bytes


CASES = [
    # M, N, K, batch
    (256, 256, 256, 1),      # the 256^3 configuration
    (100, 68, 300, 2),       # partial tiles; K tail inside a stage's third sub-slab
    (36, 40, 132, 3),        # K tail in the first sub-slab of the last stage
    (512, 512, 1024, 1),     # the longest K this kernel takes
    (200, 96, 196, 1),       # K tail in the last sub-slab
    (8, 1000, 512, 2),       # one tile row
]


@pytest.mark.parametrize("al,bl", [("mn", "mn"), ("mn", "k"), ("k", "mn"), ("k", "k")])
@pytest.mark.parametrize("M,N,K,nb", CASES)
def test_k_split_gemm_against_float64(M, N, K, nb, al, bl):
    outs, want, bound, ws_bytes = _run(M, N, K, nb, al, bl, "rows", M * 31 + N * 7 + K + nb)
    assert ws_bytes > 0  # the tile choice splits this K: the k-split kernel takes the call
    err = (outs[0].double() - want).abs()
    assert not torch.isnan(outs[0]).any()
    assert bool((err <= 1e-5 * bound + 1e-6).all()), float((err - 1e-5 * bound).max())
    assert torch.equal(outs[0], outs[1])


ONE_PER_CU = [
    # M, N, K, batch: 64x64 tiles give each CU at most one (unsplit grids; 64x64 k-split tiles
    # where they give each CU three quarters of one or more)
    (1024, 1024, 512, 1),    # 256 tiles of 64x64
    (1000, 1000, 300, 1),    # partial tiles, K tail
    (960, 1024, 1000, 1),    # 240 tiles, K tail in the last stage's last sub-slab
    (512, 512, 768, 4),      # batched: 4 x 64 tiles
    (640, 640, 256, 1),      # 100 tiles: 32x32 k-split tiles
    (768, 768, 2048, 1),     # split grid with K = 2048 and 576 tiles of 32x32
    (512, 512, 1988, 2),     # the same with a K tail
]


@pytest.mark.parametrize("al,bl", [("mn", "mn"), ("mn", "k"), ("k", "mn"), ("k", "k")])
@pytest.mark.parametrize("M,N,K,nb", ONE_PER_CU)
def test_k_split_gemm_one_tile_per_cu(M, N, K, nb, al, bl):
    outs, want, bound, _ = _run(M, N, K, nb, al, bl, "rows", M + 3 * N + K + nb)
    err = (outs[0].double() - want).abs()
    assert not torch.isnan(outs[0]).any()
    assert bool((err <= 1e-5 * bound + 1e-6).all()), float((err - 1e-5 * bound).max())
    assert torch.equal(outs[0], outs[1])


F16_CASES = [
    # M, N, K, batch: float16 split grids whose 64x64 tiles give every CU one, or a quarter of the CUs one
    (1024, 1024, 1024, 1),
    (768, 768, 2048, 1),
    (512, 512, 1000, 2),     # K tail
    (200, 520, 776, 3),      # partial tiles, batched
    (1024, 1024, 8192, 1),   # the longest K this route takes
]


@pytest.mark.parametrize("al,bl", [("mn", "mn"), ("mn", "k"), ("k", "mn"), ("k", "k")])
@pytest.mark.parametrize("M,N,K,nb", F16_CASES)
def test_k_split_gemm_float16(M, N, K, nb, al, bl):
    outs, want, bound, ws_bytes = _run(M, N, K, nb, al, bl, "rows", 7 * M + N + K, torch.float16)
    assert ws_bytes > 0  # a split grid: the k-split kernel takes the call
    err = (outs[0].double() - want).abs()
    tol = 1e-5 if K <= 2048 else 4e-5   # float32 sums of K / 4 exact float16 products per wave
    assert not torch.isnan(outs[0]).any()
    assert bool((err <= tol * bound + 1e-6).all()), float((err - tol * bound).max())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("M,N,K,nb", [(100, 68, 300, 2), (256, 256, 256, 1), (1000, 1000, 300, 1)])
def test_k_split_gemm_transposed_output(M, N, K, nb):
    outs, want, bound, _ = _run(M, N, K, nb, "mn", "mn", "cols", 5 + M)
    err = (outs[0].double() - want).abs()
    assert bool((err <= 1e-5 * bound + 1e-6).all())
    assert torch.equal(outs[0], outs[1])


def test_k_split_gemm_with_unaligned_k_in_rows_layout():
    """k-major (rows contiguous) operands take any K: K = 130 leaves two k in
    the last stage's first sub-slab and three sub-slabs wholly past K."""
    outs, want, bound, ws_bytes = _run(64, 64, 130, 2, "mn", "mn", "rows", 11)
    assert ws_bytes > 0
    err = (outs[0].double() - want).abs()
    assert bool((err <= 1e-5 * bound + 1e-6).all())


def test_k_split_gemm_special_values():
    """inf and NaN propagate as in a plain float32 sum (the zero-filled K tail
    adds +0 * +0, never 0 * inf)."""
    M, N, K = 64, 64, 300
    A = torch.randn(M, K)
    B = torch.randn(K, N)
    A[3, 7] = float("inf")
    B[11, 5] = float("nan")
    lib = abi.bind()
    d = launch.GemmDesc(dtype=launch.DT_F32, batch_shape=[1], a_bstride=[0], b_bstride=[0], c_bstride=[0],
                        M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=N, b_ns=1, c_ms=N, c_ns=1, a_numel=M * K,
                        b_numel=K * N, c_numel=M * N)
    cd = abi.gemm_desc(d)
    ws_bytes = int(lib.pe_gemm_workspace_bytes(ctypes.byref(cd)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    a, b = A.cuda(), B.cuda()
    c = torch.empty(M, N, device="cuda")
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), _ptr(c), _ptr(ws), ws_bytes, _stream())
    assert rc == 0, runtime.last_error()
    got = c.cpu()
    want = A.double() @ B.double()
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    assert torch.allclose(got.double()[fin], want[fin], rtol=1e-4, atol=1e-3)


EINSUMS = [
    # equation, sizes (i, j = contracted, k, b); float32 GEMMs whose tile choice splits a K <= 1024
    ("ij,jk->ik", dict(i=256, j=256, k=256)),        # config 1
    ("ij,jk->ki", dict(i=200, j=300, k=120)),        # transposed output store
    ("ji,kj->ik", dict(i=96, j=1000, k=64)),         # both operands read transposed
    ("bij,bjk->bki", dict(b=3, i=64, j=500, k=96)),  # batched, permuted output
    ("ijx,jxk->ik", dict(i=128, j=16, x=40, k=128)), # two contracted axes merged into K = 640
]


@pytest.mark.parametrize("eq,sizes", EINSUMS, ids=[e for e, _ in EINSUMS])
def test_k_split_gemm_through_einsum(eq, sizes):
    """The k-split kernel behind the public einsum (layouts, batches and
    permuted stores chosen by the planner), against float64."""
    from pto_einsum import einsum

    t0, rest = eq.split(",")
    t1 = rest.split("->")[0]
    g = torch.Generator().manual_seed(len(eq) + sum(sizes.values()))
    a = torch.randn(*[sizes[c] for c in t0], generator=g)
    b = torch.randn(*[sizes[c] for c in t1], generator=g)
    got = einsum(eq, a.cuda(), b.cuda()).cpu()
    want = torch.einsum(eq, a.double(), b.double())
    bound = torch.einsum(eq, a.double().abs(), b.double().abs())
    assert got.shape == want.shape
    err = (got.double() - want).abs()
    assert bool((err <= 1e-5 * bound + 1e-6).all()), float((err - 1e-5 * bound).max())
    assert torch.equal(got, einsum(eq, a.cuda(), b.cuda()).cpu())
