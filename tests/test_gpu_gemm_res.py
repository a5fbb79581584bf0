"""The short-K GEMM kernel (every k slab of a tile resident in LDS, all
loads issued up front: float16 with K in (96, 128] on 64x128 tiles, float32
with K in (112, 128] on 128x128 tiles; forced with pe_gemm_desc.tile = 2 at
sizes the automatic choice sends elsewhere): every operand layout pairing, K
tails inside the last slab, partial tiles in M and N and batches, against a
float64 reference, with run-to-run equality (the reference checks its
batched matmul the same way, test_einsum.py:244-364); config 5.1 and a
config-3-shaped product through the public einsum, which choose the float16
variant; and the tile that pe_gemm_choice reports for config 5.1."""
import ctypes

import pytest
import torch

from pto_einsum import abi, einsum, launch, runtime

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _check(got, A, B, rtol=2e-3):
    want = torch.bmm(A.double(), B.double())
    bound = torch.bmm(A.double().abs(), B.double().abs())
    assert bool(((got.cpu().double() - want).abs() <= 1e-5 * bound + 1e-6).all())


def test_refused_outside_its_range():
    lib = abi.bind()
    d = launch.GemmDesc(dtype=launch.DT_F16, batch_shape=[1], a_bstride=[0], b_bstride=[0], c_bstride=[0],
                        M=128, N=128, K=64, a_ms=64, a_ks=1, b_ks=128, b_ns=1, c_ms=128, c_ns=1,
                        a_numel=128 * 64, b_numel=64 * 128, c_numel=128 * 128, tile=2)
    assert lib.pe_gemm(ctypes.byref(abi.gemm_desc(d)), None, None, None, None, 0, None) == -3
    d.dtype, d.K = launch.DT_F32, 112
    assert lib.pe_gemm(ctypes.byref(abi.gemm_desc(d)), None, None, None, None, 0, None) == -3
    d.K = 160
    assert lib.pe_gemm(ctypes.byref(abi.gemm_desc(d)), None, None, None, None, 0, None) == -3


@pytest.mark.parametrize("al,bl", [("mn", "mn"), ("mn", "k"), ("k", "mn"), ("k", "k")])
@pytest.mark.parametrize("dt,nb,M,N,K", [("f16", 3, 128, 128, 128), ("f16", 2, 200, 136, 120),
                                         ("f16", 5, 136, 264, 104), ("f16", 1, 1000, 384, 128),
                                         ("f16", 4, 136, 72, 112), ("f32", 3, 128, 128, 128),
                                         ("f32", 2, 200, 136, 124), ("f32", 5, 136, 264, 116),
                                         ("f32", 1, 1000, 384, 128), ("f32", 4, 132, 68, 120)])
def test_short_k_kernel_against_float64(al, bl, dt, nb, M, N, K):
    g = torch.Generator().manual_seed(nb * 1000 + M + N + K)
    tdt = torch.float16 if dt == "f16" else torch.float32
    A = (torch.randn(nb, M, K, generator=g) / 8).to(tdt)
    B = (torch.randn(nb, K, N, generator=g) / 8).to(tdt)
    a_buf, a_ms, a_ks = (A.transpose(1, 2).contiguous(), 1, M) if al == "mn" else (A.contiguous(), K, 1)
    b_buf, b_ks, b_ns = (B.contiguous(), N, 1) if bl == "mn" else (B.transpose(1, 2).contiguous(), 1, K)
    d = launch.GemmDesc(dtype=launch.DT_F16 if dt == "f16" else launch.DT_F32, batch_shape=[nb],
                        a_bstride=[M * K], b_bstride=[K * N],
                        c_bstride=[M * N], M=M, N=N, K=K, a_ms=a_ms, a_ks=a_ks, b_ks=b_ks, b_ns=b_ns,
                        c_ms=N, c_ns=1, a_numel=nb * M * K, b_numel=nb * K * N, c_numel=nb * M * N, tile=2)
    lib = abi.bind()
    cd = abi.gemm_desc(d)
    assert lib.pe_gemm_workspace_bytes(ctypes.byref(cd)) == 0
    a, b = a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda()
    outs = []
    for _ in range(3):
        c = torch.full((nb, M, N), float("nan"), device="cuda")
        rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), _ptr(c), None, 0,
                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, runtime.last_error()
        outs.append(c)
    torch.cuda.synchronize()
    _check(outs[0], A, B)
    assert all(torch.equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("eq,s0,s1,dt", [("tn,sn->ts", (4096, 128), (4096, 128), "f16"),
                                         ("bshd,bthd->bsht", (2, 512, 8, 128), (2, 384, 8, 128), "f16")])
def test_public_einsum_shapes_that_take_it(eq, s0, s1, dt):
    """Config 5.1 itself and a config-3-shaped product (two batch axes, the
    fused permuted store) through einsum(), against a float64 reference."""
    g = torch.Generator().manual_seed(51)
    tdt = torch.float16 if dt == "f16" else torch.float32
    x = (torch.randn(s0, generator=g) / 8).to(tdt)
    y = (torch.randn(s1, generator=g) / 8).to(tdt)
    got = einsum(eq, x.cuda(), y.cuda()).cpu().double()
    want = torch.einsum(eq, x.double(), y.double())
    bound = torch.einsum(eq, x.double().abs(), y.double().abs())
    assert bool(((got - want).abs() <= 1e-5 * bound + 1e-6).all())


@pytest.mark.parametrize("out", ["cols", "pitch"])
@pytest.mark.parametrize("dt,al,bl,K", [("f16", "k", "mn", 120), ("f16", "mn", "k", 104),
                                        ("f32", "k", "k", 124), ("f32", "mn", "mn", 116)])
def test_short_k_output_strides(dt, al, bl, K, out):
    """The short-K kernel's stores away from contiguous rows: a column-major
    output, and rows with a pitch (N + 5) that is not a whole number of
    16-byte vectors, whose gaps stay untouched; partial tiles in M and N."""
    nb, M, N = 2, 200, 136
    g = torch.Generator().manual_seed(K * 3 + len(out))
    tdt = torch.float16 if dt == "f16" else torch.float32
    A = (torch.randn(nb, M, K, generator=g) / 8).to(tdt)
    B = (torch.randn(nb, K, N, generator=g) / 8).to(tdt)
    a_buf, a_ms, a_ks = (A.transpose(1, 2).contiguous(), 1, M) if al == "mn" else (A.contiguous(), K, 1)
    b_buf, b_ks, b_ns = (B.contiguous(), N, 1) if bl == "mn" else (B.transpose(1, 2).contiguous(), 1, K)
    c_ms, c_ns, c_bs = (1, M, M * N) if out == "cols" else (N + 5, 1, M * (N + 5))
    d = launch.GemmDesc(dtype=launch.DT_F16 if dt == "f16" else launch.DT_F32, batch_shape=[nb],
                        a_bstride=[M * K], b_bstride=[K * N], c_bstride=[c_bs], M=M, N=N, K=K, a_ms=a_ms,
                        a_ks=a_ks, b_ks=b_ks, b_ns=b_ns, c_ms=c_ms, c_ns=c_ns, a_numel=nb * M * K,
                        b_numel=nb * K * N, c_numel=nb * c_bs, tile=2)
    lib = abi.bind()
    cd = abi.gemm_desc(d)
    a, b = a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda()
    c = torch.full((nb * c_bs,), float("nan"), device="cuda")
    rc = lib.pe_gemm(ctypes.byref(cd), _ptr(a), _ptr(b), _ptr(c), None, 0,
                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, runtime.last_error()
    _check(torch.as_strided(c, (nb, M, N), (c_bs, c_ms, c_ns)), A, B)
    if out == "pitch":
        assert bool(torch.isnan(torch.as_strided(c, (nb, M, 5), (c_bs, c_ms, 1), N)).all())


def test_choice_reports_the_short_k_tile():
    """Config 5.1's product (4096^2 x 128 float16, both operands k
    contiguous) takes the short-K kernel by itself, and pe_gemm_choice says
    so with its 64x128 tile."""
    M = N = 4096
    K = 128
    d = launch.GemmDesc(dtype=launch.DT_F16, batch_shape=[1], a_bstride=[M * K], b_bstride=[K * N],
                        c_bstride=[M * N], M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=1, b_ns=K, c_ms=N, c_ns=1,
                        a_numel=M * K, b_numel=K * N, c_numel=M * N)
    info = (ctypes.c_int64 * 4)()
    assert abi.bind().pe_gemm_choice(ctypes.byref(abi.gemm_desc(d)), info) == 0
    assert list(info) == [64, 128, 1, 128]
