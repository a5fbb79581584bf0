"""The 256x256-tile float16 GEMM (pe_gemm_big.h) against float64 references:
every operand layout pairing, partial tiles in M and N, K tails inside the
last slab, batched operands, grids with more tiles than CUs (each block
walks several tiles, and the LDS ring carries the next tile's first slabs),
run-to-run equality, and the automatic choice on compute-bound einsums."""
import pytest
import torch

from pto_einsum import einsum, launch
from test_gpu_components import _gemm_direct, _gemm_out_strides

pytestmark = pytest.mark.gpu

RTOL = 2e-3


def _operands(nbatch, M, N, K, layout_a, layout_b, seed):
    g = torch.Generator().manual_seed(seed)
    A = (torch.randn(nbatch, M, K, generator=g) * 0.5).half()
    B = (torch.randn(nbatch, K, N, generator=g) * 0.5).half()
    if layout_a == "mn":    # A stored [K][M]
        a_buf, a_ms, a_ks = A.transpose(1, 2).contiguous(), 1, M
    else:                   # A stored [M][K]
        a_buf, a_ms, a_ks = A.contiguous(), K, 1
    if layout_b == "mn":    # B stored [K][N]
        b_buf, b_ks, b_ns = B.contiguous(), N, 1
    else:                   # B stored [N][K]
        b_buf, b_ks, b_ns = B.transpose(1, 2).contiguous(), 1, K
    return A, B, a_buf.reshape(-1).cuda(), b_buf.reshape(-1).cuda(), a_ms, a_ks, b_ks, b_ns


LAYOUTS = [("k", "mn"), ("k", "k"), ("mn", "mn"), ("mn", "k")]
SHAPES = [(1, 512, 512, 64), (2, 520, 264, 104), (3, 256, 768, 1000), (1, 2048, 2048, 96),
          (9, 1280, 2048, 40), (1, 264, 256, 24), (9, 1280, 2048, 64), (4, 2560, 2048, 256)]


@pytest.mark.parametrize("layout_a,layout_b", LAYOUTS, ids=lambda v: v)
@pytest.mark.parametrize("nbatch,M,N,K", SHAPES, ids=lambda v: str(v))
def test_big_tile_direct(layout_a, layout_b, nbatch, M, N, K):
    print(f"big f16: {layout_a}/{layout_b} b={nbatch} {M}x{N}x{K}", flush=True)
    A, B, a, b, a_ms, a_ks, b_ks, b_ns = _operands(nbatch, M, N, K, layout_a, layout_b, nbatch * 7 + M + N + K)
    got = _gemm_direct(a, b, M, N, K, a_ms, a_ks, b_ks, b_ns, launch.DT_F16, tile=1, nbatch=nbatch)
    want = torch.bmm(A.double().cuda(), B.double().cuda()).cpu()
    scale = float(want.abs().max())
    assert float((got.double() - want).abs().max()) <= RTOL * scale
    again = _gemm_direct(a, b, M, N, K, a_ms, a_ks, b_ks, b_ns, launch.DT_F16, tile=1, nbatch=nbatch)
    assert torch.equal(got, again)


def test_big_tile_rows_contiguous_any_k():
    """Both operands with rows contiguous take any K (no 16-byte k vectors):
    a K tail that is not a multiple of 8."""
    A, B, a, b, a_ms, a_ks, b_ks, b_ns = _operands(2, 264, 520, 77, "mn", "mn", 5)
    got = _gemm_direct(a, b, 264, 520, 77, a_ms, a_ks, b_ks, b_ns, launch.DT_F16, tile=1, nbatch=2)
    want = torch.bmm(A.double().cuda(), B.double().cuda()).cpu()
    assert float((got.double() - want).abs().max()) <= RTOL * float(want.abs().max())


@pytest.mark.parametrize("eq", ["ij,jk->ik", "ik,jk->ij", "bij,bjk->bik"])
def test_big_tile_auto_choice(eq):
    """Compute-bound float16 einsums with at least one round of 256x256 tiles
    take the kernel by themselves (4096^3: 256 tiles; batched: 8 x 2048^2)."""
    g = torch.Generator().manual_seed(11)
    if eq.startswith("b"):
        x = (torch.randn(8, 2048, 1024, generator=g) * 0.5).half().cuda()
        y = (torch.randn(8, 1024, 2048, generator=g) * 0.5).half().cuda()
    else:
        x = (torch.randn(4096, 4096, generator=g) * 0.5).half().cuda()
        y = (torch.randn(4096, 4096, generator=g) * 0.5).half().cuda()
    print(f"big f16 auto: {eq} {tuple(x.shape)} x {tuple(y.shape)}", flush=True)
    got = einsum(eq, x, y)
    want = torch.einsum(eq, x.double(), y.double())
    assert float((got.double() - want).abs().max()) <= RTOL * float(want.abs().max())
    assert torch.equal(got, einsum(eq, x, y))


def test_big_tile_auto_choice_below_one_round():
    """A compute-bound float16 GEMM with 256x256 tiles for fewer CUs than the
    device has (3072 x 2048 x 3072: 144 tiles) takes the kernel too, one
    block per tile."""
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(3072, 2048, generator=g) * 0.5).half().cuda()
    y = (torch.randn(2048, 3072, generator=g) * 0.5).half().cuda()
    print("big f16 auto: ij,jk->ik (3072, 2048) x (2048, 3072)", flush=True)
    got = einsum("ij,jk->ik", x, y)
    want = torch.einsum("ij,jk->ik", x.double(), y.double())
    assert float((got.double() - want).abs().max()) <= RTOL * float(want.abs().max())
    assert torch.equal(got, einsum("ij,jk->ik", x, y))


@pytest.mark.parametrize("out", ["cols", "pitch"])
@pytest.mark.parametrize("layout_a,layout_b,K", [("k", "k", 64), ("k", "mn", 104), ("mn", "mn", 96),
                                                 ("mn", "k", 64)], ids=lambda v: str(v))
def test_big_tile_output_strides(layout_a, layout_b, K, out):
    """The 256x256 kernel's output addressing away from contiguous rows: a
    column-major output and rows with a pitch that is not a whole number of
    16-byte vectors, with partial tiles in M and N, on both of its schedules
    (k-contiguous A with an even slab count: 16x16x32 blocks; otherwise
    32x32x16)."""
    nbatch, M, N = 2, 520, 264
    print(f"big f16 out={out}: {layout_a}/{layout_b} b={nbatch} {M}x{N}x{K}", flush=True)
    A, B, a, b, a_ms, a_ks, b_ks, b_ns = _operands(nbatch, M, N, K, layout_a, layout_b, 31 + K)
    got, gaps = _gemm_out_strides(A, B, a, b, a_ms, a_ks, b_ks, b_ns, launch.DT_F16, 1, out)
    want = torch.bmm(A.double(), B.double())
    assert float((got.double() - want).abs().max()) <= RTOL * float(want.abs().max())
    if gaps is not None:
        assert bool(torch.isnan(gaps).all())
