"""The GEMM tile / split choice, read on the CPU through pe_gemm_choice (the
choice the workspace query sizes for; with no GPU the library assumes
MI355X's 256 CUs), and the workspace size that follows from it.  Pins the choices
the measured tuning made: the busiest-CU split counts of long-K grids, the
rebalancing of part-filled rounds, and the grids that must keep their choice
(the benchmark configurations)."""
import ctypes

import pytest

from pto_einsum import abi, launch


def _splits(M, N, K, dtype="f32", nb=1):
    code = launch.DT_F32 if dtype == "f32" else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[nb], a_bstride=[M * K], b_bstride=[K * N], c_bstride=[M * N],
                        M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=N, b_ns=1, c_ms=N, c_ns=1,
                        a_numel=nb * M * K, b_numel=nb * K * N, c_numel=nb * M * N)
    lib = abi.bind()
    info = (ctypes.c_int64 * 4)()
    assert lib.pe_gemm_choice(ctypes.byref(abi.gemm_desc(d)), info) == 0
    bm, bn, split, kps = list(info)
    ws = int(lib.pe_gemm_workspace_bytes(ctypes.byref(abi.gemm_desc(d))))
    if split == 1:
        assert ws == 0
        return 0
    assert ws == split * nb * M * N * 4     # the partials of every split
    assert split == -(-K // kps)
    return split


@pytest.mark.parametrize("shape,dtype,want", [
    ((4096, 128, 4096), "f32", 16),      # config 5.3: 32 tiles of 128x128, two blocks per CU
    ((768, 768, 4096), "f32", 14),       # 36 tiles: 504 blocks, 63 per XCD, two per CU
    ((1024, 1536, 4096), "f32", 8),      # 96 tiles: 768 blocks, three per CU
    ((2304, 2304, 6144), "f32", 7),      # 324 unsplit tiles left 1.27 per CU
    ((2816, 1664, 3072), "f16", 4),      # float16, 286 unsplit tiles
])
def test_split_counts_of_uneven_grids(shape, dtype, want):
    assert _splits(*shape, dtype=dtype) == want


@pytest.mark.parametrize("shape,dtype,nb", [
    ((1000, 1536, 777), "f32", 16),      # config 2: 1536 tiles of 128x128, four blocks per CU
    ((2048, 2048, 128), "f16", 128),     # config 3's per-head products
    ((4096, 4096, 128), "f16", 1),       # config 5.1
    ((128, 128, 128), "f32", 256),       # the GDN contraction set, 16 x 16
    ((8192, 8192, 8192), "f16", 1),      # the 256x256 float16 kernel
    ((4096, 4096, 4096), "f32", 1),
])
def test_full_grids_stay_unsplit(shape, dtype, nb):
    assert _splits(*shape, dtype=dtype, nb=nb) == 0


def _tile(M, N, K, dtype="f32", nb=1):
    code = launch.DT_F32 if dtype == "f32" else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[nb], a_bstride=[M * K], b_bstride=[K * N], c_bstride=[M * N],
                        M=M, N=N, K=K, a_ms=1, a_ks=M, b_ks=N, b_ns=1, c_ms=N, c_ns=1,
                        a_numel=nb * M * K, b_numel=nb * K * N, c_numel=nb * M * N)
    info = (ctypes.c_int64 * 4)()
    assert abi.bind().pe_gemm_choice(ctypes.byref(abi.gemm_desc(d)), info) == 0
    return info[0], info[1]


@pytest.mark.parametrize("shape,nb", [((1000, 1536, 777), 16), ((2048, 2048, 512), 8), ((4096, 4096, 4096), 1)])
def test_float32_direct_load_grids_keep_128_tiles(shape, nb):
    """MFMA-bound float32 grids with rows-contiguous operands (config 2's
    layout) stay on 128x128 tiles: at steady clocks they beat the 256-wide
    ones (config 2 278 against 292 us)."""
    assert _tile(*shape, nb=nb) == (128, 128)


@pytest.mark.parametrize("dtype,K,want", [("f16", 128, [64, 128, 1, 128]), ("f32", 120, [128, 128, 1, 120])])
def test_short_k_tile_reported(dtype, K, want):
    """pe_gemm_desc.tile = 2 (the short-K kernel) is reported with that
    kernel's tile: 64x128 for float16, 128x128 for float32, unsplit."""
    M = N = 1024
    code = launch.DT_F32 if dtype == "f32" else launch.DT_F16
    d = launch.GemmDesc(dtype=code, batch_shape=[1], a_bstride=[M * K], b_bstride=[K * N], c_bstride=[M * N],
                        M=M, N=N, K=K, a_ms=K, a_ks=1, b_ks=1, b_ns=K, c_ms=N, c_ns=1,
                        a_numel=M * K, b_numel=K * N, c_numel=M * N, tile=2)
    info = (ctypes.c_int64 * 4)()
    assert abi.bind().pe_gemm_choice(ctypes.byref(abi.gemm_desc(d)), info) == 0
    assert list(info) == want
