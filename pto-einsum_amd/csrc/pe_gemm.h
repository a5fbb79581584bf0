// Batched strided GEMM on CDNA4 matrix cores (gfx950).
//
// Reference counterparts: batched_matmul_inline and its tile schedules
// (pto_einsum_matmul.h:115-970) plus the operand transposes of Phase A
// (pto_einsum_transpose.h) and the fused permuted store
// (pto_einsum_matmul.h:614-639).  Here one kernel reads both operands at
// their own strides (any of the reference's NT / NN-strided / TN direct-read
// modes and the identity case, plus the transposed reads the reference
// gathers first) and stores each tile straight into the permuted output.
//
//   C[b, m, n] = sum_k A[b, m, k] * B[b, k, n]      (float32 accumulation)
//
// Tiling: a 256-thread block (four 64-wide waves, 2x2) owns a BM x BN output
// tile and walks K in BK slabs through double-buffered LDS.  Each wave owns
// (BM/2) x (BN/2) as 32x32 MFMA blocks:
//   float32: v_mfma_f32_32x32x2_f32  (2 k per instruction)
//   float16: v_mfma_f32_32x32x16_f16 (16 k per instruction, gfx950)
// Operand layouts in LDS are chosen so each lane's MFMA fragment is one LDS
// read: float32 keeps [BK][BM] (lanes read 32 consecutive m), float16 keeps
// [BM][BK] (each lane reads 8 consecutive k as one 16-byte read).
//
// Boundaries: rows m >= M and columns n >= N of a partial tile load clamped
// (in-bounds, arbitrary) data -- they only feed outputs that are never
// stored.  The K tail is zero-filled in both operands, so no garbage value
// (not even inf/NaN) reaches a stored sum.  Every batch count and every
// M/N/K works, including the batched partial tiles the reference rejects
// (builder.py:593-604).
//
// Thin grids use a deterministic split-K: each split writes its partial tile
// to a workspace slab and a second kernel sums the slabs in split order.
#pragma once

#include "pe_common.h"

// GEMMs whose operands qualify take the direct-load kernel (float16 ones
// only with PE_GEMM_DL_F16).
#ifndef PE_GEMM_DL
#define PE_GEMM_DL 1
#endif
#ifndef PE_GEMM_DL_F16
#define PE_GEMM_DL_F16 1
#endif

namespace pe {

// Operand layout classes (chosen on the host from the strides).
enum Layout : int {
    L_GENERIC = 0,  // element-wise loads at arbitrary strides
    L_MN = 1,       // m (A) / n (B) contiguous, 16-byte vectors along it
    L_K = 2         // k contiguous, 16-byte vectors along k
};

struct GemmArgs {
    const void* a;
    const void* b;
    float* c;
    float* partial;           // split-K workspace, [split][batch][M][N]
    int32_t M, N, K;
    int32_t nsplit;
    int32_t k_per_split;      // multiple of BK
    int32_t tiles_m, tiles_n;
    uint32_t tiles_per_batch; // tiles_m * tiles_n
    uint32_t nbatch_total;
    uint32_t total_blocks;    // tiles_per_batch * nbatch_total * nsplit
    uint32_t grid;            // launched blocks (persistent when < total_blocks)
    int32_t store_nt;         // non-temporal stores for the output
    int32_t off32;            // direct-load kernel: full slabs load from 32-bit per-lane offsets
    int64_t a_ms, a_ks, b_ks, b_ns, c_ms, c_ns;
    int32_t nbatch;
    FastDiv batch_div[PE_MAX_DIMS];
    int64_t a_bs[PE_MAX_DIMS], b_bs[PE_MAX_DIMS], c_bs[PE_MAX_DIMS];
};

struct ReduceArgs {
    const float* partial;
    float* c;
    int32_t nsplit;
    uint32_t per_split;       // nbatch_total * M * N
    FastDiv n_div, m_div;     // flat -> (batch, m, n)
    int64_t c_ms, c_ns;
    int32_t nbatch;
    int32_t store_nt;
    FastDiv batch_div[PE_MAX_DIMS];
    int64_t c_bs[PE_MAX_DIMS];
};

// Deterministic split reduction: c = sum over the nsplit partial slabs in
// ascending order from +0 (nsplit = 0 writes +0 everywhere).  Enqueues the
// reduction kernel (pe_gemm.hip).
hipError_t launch_splitk_reduce(const ReduceArgs& r, hipStream_t s);

// Host-side launch entry for one (dtype, tile) family; defined per family
// in pe_gemm_f32.hip / pe_gemm_f16.hip.
// Slab depth (k per LDS stage) of each family, for the split-K granularity.
int gemm_bk(int dtype);
// (bm, bn) is one of 64x64, 128x128, 256x128, 128x256.  gemm_occupancy_*
// returns resident blocks per CU of that tile (runtime occupancy query).
int gemm_occupancy_f32(int bm, int bn);
int gemm_occupancy_f16(int bm, int bn);
// persist: 0 = one block per tile; > 0 = at most that many blocks per CU;
// < 0 = as many blocks per CU as the launched kernel keeps resident.
hipError_t launch_gemm_f32(int bm, int bn, int alayout, int blayout, int persist, const GemmArgs& g,
                           hipStream_t s);
// Direct-load kernel (pe_gemm_dl.h, float32 and float16): 64x64, 128x128,
// 256x128 and 128x256 tiles, L_MN or L_K operands with the vector and
// output-stride conditions gemm_dl_eligible checks.  minb: register budget
// of the 256-wide tiles (2 or 3 resident blocks per CU; 64x64 / 128x128
// always use 4).
// gemm_dl_resident returns the resident blocks per CU of one instantiation,
// or 0 when the compiler spilled more than a few of its registers (never
// launched).  persist: a grid of resident blocks walking the tiles (else one
// block per tile).
bool gemm_dl_eligible(int dtype, int al, int bl, int64_t M, int64_t N, int64_t K, int64_t c_ms, int64_t c_ns);
int gemm_dl_resident(int dtype, int bm, int bn, int minb, int al, int bl);
hipError_t launch_gemm_dl(int dtype, int bm, int bn, int minb, int al, int bl, bool persist, const GemmArgs& g,
                          hipStream_t s);
hipError_t launch_gemm_f16(int bm, int bn, int alayout, int blayout, int persist, const GemmArgs& g,
                           hipStream_t s);
// Short-K kernel (gemm_res_kernel in pe_gemm_dl.h): every k slab resident in
// LDS (float16: 64x128 tiles, four 32-k slabs, K in (96, 128]; float32:
// 128x128 tiles, eight 16-k slabs, K in (112, 128]), one block per tile,
// operands L_MN or L_K under the gemm_dl_eligible conditions, no split.
// gemm_res_resident: resident blocks per CU (0 when it spilled);
// gemm_res_tile_m / _n: its tile rows (of A) and columns (rows of B).
int gemm_res_resident(int dtype, int alayout, int blayout);
int gemm_res_tile_m(int dtype);
int gemm_res_tile_n(int dtype);
hipError_t launch_gemm_res(int dtype, int alayout, int blayout, const GemmArgs& g, hipStream_t s);
// k-split kernel (pe_gemm_ks.h): float32 32x32 or 64x64 tiles, float16 64x64
// tiles (`tile`), one block per tile and batch, the block's waves splitting
// K; L_MN or L_K operands under the gemm_dl_eligible conditions, no
// workspace.  gemm_ks_resident: resident blocks per CU (0 when it spilled or
// for other dtypes, layouts and tiles).
int gemm_ks_resident(int dtype, int alayout, int blayout, int tile);
hipError_t launch_gemm_ks(int dtype, int alayout, int blayout, int tile, const GemmArgs& g, hipStream_t s);
// Large float16 kernel (pe_gemm_big.h): 256x256 tiles, one block per CU,
// operands L_MN or L_K under the gemm_dl_eligible conditions, no K split.
// gemm_big_resident: resident blocks per CU (0 when it spilled).
int gemm_big_resident(int alayout, int blayout);
hipError_t launch_gemm_big(int alayout, int blayout, const GemmArgs& g, hipStream_t s);

}  // namespace pe
