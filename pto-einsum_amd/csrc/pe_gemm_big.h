// Large float16 GEMM (gfx950): 256 x 256 block tiles, one block per CU.
//
// Same contract, operand layouts (L_MN / L_K, 16-byte vectors) and output
// addressing as gemm_dl_kernel (pe_gemm_dl.h); this variant is for float16
// GEMMs that are bound by matrix-core issue, where the 128 x 256 tiles of
// that kernel at two blocks per CU ask more of the LDS than it delivers:
//
//  * four waves (2 x 2), each owning a 128 x 128 wave tile as 4 x 4 blocks
//    of v_mfma_f32_32x32x16_f16: per 16 k a wave issues 16 MFMAs against 8
//    fragment reads (4 for A, 4 for B), so LDS traffic per MFMA is a third
//    below the 64 x 128 wave tile's; with a k-contiguous A (and an even
//    number of slabs per tile) the wave tile runs as 8 x 8 blocks of
//    v_mfma_f32_16x16x32_f16 instead (same LDS bytes per MFMA flop; the
//    smaller MFMA keeps a higher clock at this data's power);
//  * K walks in 32-deep slabs (64 bytes of each row) through a ring of four
//    LDS stages (32 KB each), filled by global_load_lds_dwordx4 (no register
//    staging); the loads of slab s + 3 are issued while slab s is
//    multiplied, and each wave waits only for the slab it needs next
//    (s_waitcnt vmcnt with the later slab's loads still in flight);
//  * one barrier per slab, placed so that the next slab's first fragments
//    are read before the current slab's last MFMAs issue;
//  * tiles are walked in groups of four tile rows, so the 32 blocks of one
//    XCD (consecutive tiles of the XCD-aware walk) cover 4 x 8 tiles and
//    their L2 holds the shared A rows and B columns.
//
// LDS layouts of one stage (the fragment reads of each measured free of
// bank conflicts with the SQ_LDS_BANK_CONFLICT counter):
//   L_K : [256 rows][32 k], 64-byte rows of four 16-byte groups; logical
//         group g of row r sits in slot g ^ ((r / 4) % 4) (g ^ ((r / 2) % 4)
//         for the 16x16x32 schedule);
//   L_MN: [32 k][256 rows], 512-byte k rows of 32 groups; logical group g of
//         k row k sits in slot g ^ (4 (k % 4)) (also ^ 2 ((k / 8) % 2) for
//         the 16x16x32 schedule).
// A lane's direct load fetches the global vector that its slot holds.
//
// Boundaries as in gemm_dl_kernel: rows past M / N load clamped in-bounds
// vectors that only reach unstored outputs; the K tail of a tile's last slab
// is zeroed in LDS before any MFMA reads it.
#pragma once

#include "pe_gemm_dl.h"

namespace pe {

constexpr int kBigStages = 4;        // LDS ring: four 32 KB stages
constexpr int kBigTile = 256;
constexpr int kBigBK = 32;           // k per slab
constexpr int kBigGroupRows = 4;     // tile rows per walk group

// Output stores of a 128 x 128 wave tile straight from the accumulation
// registers (global_store_dword takes AGPR data on gfx950), addressed as in
// dl_store_tile: a wave-uniform 64-bit base in scalar registers, a 32-bit
// byte offset per lane and one of four uniform row offsets added in the
// same assembly block.
template <int NTM, bool MASKED, int FM, int FN>
__device__ __forceinline__ void big_store_tile(const float* wbase, uint32_t lane_off, uint32_t cms4, uint32_t cns4,
                                               int rrem, int crem, const f32x16 (&acc)[FM][FN]) {
    uint32_t rs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rs[r] = uint32_t(r) * cms4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            if (MASKED && 32 * j >= crem) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t bq = lane_off + uint32_t(32 * i + 8 * q) * cms4 + uint32_t(32 * j) * cns4;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (MASKED && 32 * i + 8 * q + r >= rrem) continue;
                    uint32_t t;
                    if constexpr (NTM == 2)
                        asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4 nt sc0 sc1"
                                     : "=&v"(t)
                                     : "s"(rs[r]), "v"(bq), "a"(acc[i][j][4 * q + r]), "s"(wbase));
                    else if constexpr (NTM == 1)
                        asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4 nt"
                                     : "=&v"(t)
                                     : "s"(rs[r]), "v"(bq), "a"(acc[i][j][4 * q + r]), "s"(wbase));
                    else
                        asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4"
                                     : "=&v"(t)
                                     : "s"(rs[r]), "v"(bq), "a"(acc[i][j][4 * q + r]), "s"(wbase));
                }
            }
        }
}

// Output stores of a 128 x 128 wave tile of 16 x 16 accumulator blocks
// (v_mfma_f32_16x16x32_f16: lane l, register r of block (i, j) holds row
// 16 i + 4 (l / 16) + r, column 16 j + l % 16), addressed as big_store_tile.
template <int NTM, bool MASKED>
__device__ __forceinline__ void big_store_tile16(const float* wbase, uint32_t lane_off, uint32_t cms4, uint32_t cns4,
                                                 int rrem, int crem, const f32x4 (&acc)[8][8]) {
    uint32_t rs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rs[r] = uint32_t(r) * cms4;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (MASKED && 16 * j >= crem) continue;
            const uint32_t bq = lane_off + uint32_t(16 * i) * cms4 + uint32_t(16 * j) * cns4;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (MASKED && 16 * i + r >= rrem) continue;
                uint32_t t;
                if constexpr (NTM == 2)
                    asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4 nt sc0 sc1"
                                 : "=&v"(t)
                                 : "s"(rs[r]), "v"(bq), "a"(acc[i][j][r]), "s"(wbase));
                else if constexpr (NTM == 1)
                    asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4 nt"
                                 : "=&v"(t)
                                 : "s"(rs[r]), "v"(bq), "a"(acc[i][j][r]), "s"(wbase));
                else
                    asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4"
                                 : "=&v"(t)
                                 : "s"(rs[r]), "v"(bq), "a"(acc[i][j][r]), "s"(wbase));
            }
        }
}

// M16: the L_K swizzle of the 16x16x32 schedule (see swz_k).
template <int LAYOUT, bool M16 = false>
struct BigOperand {
    static constexpr int ROWS = kBigTile;
    static constexpr int BK = kBigBK;
    static constexpr int STAGE_BYTES = ROWS * BK * 2;            // 16 KB
    static constexpr int NI = STAGE_BYTES / 1024 / 4;            // 1 KB loads per wave per slab
    static constexpr int GPR = BK / 8;                           // L_K: 16-byte groups per row
    static constexpr int RPC = 64 / GPR;                         // L_K: rows per 1 KB chunk
    static constexpr int VPK = ROWS / 8;                         // L_MN: vectors per k row
    static constexpr int KPC = 64 / VPK;                         // L_MN: k rows per chunk
    static_assert(LAYOUT == L_K || LAYOUT == L_MN, "16-byte vector layouts only");
    static_assert(NI * 4 * 1024 == STAGE_BYTES, "whole chunks per wave");

    // L_K, by row: (r / 4) % 4 for the 32x32x16 fragment reads (32 rows by
    // two groups per ds_read_b128), (r / 2) % 4 for the 16x16x32 ones (16
    // rows by four groups).  Both measured free of bank conflicts
    // (SQ_LDS_BANK_CONFLICT); the 16x16 reads under (r / 4) % 4 measured 4
    // conflict cycles per read, although 16 consecutive lanes of them hit 16
    // distinct bank groups: the hardware does not serve ds_read_b128 as
    // 16 consecutive lanes per cycle (a probe of seventeen lane patterns
    // fits lane groups of mixed bits instead).
    __device__ __forceinline__ static int swz_k(int r) {
        return M16 ? ((r >> 1) & 3) : (r >> 2) & 3;
    }
    // L_MN, by k row: 4 (k % 4); for the 16x16x32 reads (k rows 8 apart in
    // the two 16-lane groups a transposing read serves together) also
    // XORed with 2 ((k / 8) % 2).
    __device__ __forceinline__ static int swz_mn(int k) { return 4 * (k & 3) ^ (M16 ? 2 * ((k >> 3) & 1) : 0); }

    // Issues this wave's share of one slab.  base: operand at (batch, tile
    // row 0, slab k 0); rs / ks: row and k strides; rows_left / k_left:
    // valid extent from there; stage: LDS byte address of the stage.
    __device__ __forceinline__ static void load(const _Float16* base, int64_t rs, int64_t ks, int rows_left,
                                                int k_left, uint32_t stage, int lane, int wave) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c = i * 4 + wave;
            int r, k;
            if constexpr (LAYOUT == L_K) {
                const int row = c * RPC + lane / GPR;
                r = min(row, rows_left - 1);
                k = min(8 * ((lane % GPR) ^ swz_k(row)), k_left - 8);
            } else {
                const int kk = c * KPC + lane / VPK;
                k = min(kk, k_left - 1);
                r = min(8 * ((lane % VPK) ^ swz_mn(kk)), rows_left - 8);
            }
            const _Float16* g = base + int64_t(r) * rs + int64_t(k) * ks;
            const uint32_t l = stage + uint32_t(c) * 1024u;
            asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                         : : "v"(g), "s"(l) : "memory", "m0");
        }
    }

    // Per-lane byte offsets, from the tile's base at the slab's first k, of
    // this wave's NI loads of a full slab (no k clamp needed: every k of a
    // full slab is in range).
    __device__ __forceinline__ static void offsets(int64_t rs, int64_t ks, int rows_left, int lane, int wave,
                                                   uint32_t (&off)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c = i * 4 + wave;
            int r, k;
            if constexpr (LAYOUT == L_K) {
                const int row = c * RPC + lane / GPR;
                r = min(row, rows_left - 1);
                k = 8 * ((lane % GPR) ^ swz_k(row));
            } else {
                k = c * KPC + lane / VPK;
                r = min(8 * ((lane % VPK) ^ swz_mn(k)), rows_left - 8);
            }
            off[i] = uint32_t((int64_t(r) * rs + int64_t(k) * ks) * 2);
        }
    }

    // One direct load of a full slab: 16 bytes per lane from sbase + off
    // (sbase wave-uniform, in scalar registers) into LDS at `lds_addr`.
    __device__ __forceinline__ static void load1(const _Float16* sbase, uint32_t off, uint32_t lds_addr) {
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                     : : "v"(off), "s"(sbase), "s"(lds_addr) : "memory", "m0");
    }

    // Zeroes every k >= k_left (0 < k_left < BK) of a stage.
    __device__ __forceinline__ static void zero_tail(_Float16* stage, int k_left, int tid) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (LAYOUT == L_MN) {
            for (int idx = tid; idx < (BK - k_left) * VPK; idx += kGemmThreads) {
                const int k = k_left + idx / VPK, c = idx % VPK;
                *reinterpret_cast<f32x4*>(stage + k * ROWS + 8 * c) = z;
            }
        } else {
            for (int idx = tid; idx < ROWS * GPR; idx += kGemmThreads) {
                const int r = idx / GPR, slot = idx % GPR;
                if (8 * (slot ^ swz_k(r)) >= k_left) *reinterpret_cast<f32x4*>(stage + r * BK + 8 * slot) = z;
            }
        }
    }

    // Per-lane byte offsets of the fragment reads, relative to the wave's
    // first row (a multiple of 128) in a stage.
    //   L_K : o[st] for k step st (logical group 2 st + lane / 32 of row
    //         lane % 32); block i adds 32 * 64 i bytes.
    //   L_MN: o[j] for block j (columns 32 j .. 32 j + 31): lane l of 16-lane
    //         group G points at k row 8 (G / 2) + y (y = (l % 16) / 4) and
    //         columns 16 (G % 2) + 4 (l % 4); step st adds 16 st k rows and
    //         the second half-read 4 k rows.
    struct LaneOff {
        uint32_t o[4];
    };
    __device__ __forceinline__ static LaneOff lane_off(int lane) {
        LaneOff x;
        if constexpr (LAYOUT == L_K) {
            const int r = lane & 31, h = lane >> 5;
#pragma unroll
            for (int st = 0; st < 2; ++st) x.o[st] = uint32_t(r * BK * 2 + 16 * ((2 * st + h) ^ swz_k(r)));
            x.o[2] = x.o[3] = 0;
        } else {
            const int G = lane >> 4, i = lane & 15, y = i >> 2, q = i & 3;
            const int base = (8 * (G >> 1) + y) * ROWS * 2 + 16 * (2 * (G & 1) + (q >> 1)) + 8 * (q & 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) x.o[j] = uint32_t(base + 64 * (j ^ y));
        }
        return x;
    }

    // Fragment of block i (rows 32 i.. of the wave) for k step st.
    // wbase: LDS byte address of the stage plus the wave's row offset.
    __device__ __forceinline__ static f16x8 frag(uint32_t wbase, const LaneOff& lo, int i, int st) {
        if constexpr (LAYOUT == L_K) {
            const uint32_t a = wbase + lo.o[st] + uint32_t(i * 32 * BK * 2);
            return *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(uintptr_t(a));
        } else {
            const uint32_t a = wbase + lo.o[i] + uint32_t(st * 16 * ROWS * 2);
            const i16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<__attribute__((address_space(3))) i16x4*>(uintptr_t(a)));
            const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<__attribute__((address_space(3))) i16x4*>(uintptr_t(a + 4 * ROWS * 2)));
            typedef short i16x8 __attribute__((ext_vector_type(8)));
            const i16x8 w = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            return __builtin_bit_cast(f16x8, w);
        }
    }

    // v_mfma_f32_16x16x32_f16 fragments of block i (16 rows or columns).
    //   L_K : lane l reads row l % 16, logical group l / 16 (eight k); block
    //         i adds 16 * 64 i bytes.
    //   L_MN: two ds_read_b64_tr_b16: lane q of 16-lane group G points at k
    //         row 8 G + q / 4 (the second read 4 k rows on) and columns
    //         16 i + 4 (q % 4) .. + 3, so that after the transpose lane q
    //         holds column 16 i + q at k 8 G .. 8 G + 7; one offset per block
    //         (the swizzle is an XOR).
    struct LaneOff16 {
        uint32_t o[LAYOUT == L_K ? 1 : 8];
    };
    __device__ __forceinline__ static LaneOff16 lane_off16(int lane) {
        LaneOff16 x;
        if constexpr (LAYOUT == L_K) {
            const int r = lane & 15;
            x.o[0] = uint32_t(r * BK * 2 + 16 * ((lane >> 4) ^ swz_k(r)));
        } else {
            const int q = lane & 15, k = 8 * (lane >> 4) + (q >> 2);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                x.o[i] = uint32_t(k * ROWS * 2 + 16 * ((2 * i + ((q & 3) >> 1)) ^ swz_mn(k)) + 8 * (q & 1));
        }
        return x;
    }
    __device__ __forceinline__ static f16x8 frag16(uint32_t wbase, const LaneOff16& lo, int i) {
        if constexpr (LAYOUT == L_K) {
            const uint32_t a = wbase + lo.o[0] + uint32_t(i * 16 * BK * 2);
            return *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(uintptr_t(a));
        } else {
            const uint32_t a = wbase + lo.o[i];
            const i16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<__attribute__((address_space(3))) i16x4*>(uintptr_t(a)));
            const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<__attribute__((address_space(3))) i16x4*>(uintptr_t(a + 4 * ROWS * 2)));
            typedef short i16x8 __attribute__((ext_vector_type(8)));
            const i16x8 w = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            return __builtin_bit_cast(f16x8, w);
        }
    }

    // Byte offset of the wave's first row within a stage.
    __device__ __forceinline__ static uint32_t wave_row_off(int wrow0) {
        return LAYOUT == L_K ? uint32_t(wrow0 * BK * 2) : uint32_t(wrow0 * 2);
    }
};

// A wave-uniform 32-bit value in a scalar register.
__device__ __forceinline__ uint32_t big_uniform(uint32_t v) { return uint32_t(__builtin_amdgcn_readfirstlane(int(v))); }
// A wave-uniform pointer in scalar registers (each half widened as unsigned).
__device__ __forceinline__ const _Float16* big_uniform(const _Float16* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = big_uniform(uint32_t(v)), hi = big_uniform(uint32_t(v >> 32));
    return reinterpret_cast<const _Float16*>((uint64_t(hi) << 32) | uint64_t(lo));
}

// TAIL: K is not a whole number of 32-k slabs (the last slab of each tile
// has a K tail); without one, the per-slab tail checks are compiled out.
// M16 (k-contiguous A only): each wave's 128 x 128 tile as 8 x 8
// blocks of v_mfma_f32_16x16x32_f16, one MFMA per block and slab (64 per
// slab, accumulators in all 256 AGPRs), the next slab's 16 fragments read
// into a second register set during the slab's MFMAs; the same loads, LDS
// ring and barriers as the 32x32x16 schedule.
template <int AL, int BL, bool TAIL, bool M16>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_big_kernel(GemmArgs g) {
    using OA = BigOperand<AL, M16>;
    using OB = BigOperand<BL, M16>;
    constexpr int BM = kBigTile, BN = kBigTile, BK = kBigBK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr uint32_t STAGE = OA::STAGE_BYTES + OB::STAGE_BYTES;   // one slab of A and B: 32 KB
    constexpr uint32_t RING = kBigStages * STAGE;                   // 128 KB
    static_assert((RING & (RING - 1)) == 0, "stage offsets wrap with a mask");
    // Past the ring: one 1 KB chunk per wave that the streamed loads of a
    // slab with nothing to stream write into (never read), so those loads
    // need no branch.
    constexpr uint32_t SPARE = 4 * 1024;
    static_assert(RING + SPARE <= 160 * 1024, "LDS budget");
    static_assert(OA::NI == 4 && OB::NI == 4, "the schedule places four loads per operand per slab");
    __shared__ __attribute__((aligned(1024))) _Float16 lds[(RING + SPARE) / 2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t tiles_all = g.tiles_per_batch * g.nbatch_total;
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(
        (const __attribute__((address_space(3))) _Float16*)(lds)));
    const int nslabs = (g.K + BK - 1) / BK;                  // slabs per tile (every tile has all of K)
    const int tail_slab = TAIL ? nslabs - 1 : nslabs;        // the slab with a K tail, if any
    // Byte steps of the load pointers per slab.
    const int64_t step_a = int64_t(BK) * g.a_ks, step_b = int64_t(BK) * g.b_ks;

    struct Tile {
        const _Float16* A;
        const _Float16* B;
        int64_t c_off;
        int m0, n0, rows_a, rows_b;
    };
    auto locate = [&](uint32_t bid) {
        Tile x;
        const uint32_t batch = bid / g.tiles_per_batch;
        const uint32_t t = bid - batch * g.tiles_per_batch;
        // Groups of kBigGroupRows tile rows, walked column by column.
        const uint32_t gsz = uint32_t(kBigGroupRows) * uint32_t(g.tiles_n);
        const uint32_t grp = t / gsz;
        const uint32_t first = grp * kBigGroupRows;
        const uint32_t gm = min(uint32_t(g.tiles_m) - first, uint32_t(kBigGroupRows));
        const uint32_t w = t - grp * gsz;
        const uint32_t tn = w / gm;
        const uint32_t tm = first + (w - tn * gm);
        // One batch axis at most (the host merges composable batch axes and
        // sends other GEMMs elsewhere): no kernel-argument array indexed at
        // run time, so the loop holds no scalar-memory load, whose
        // out-of-order completion would force full LDS-count waits.
        const int64_t a_off = int64_t(batch) * g.a_bs[0];
        const int64_t b_off = int64_t(batch) * g.b_bs[0];
        x.c_off = int64_t(batch) * g.c_bs[0];
        x.m0 = int(big_uniform(tm)) * BM;
        x.n0 = int(big_uniform(tn)) * BN;
        x.rows_a = g.M - x.m0;
        x.rows_b = g.N - x.n0;
        x.A = big_uniform(static_cast<const _Float16*>(g.a) + a_off + int64_t(x.m0) * g.a_ms);
        x.B = big_uniform(static_cast<const _Float16*>(g.b) + b_off + int64_t(x.n0) * g.b_ns);
        return x;
    };

    const typename OA::LaneOff loa = OA::lane_off(lane);
    const typename OB::LaneOff lob = OB::lane_off(lane);
    const uint32_t wa_off = OA::wave_row_off(wm * WM), wb_off = OB::wave_row_off(wn * WN);

    TileWalk walk(tiles_all);
    uint32_t cbid = walk.next;
    if (cbid >= walk.end) return;
    Tile ct = locate(cbid);  // tile being computed
    // Load side: tile lt, its next slab ls, the scalar pointers of that slab,
    // the LDS stage (byte offset in the ring) it goes to, and whether any
    // slab is left (lvalid).  gi counts the slabs issued.
    Tile lt = ct;
    uint32_t lbid = cbid;
    int ls = 0;
    bool lvalid = true;
    uint32_t lstage = 0;
    int gi = 0;
    const _Float16* pa = lt.A;
    const _Float16* pb = lt.B;
    uint32_t offa[OA::NI], offb[OB::NI];  // full-slab load offsets of tile lt
    OA::offsets(g.a_ms, g.a_ks, lt.rows_a, lane, wave, offa);
    OB::offsets(g.b_ns, g.b_ks, lt.rows_b, lane, wave, offb);

    // Moves the load side on by one slab (to the next tile after the last).
    auto advance_load = [&]() {
        ++gi;
        lstage = (lstage + STAGE) & (RING - 1);
        pa += step_a;
        pb += step_b;
        if (__builtin_expect(++ls == nslabs, 0)) {
            lbid += walk.step;
            lvalid = lbid < walk.end;
            if (lvalid) {
                lt = locate(lbid);
                ls = 0;
                pa = lt.A;
                pb = lt.B;
                OA::offsets(g.a_ms, g.a_ks, lt.rows_a, lane, wave, offa);
                OB::offsets(g.b_ns, g.b_ks, lt.rows_b, lane, wave, offb);
            }
        }
    };
    // A whole slab outside the MFMA stream: the prologue, and slabs with a K
    // tail (every address clamped).
    auto issue_whole = [&]() {
        if (!lvalid) return;
        if (TAIL && ls == tail_slab) {
            const int kl = g.K - ls * BK;
            OA::load(pa, g.a_ms, g.a_ks, lt.rows_a, kl, lds0 + lstage, lane, wave);
            OB::load(pb, g.b_ns, g.b_ks, lt.rows_b, kl, lds0 + lstage + OA::STAGE_BYTES, lane, wave);
        } else {
#pragma unroll
            for (int i = 0; i < OA::NI; ++i) OA::load1(pa, offa[i], lds0 + lstage + uint32_t(i * 4 + wave) * 1024u);
#pragma unroll
            for (int i = 0; i < OB::NI; ++i)
                OB::load1(pb, offb[i], lds0 + lstage + OA::STAGE_BYTES + uint32_t(i * 4 + wave) * 1024u);
        }
        advance_load();
    };
    // Zeroes the K tail of the stage at byte offset `stage` (the slab with
    // index `slab` in its tile) when it has one.
    auto tail_fix = [&](int slab, uint32_t stage) {
        if (TAIL && slab == tail_slab) {
            const int k_left = g.K - slab * BK;
            OA::zero_tail(reinterpret_cast<_Float16*>(lds) + stage / 2, k_left, tid);
            OB::zero_tail(reinterpret_cast<_Float16*>(lds) + (stage + OA::STAGE_BYTES) / 2, k_left, tid);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
    };

    // Prologue: slabs 0, 1, 2 in flight; wait for slab 0.
#pragma unroll
    for (int p = 0; p < kBigStages - 1; ++p) issue_whole();
    if (gi >= 3) asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
    else if (gi == 2) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    tail_fix(0, 0);

    if constexpr (M16) {
        static_assert(AL == L_K, "16x16x32 schedule: k-contiguous A");
        uint32_t cstage = 0;  // byte offset of the stage being computed
        int gs = 0;           // slabs computed
        const typename OA::LaneOff16 loa16 = OA::lane_off16(lane);
        const typename OB::LaneOff16 lob16 = OB::lane_off16(lane);
        f16x8 xa[8], xb[8], ya[8], yb[8];
        // Fragment reads in the order the MFMAs use them (A 0, B 0..7, A 1..7).
        auto read16 = [&](f16x8 (&fa)[8], f16x8 (&fb)[8], uint32_t a, uint32_t b, int u) {
            if (u == 0) fa[0] = OA::frag16(a, loa16, 0);
            else if (u <= 8) fb[u - 1] = OB::frag16(b, lob16, u - 1);
            else fa[u - 8] = OA::frag16(a, loa16, u - 8);
        };
#pragma unroll
        for (int u = 0; u < 16; ++u) read16(xa, xb, lds0 + wa_off, lds0 + OA::STAGE_BYTES + wb_off, u);

        for (;;) {
            f32x4 acc[8][8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
            // One slab of tile ct from fragments (ca, cb), reading the next
            // slab's into (na_, nb_); true after the tile's last slab.
            auto slab = [&](const f16x8 (&ca)[8], const f16x8 (&cb)[8], f16x8 (&na_)[8], f16x8 (&nb_)[8], int cs) {
                if (__builtin_expect(gi - gs > 2, 1)) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
                const bool last = cs + 1 == nslabs;
                const bool more = !last || cbid + walk.step < walk.end;
                const uint32_t nstage = (cstage + STAGE) & (RING - 1);
                if (TAIL && more) tail_fix(last ? 0 : cs + 1, nstage);
                const bool fast = lvalid && (!TAIL || ls != tail_slab);
                if (TAIL && !fast) issue_whole();
                const _Float16* sa = fast ? pa : static_cast<const _Float16*>(g.a);
                const _Float16* sb = fast ? pb : static_cast<const _Float16*>(g.b);
                const uint32_t spare = lds0 + RING + uint32_t(wave) * 1024u;
                const uint32_t la = lds0 + lstage + uint32_t(wave) * 1024u;
                const uint32_t lb = la + OA::STAGE_BYTES;
                const uint32_t lda = fast ? 4096u : 0u;
                const uint32_t na = lds0 + nstage + wa_off, nb = lds0 + nstage + OA::STAGE_BYTES + wb_off;
                __builtin_amdgcn_s_setprio(1);
                __builtin_amdgcn_sched_barrier(0);
                // 64 MFMAs; the next slab's reads in slots 1, 5, .., 61, the load
                // slab's A loads in slots 2, 18, 34, 50 and B loads in 10, 26,
                // 42, 58.
#pragma unroll
                for (int t = 0; t < 64; ++t) {
                    acc[t / 8][t % 8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ca[t / 8], cb[t % 8], acc[t / 8][t % 8], 0, 0, 0);
                    if (t % 4 == 1) read16(na_, nb_, na, nb, t / 4);
                    else if (t % 16 == 2) OA::load1(sa, fast ? offa[t / 16] : 0u, (fast ? la : spare) + uint32_t(t / 16) * lda);
                    else if (t % 16 == 10) OB::load1(sb, fast ? offb[t / 16] : 0u, (fast ? lb : spare) + uint32_t(t / 16) * lda);
                    if (t == 63 && fast) advance_load();
                    __builtin_amdgcn_sched_barrier(0);
                }
                __builtin_amdgcn_s_setprio(0);
                cstage = nstage;
                ++gs;
                return last;
            };
            // Slabs in pairs (the host sends only tiles of an even number of
            // slabs here), so each register set keeps its role.
            for (int cs = 0;; cs += 2) {
                slab(xa, xb, ya, yb, cs);
                if (__builtin_expect(slab(ya, yb, xa, xb, cs + 1), 0)) break;
            }

            const int ntm = g.store_nt;  // store flavour (nt_mode)
            float* __restrict__ C = g.c + ct.c_off;
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
            const int wm0 = ct.m0 + wm * WM, wn0 = ct.n0 + wn * WN;
            const float* wbase = dl_uniform_base(C + int64_t(wm0) * g.c_ms + int64_t(wn0) * g.c_ns);
            uint32_t cms4 = uint32_t(__builtin_amdgcn_readfirstlane(int(g.c_ms) * 4));
            uint32_t cns4 = uint32_t(__builtin_amdgcn_readfirstlane(int(g.c_ns) * 4));
            uint32_t ln = uint32_t(lane);
            int rrem = __builtin_amdgcn_readfirstlane(g.M - wm0), crem = __builtin_amdgcn_readfirstlane(g.N - wn0);
            asm volatile("" : "+s"(cms4), "+s"(cns4), "+v"(ln), "+s"(rrem), "+s"(crem));
            const uint32_t lo = (ln >> 4) * 4u * cms4 + (ln & 15u) * cns4;
            if (ct.m0 + BM <= g.M && ct.n0 + BN <= g.N) {
                if (ntm == 2) big_store_tile16<2, false>(wbase, lo, cms4, cns4, 0, 0, acc);
                else if (ntm == 1) big_store_tile16<1, false>(wbase, lo, cms4, cns4, 0, 0, acc);
                else big_store_tile16<0, false>(wbase, lo, cms4, cns4, 0, 0, acc);
    
    } else {
            const int rr = rrem - 4 * int(ln >> 4), cr = crem - int(ln & 15u);
            // (partial tiles: the system-scope flavour is not instantiated)
            if (ntm != 0) big_store_tile16<1, true>(wbase, lo, cms4, cns4, rr, cr, acc);
            else big_store_tile16<0, true>(wbase, lo, cms4, cns4, rr, cr, acc);
        }
        cbid += walk.step;
        if (cbid >= walk.end) break;
        ct = locate(cbid);
    }
    } else {
        uint32_t cstage = 0;  // byte offset of the stage being computed
        int gs = 0;           // slabs computed
        f16x8 f0a[FM], f0b[FN], f1a[FM], f1b[FN];
        // Fragment reads in the order the MFMAs use them (A 0, B 0..3, A 1..3):
        // unit u of step st from the stage at (a, b).
        auto read_unit = [&](f16x8 (&fa)[FM], f16x8 (&fb)[FN], uint32_t a, uint32_t b, int u, int st) {
            if (u == 0) fa[0] = OA::frag(a, loa, 0, st);
            else if (u <= 4) fb[u - 1] = OB::frag(b, lob, u - 1, st);
            else fa[u - 4] = OA::frag(a, loa, u - 4, st);
        };
    #pragma unroll
        for (int u = 0; u < 8; ++u) read_unit(f0a, f0b, lds0 + wa_off, lds0 + OA::STAGE_BYTES + wb_off, u, 0);

        for (;;) {
            f32x16 acc[FM][FN];
    #pragma unroll
            for (int i = 0; i < FM; ++i)
    #pragma unroll
                for (int j = 0; j < FN; ++j)
    #pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
            for (int cs = 0;; ++cs) {
                // Slab cs of tile ct is visible and its step-0 fragments are
                // read.  Wait for this wave's loads of the next slab; the barrier
                // then makes every wave's visible and frees the stage read two
                // slabs ago, which this iteration refills.  (Loads complete in
                // issue order; at most the slab after next is in flight.)
                if (__builtin_expect(gi - gs > 2, 1)) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
                const bool last = cs + 1 == nslabs;
                const bool more = !last || cbid + walk.step < walk.end;
                const uint32_t nstage = (cstage + STAGE) & (RING - 1);
                if (TAIL && more) tail_fix(last ? 0 : cs + 1, nstage);
                // The load slab of this iteration: streamed between the MFMAs
                // unless it has a K tail (then issued whole, here).
                const bool fast = lvalid && (!TAIL || ls != tail_slab);
                if (TAIL && !fast) issue_whole();
                // A slab with nothing to stream (the block's last slabs, or the
                // load slab has a K tail and went whole above) still issues its
                // eight streamed loads, each lane reading the operand's first 16
                // bytes (in bounds for any shape), into the spare chunk: a
                // branch around each load made the wave refetch instructions
                // between MFMAs, with one wave per SIMD leaving the matrix core
                // idle.
                const _Float16* sa = fast ? pa : static_cast<const _Float16*>(g.a);
                const _Float16* sb = fast ? pb : static_cast<const _Float16*>(g.b);
                const uint32_t spare = lds0 + RING + uint32_t(wave) * 1024u;
                const uint32_t la = lds0 + lstage + uint32_t(wave) * 1024u;
                const uint32_t lb = la + OA::STAGE_BYTES;
                const uint32_t lda = fast ? 4096u : 0u;  // LDS step between a wave's loads of a slab
                const uint32_t ba = lds0 + cstage + wa_off, bb = lds0 + cstage + OA::STAGE_BYTES + wb_off;
                const uint32_t na = lds0 + nstage + wa_off, nb = lds0 + nstage + OA::STAGE_BYTES + wb_off;
                __builtin_amdgcn_s_setprio(1);
                __builtin_amdgcn_sched_barrier(0);
                // Step 0 and step 1, 32 MFMAs, with the slab's other instructions
                // between them: the load slab's eight loads one per four MFMAs (A
                // at step-0 slots 0, 4, 8, 12, B at step-1 slots 2, 6, 10, 14:
                // each 1 KB load holds the CU's address unit for about 16
                // cycles, so the four waves' 32 loads fit a slab only when
                // spread), the step-1 fragment reads in step 0's odd slots, the
                // next slab's step-0 reads in step 1's odd slots, and the scalar
                // bookkeeping for the next iteration in the remaining slots, in
                // the shadow of the MFMAs (issued anywhere else, it would leave
                // the matrix core idle while it runs).
    #pragma unroll
                for (int t = 0; t < 16; ++t) {
                    acc[t / 4][t % 4] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(f0a[t / 4], f0b[t % 4], acc[t / 4][t % 4], 0, 0, 0);
                    if (t % 2 == 1) read_unit(f1a, f1b, ba, bb, t / 2, 1);
                    else if (t % 4 == 0) OA::load1(sa, fast ? offa[t / 4] : 0u, (fast ? la : spare) + uint32_t(t / 4) * lda);
                    __builtin_amdgcn_sched_barrier(0);
                }
    #pragma unroll
                for (int t = 0; t < 16; ++t) {
                    acc[t / 4][t % 4] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(f1a[t / 4], f1b[t % 4], acc[t / 4][t % 4], 0, 0, 0);
                    // (The next slab's reads are issued even after the block's
                    // last slab, when their values go unused: reads of an LDS
                    // stage are always in bounds, and a read under a branch would
                    // leave the compiler unsure how many LDS reads are in flight,
                    // so it would wait for all of them before the MFMAs below.)
                    if (t % 2 == 1) read_unit(f0a, f0b, na, nb, t / 2, 0);
                    else if (t % 4 == 2) OB::load1(sb, fast ? offb[t / 4] : 0u, (fast ? lb : spare) + uint32_t(t / 4) * lda);
                    // (After the slab's last load: a move to the next tile
                    // recomputes the load offsets.)
                    if (t == 15 && fast) advance_load();
                    __builtin_amdgcn_sched_barrier(0);
                }
                __builtin_amdgcn_s_setprio(0);
                cstage = nstage;
                ++gs;
                if (__builtin_expect(last, 0)) break;
            }

            // Epilogue: the accumulators straight to the output.
            const int ntm = g.store_nt;  // store flavour (nt_mode)
            float* __restrict__ C = g.c + ct.c_off;
            // The store assembly reads accumulators the MFMAs just wrote, a read
            // the compiler cannot see: keep every MFMA above this point and leave
            // the wait states an MFMA result needs before a vector-memory
            // instruction reads it.
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
            const int wm0 = ct.m0 + wm * WM, wn0 = ct.n0 + wn * WN;
            const float* wbase = dl_uniform_base(C + int64_t(wm0) * g.c_ms + int64_t(wn0) * g.c_ns);
            // (wave-uniform values, moved to scalar registers explicitly: the
            // assembly below takes them as scalar operands)
            uint32_t cms4 = uint32_t(__builtin_amdgcn_readfirstlane(int(g.c_ms) * 4));
            uint32_t cns4 = uint32_t(__builtin_amdgcn_readfirstlane(int(g.c_ns) * 4));
            uint32_t ln = uint32_t(lane);
            int rrem = __builtin_amdgcn_readfirstlane(g.M - wm0), crem = __builtin_amdgcn_readfirstlane(g.N - wn0);
            asm volatile("" : "+s"(cms4), "+s"(cns4), "+v"(ln), "+s"(rrem), "+s"(crem));
            const uint32_t lo = (ln >> 5) * 4u * cms4 + (ln & 31u) * cns4;
            if (ct.m0 + BM <= g.M && ct.n0 + BN <= g.N) {
                if (ntm == 2) big_store_tile<2, false>(wbase, lo, cms4, cns4, 0, 0, acc);
                else if (ntm == 1) big_store_tile<1, false>(wbase, lo, cms4, cns4, 0, 0, acc);
                else big_store_tile<0, false>(wbase, lo, cms4, cns4, 0, 0, acc);
            } else {
                const int rr = rrem - 4 * int(ln >> 5), cr = crem - int(ln & 31u);
                // (partial tiles: the system-scope flavour is not instantiated)
                if (ntm != 0) big_store_tile<1, true>(wbase, lo, cms4, cns4, rr, cr, acc);
                else big_store_tile<0, true>(wbase, lo, cms4, cns4, rr, cr, acc);
            }
            cbid += walk.step;
            if (cbid >= walk.end) break;
            ct = locate(cbid);
        }
    }
}

}  // namespace pe
