// Batched GEMM with direct global -> LDS operand loads (gfx950), float32
// and float16 operands, float32 accumulation and output.
//
// Same contract and tile walk as gemm_kernel (pe_gemm_kernel.h), for operands
// whose 16-byte vectors run along M / N (L_MN) or along K (L_K).  What
// differs is how a slab reaches LDS:
//
//  * each wave issues global_load_lds_dwordx4: 64 lanes x 16 bytes land in one
//    1 KB LDS chunk, lane p at byte 16 p, with no register staging and no
//    ds_write;
//  * two LDS stages: the loads of slab s+1 (of this tile, or the first slab
//    of the block's next tile) are in flight while slab s feeds the MFMAs,
//    so every slab costs one barrier and the next tile's first slab overlaps
//    the current tile's epilogue;
//  * each lane reads its MFMA fragments for the next k step while the
//    current step's MFMAs issue.
//
// A slab is 64 bytes of k per row: 16 float32 (8 steps of
// v_mfma_f32_32x32x2_f32) or 32 float16 (2 steps of v_mfma_f32_32x32x16_f16).
// LDS layouts per stage:
//   L_MN: [BK][ROWS] k-major.  float32 fragments are one 32-lane contiguous
//         read per k.  float16 fragments (8 consecutive k of one row per
//         lane) come from two ds_read_b64_tr_b16: within each 16-lane group,
//         lane i receives element i % 4 of the 8-byte blocks addressed by
//         lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4, so lanes 4 j + q
//         pointing at k row kb + j, columns n0 + 4 q give lane i the four k
//         values of column n0 + i.  The 16-byte groups of a float16 k row
//         are XOR-swizzled by 2 (k % 4), so the four rows of one such read
//         fall in eight distinct groups (no bank conflicts).
//   L_K : [ROWS][BK] k contiguous, 16-byte groups XOR-swizzled by
//         (row / 4) % 4, so the lanes of one read phase (consecutive rows at
//         one k) hit distinct banks.
// A lane's load fetches the global vector that its swizzled slot holds.  Both
// operands use the same k order inside a slab: lane half h = lane / 32 of MFMA
// step st consumes k = 8 h + st (float32) or 16 st + 8 h + 0..7 (float16).
//
// Boundaries: rows past M / N load a clamped (in-bounds) vector and only
// feed outputs that are never stored.  The K tail of a tile's last slab
// loads clamped (in-bounds) data and is then overwritten with zeros in LDS
// before any MFMA reads it, so no value from outside the operand reaches a
// stored sum.  Host-side conditions (see gemm_dl_eligible): L_MN operands
// need M (resp. N) to be a whole number of 16-byte vectors, L_K operands K
// (and so every split's k extent), and both 16-byte aligned vectors; the
// output's strides keep every element of a tile within 2^31 bytes of the
// tile's corner (32-bit store offsets).
#pragma once

#include "pe_gemm_kernel.h"


namespace pe {

// Output stores of one wave's tile, as inline assembly: a compiler-issued
// store would be a tracked vector-memory operation, and the compiler then
// waits for the whole vector-memory counter (in-flight slab loads included)
// before reusing any register the store read.  Addressing: one wave-uniform
// 64-bit base in scalar registers and a 32-bit byte offset per lane; each
// store adds one of four uniform row offsets to its row group's lane offset
// in the same assembly block, so one temporary register serves every store.
// Register 4 q + s of fragment block (i, j) is row 32 i + 8 q + s (plus 4 in
// the upper half-wave, folded into lane_off) and column 32 j (plus the
// lane's column, also in lane_off).  cms4 / cns4: row / column strides in
// bytes.  MASKED: only rows below rrem and columns below crem (both relative
// to the lane's first element) are stored.  The caller passes the strides
// and lane values through opaque moves made in the epilogue, so nothing
// derived from them is hoisted out of the tile loop to hold registers through
// the MFMA loop.
template <int NTM, bool MASKED, int FM, int FN>
__device__ __forceinline__ void dl_store_tile(const float* wbase, uint32_t lane_off, uint32_t cms4, uint32_t cns4,
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
                                     : "s"(rs[r]), "v"(bq), "v"(acc[i][j][4 * q + r]), "s"(wbase));
                    else if constexpr (NTM == 1)
                        asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4 nt"
                                     : "=&v"(t)
                                     : "s"(rs[r]), "v"(bq), "v"(acc[i][j][4 * q + r]), "s"(wbase));
                    else
                        asm volatile("v_add_u32 %0, %1, %2\n\tglobal_store_dword %0, %3, %4"
                                     : "=&v"(t)
                                     : "s"(rs[r]), "v"(bq), "v"(acc[i][j][4 * q + r]), "s"(wbase));
                }
            }
        }
}

// A wave-uniform 64-bit address moved to scalar registers for use as the
// scalar base of vector-memory instructions.  The moves are the compiler's
// readfirstlane (it keeps the wait state a readfirstlane needs after the
// vector instruction that wrote its source); each half is widened as
// unsigned (readfirstlane returns int, and a sign-extended low half would
// corrupt the high half).  A vector instruction writing a scalar register
// that a vector-memory instruction then reads needs five wait states: the
// s_nop, which the stores depend on through the base.
__device__ __forceinline__ const float* dl_uniform_base(const float* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(v)));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(v >> 32)));
    const float* b = reinterpret_cast<const float*>((uint64_t(hi) << 32) | uint64_t(lo));
    asm volatile("s_nop 4" : "+s"(b));
    return b;
}

// LDS byte address of a pointer into a __shared__ array.  Taken once per
// stage at kernel entry, where it folds to a constant: converted inside the
// slab loop, the generic pointer is kept live and null-checked per load.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

// 16 bytes per lane from global memory into LDS at lds + 16 * lane.  Written
// as inline assembly so the compiler does not treat the in-flight load as a
// pending write to every LDS array: it would otherwise wait for it before the
// first read of the other stage, serialising loads and MFMAs.  Completion is
// awaited explicitly (s_waitcnt vmcnt(0) before the barrier of the slab that
// reads it).
__device__ __forceinline__ void dma16(const float* gptr, uint32_t lds) {
    // The LDS address is wave-uniform (M0 takes a scalar register).
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
    // One wait state between writing M0 and the load that reads it.
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(l) : "memory", "m0");
}
__device__ __forceinline__ void dma16(const float* gptr, const float* lds) { dma16(gptr, lds_addr(lds)); }

// As dma16, from a wave-uniform 64-bit base (scalar registers) plus a
// per-lane 32-bit byte offset: no per-lane 64-bit address arithmetic.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t off, uint32_t lds) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 : : "v"(off), "s"(sbase), "s"(l) : "memory", "m0");
}

// Per-type slab geometry and MFMA.
template <typename E>
struct DlMath;
template <>
struct DlMath<F32> {
    static constexpr int BK = 16;     // k per slab (64 bytes)
    static constexpr int STEPS = 8;   // MFMA k steps per slab
    using Frag = float;
    __device__ __forceinline__ static f32x16 mfma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};
template <>
struct DlMath<F16> {
    static constexpr int BK = 32;
    static constexpr int STEPS = 2;
    using Frag = f16x8;
    __device__ __forceinline__ static f32x16 mfma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));

// One operand's share of a slab: ROWS rows (m or n) x BK k.  Stateless:
// per-lane offsets are recomputed from the lane index at each use, so no
// register stays live across slabs for them.
template <typename E, int ROWS, int LAYOUT, bool SMALL_TILE>
struct DlOperand {
    using T = typename E::T;
    static_assert(LAYOUT == L_MN || LAYOUT == L_K, "direct loads need 16-byte vectors");
    static constexpr bool kF32 = E::kBytes == 4;
    static constexpr int BK = DlMath<E>::BK;
    static constexpr int EPV = 16 / E::kBytes;        // elements per 16-byte vector
    static constexpr int ELEMS = ROWS * BK;           // elements per stage
    static constexpr int NCHUNK = ELEMS * E::kBytes / 1024;  // 1 KB chunks, one wave instruction each
    static constexpr int NI = NCHUNK / 4;             // instructions per wave per slab
    static constexpr int LPR = ROWS / EPV;            // L_MN: lanes (vectors) per k row
    static constexpr int KPC = 64 / LPR;              // L_MN: k rows per chunk
    static_assert(kF32 || LAYOUT == L_K || LPR >= 8, "float16 k-major swizzle needs 8 vectors per row");
    // float32 L_K fragments: four k per 16-byte read in tiles of at most
    // 128 x 128; 256-wide tiles keep 8-byte reads (k pairs), whose smaller
    // ring fits the register budget of three resident blocks per CU.
    static constexpr bool kQuadK = kF32 && LAYOUT == L_K && SMALL_TILE;
    // Fragment ring.  float32: L_MN reads one k per step (current + next);
    // L_K reads four k (or a k pair) at a time, the next ones while the
    // current ones are consumed.  float16: one 8-element fragment per step
    // (current + next).
    static constexpr int RING = !kF32 ? 2 : (LAYOUT == L_MN ? 2 : (kQuadK ? 8 : 4));
    using Frag = typename DlMath<E>::Frag;

    // float16 k-major swizzle: logical 16-byte group g of k row k sits at
    // g ^ (2 (k % 4)).
    __device__ __forceinline__ static int kswz(int k) { return kF32 ? 0 : 2 * (k & 3); }

    // Issues the slab's loads into `stage`.  base: operand at (batch, tile
    // row 0, slab k 0); rows_left / k_left: valid extent from there.
    // stage: LDS byte address.
    __device__ __forceinline__ static void load(const T* base, int64_t rs, int64_t ks, int rows_left,
                                                int k_left, uint32_t stage, int lane, int wave) {
        static_assert(NI >= 1 && NCHUNK % 4 == 0, "every wave issues whole chunks");
#pragma unroll
        for (int i = 0; i < NI; ++i) load_chunk(base, rs, ks, rows_left, k_left, stage, lane, i * 4 + wave);
    }
    __device__ __forceinline__ static void load(const T* base, int64_t rs, int64_t ks, int rows_left,
                                                int k_left, T* stage, int lane, int wave) {
        load(base, rs, ks, rows_left, k_left, lds_addr(stage), lane, wave);
    }

    // Row and k (relative to the stage's first row and k) that lane `lane`
    // fetches for chunk c (0 <= c < NCHUNK) of a stage, clamped into the
    // valid extent.  Needs rows_left >= EPV (L_MN) and k_left >= EPV (L_K)
    // or >= 1 (L_MN).
    __device__ __forceinline__ static void chunk_rk(int lane, int c, int rows_left, int k_left, int& r, int& k) {
        if constexpr (LAYOUT == L_MN) {
            const int kk = c * KPC + lane / LPR;
            k = min(kk, k_left - 1);
            r = min(((lane % LPR) ^ kswz(kk)) * EPV, rows_left - EPV);
        } else {
            r = min(c * 16 + lane / 4, rows_left - 1);
            k = min(EPV * ((lane % 4) ^ (lane / 16)), k_left - EPV);
        }
    }

    // One wave's load of chunk c of a stage.
    __device__ __forceinline__ static void load_chunk(const T* base, int64_t rs, int64_t ks, int rows_left,
                                                      int k_left, uint32_t stage, int lane, int c) {
        int r, k;
        chunk_rk(lane, c, rows_left, k_left, r, k);
        dma16(reinterpret_cast<const float*>(base + int64_t(r) * rs + int64_t(k) * ks), stage + uint32_t(c) * 1024u);
    }
    __device__ __forceinline__ static void load_chunk(const T* base, int64_t rs, int64_t ks, int rows_left,
                                                      int k_left, T* stage, int lane, int c) {
        load_chunk(base, rs, ks, rows_left, k_left, lds_addr(stage), lane, c);
    }

    // Full-slab loads (every k of the slab in range; for L_K also every row of
    // the tile) from one per-lane byte offset: this wave's chunk 4 i + wave
    // sits at base + i * chunk_step + full_off.  L_MN: chunks differ only in
    // k, by 4 KPC k rows (a multiple of 4, so the float16 swizzle and the row
    // clamp are the same for all of them); L_K: by 64 rows.  Needs every
    // offset below 2^32 bytes (GemmArgs::off32).
    __device__ __forceinline__ static uint32_t full_off(int64_t rs, int64_t ks, int rows_left, int lane, int wave) {
        int r, k;
        chunk_rk(lane, wave, rows_left, BK, r, k);
        return uint32_t((int64_t(r) * rs + int64_t(k) * ks) * E::kBytes);
    }
    __device__ __forceinline__ static int64_t chunk_step(int64_t rs, int64_t ks) {
        return LAYOUT == L_MN ? int64_t(4 * KPC) * ks : int64_t(64) * rs;
    }
    __device__ __forceinline__ static bool full_ok(int rows_left) { return LAYOUT == L_MN || rows_left >= ROWS; }
    __device__ __forceinline__ static void load_full(const T* base, int64_t step, uint32_t off, uint32_t stage,
                                                     int wave) {
#pragma unroll
        for (int i = 0; i < NI; ++i) dma16s(base + i * step, off, stage + uint32_t(i * 4 + wave) * 1024u);
    }

    // Zeroes every k >= k_left of a stage (0 < k_left < BK).
    __device__ __forceinline__ static void zero_tail(T* stage, int k_left, int tid) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (LAYOUT == L_MN) {
            const int n = (BK - k_left) * LPR;
            for (int idx = tid; idx < n; idx += kGemmThreads) {
                const int k = k_left + idx / LPR, c = (idx % LPR) * EPV;
                *reinterpret_cast<f32x4*>(stage + k * ROWS + c) = z;
            }
        } else {
            for (int idx = tid; idx < ROWS * 4; idx += kGemmThreads) {
                const int r = idx / 4, pc = idx % 4;
                const int lc = pc ^ ((r >> 2) & 3);
                if (EPV * lc >= k_left) *reinterpret_cast<f32x4*>(stage + r * BK + pc * EPV) = z;
            }
        }
    }

    // Per-lane fragment offsets (elements from the stage origin) for a wave
    // whose fragment rows start at wrow0 (a multiple of 32).
    //   float32 L_MN: o[0]; float32 L_K: o[q] per half slab (the swizzled
    //   group of k = 8 h + 4 q); float16 L_K: o[st] per step (group 2 st + h);
    //   float16 L_MN: o[par] for fragment blocks whose 8-column group index
    //   (wrow0 + 32 i) / 8 has bit 2 clear (par 0) or set (par 1), which the
    //   XOR swizzle folds into the lane's group.
    struct LaneOff {
        int o[2];
    };
    __device__ __forceinline__ static LaneOff lane_off(int lane, int wrow0) {
        const int h = lane >> 5, r = wrow0 + (lane & 31);
        LaneOff x;
        if constexpr (kF32 && LAYOUT == L_MN) {
            x.o[0] = 8 * h * ROWS + r;
            x.o[1] = 0;
        } else if constexpr (kF32) {
            // half slab q: lane half h owns k = 8 h .. 8 h + 7, groups 2 h + q
#pragma unroll
            for (int q = 0; q < 2; ++q) x.o[q] = r * BK + (((2 * h + q) ^ ((r >> 2) & 3)) * EPV);
        } else if constexpr (LAYOUT == L_K) {
            // step st: k = 16 st + 8 h .. + 7, group 2 st + h
#pragma unroll
            for (int st = 0; st < 2; ++st) x.o[st] = r * BK + (((2 * st + h) ^ ((r >> 2) & 3)) * EPV);
        } else {
            // Lane l of 16-lane group G = l / 16 points at k row 8 (G / 2) + j
            // (j = (l % 16) / 4) and columns n0 + 4 q (n0 = 16 (G % 2),
            // q = l % 4) of the fragment block; its 16-byte group is
            // (C + 2 (G % 2) + q / 2) ^ 2 j with C = (wrow0 + 32 i) / 8.
            const int G = lane >> 4, j = (lane & 15) >> 2, q = lane & 3;
            const int zz = (2 * (G & 1) + (q >> 1)) ^ (2 * j);
#pragma unroll
            for (int par = 0; par < 2; ++par)
                x.o[par] = (8 * (G >> 1) + j) * ROWS + 8 * (zz ^ (4 * par)) + 4 * (q & 1);
        }
        return x;
    }

    // Reads what MFMA step st needs for fragment block i (rows 32 i ..
    // 32 i + 31 of the wave, which starts at wrow0) into ring slot
    // st % RING.  float32 L_K reads four k at steps 0 and 4 (slots st ..
    // st + 3), or k pairs at even steps (slots st % 4 and (st + 1) % 4).
    // All offsets but the lane's are uniform.
    __device__ __forceinline__ static void frag(const T* stage, const LaneOff& lo, int wrow0, int i, int st,
                                                Frag (&v)[RING]) {
        if constexpr (kF32 && LAYOUT == L_MN) {
            v[st % 2] = stage[lo.o[0] + st * ROWS + i * 32];
        } else if constexpr (kF32) {
            // One 16-byte read per lane covers four steps.  A 16-lane phase
            // of ds_read_b128 spans rows r0 .. r0 + 15, whose (r % 4, group)
            // pairs are all distinct under the (r / 4) % 4 swizzle: no bank
            // conflicts.  8-byte reads (k pairs) are processed in 32-lane
            // phases that pair row r with row r + 16 on the same banks: two
            // ways in conflict.
            if constexpr (kQuadK) {
                if (st % 4 == 0) {
                    const f32x4 x = *reinterpret_cast<const f32x4*>(stage + lo.o[st / 4] + i * 32 * BK);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[st + e] = x[e];
                }
            } else if (st % 2 == 0) {
                typedef float f32x2 __attribute__((ext_vector_type(2)));
                const f32x2 x = *reinterpret_cast<const f32x2*>(stage + lo.o[st / 4] + i * 32 * BK + st % 4);
                v[st % 4] = x[0];
                v[(st + 1) % 4] = x[1];
            }
        } else if constexpr (LAYOUT == L_K) {
            v[st % 2] = *reinterpret_cast<const f16x8*>(stage + lo.o[st] + i * 32 * BK);
        } else {
            const int C = wrow0 / 8 + 4 * i;
            // A select, not an index: with 32-row wave tiles the parity
            // depends on the wave, and an indexed lane_off array would be
            // kept in scratch memory.
            const int lo_par = ((C >> 2) & 1) ? lo.o[1] : lo.o[0];
            const T* p = stage + lo_par + 8 * (C & ~7) + 16 * st * ROWS;
            const i16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(p));
            const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(p + 4 * ROWS));
            typedef short i16x8 __attribute__((ext_vector_type(8)));
            const i16x8 w = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            v[st % 2] = __builtin_bit_cast(f16x8, w);
        }
    }
};

// MINB: resident blocks per CU the register allocation is held to (four
// waves per block, one per SIMD, so MINB waves per SIMD).
template <typename E, int BM, int BN, int AL, int BL, int MINB>
__global__ __launch_bounds__(kGemmThreads, MINB) void gemm_dl_kernel(GemmArgs g) {
    using T = typename E::T;
    using M = DlMath<E>;
    using OA = DlOperand<E, BM, AL, (BM <= 128 && BN <= 128)>;
    using OB = DlOperand<E, BN, BL, (BM <= 128 && BN <= 128)>;
    constexpr int BK = M::BK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    __shared__ __attribute__((aligned(16))) T sa0[OA::ELEMS];
    __shared__ __attribute__((aligned(16))) T sa1[OA::ELEMS];
    __shared__ __attribute__((aligned(16))) T sb0[OB::ELEMS];
    __shared__ __attribute__((aligned(16))) T sb1[OB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5;
    const uint32_t tiles_all = g.tiles_per_batch * g.nbatch_total;

    struct Tile {
        const T* A;
        const T* B;
        int64_t c_off;
        uint32_t split, batch;
        int m0, n0, rows_a, rows_b, k_len, nslabs;
    };
    auto locate = [&](uint32_t bid) {
        Tile x;
        x.split = bid / tiles_all;
        uint32_t t = bid - x.split * tiles_all;
        x.batch = t / g.tiles_per_batch;
        t -= x.batch * g.tiles_per_batch;
        const int tm = int(t / uint32_t(g.tiles_n));
        const int tn = int(t - uint32_t(tm) * uint32_t(g.tiles_n));
        int64_t a_off = 0, b_off = 0, c_off = 0;
        uint32_t rem = x.batch;
        for (int d = g.nbatch - 1; d >= 0; --d) {
            uint32_t q, r;
            g.batch_div[d].divmod(rem, q, r);
            a_off += int64_t(r) * g.a_bs[d];
            b_off += int64_t(r) * g.b_bs[d];
            c_off += int64_t(r) * g.c_bs[d];
            rem = q;
        }
        x.m0 = tm * BM;
        x.n0 = tn * BN;
        const int kb = int(x.split) * g.k_per_split;
        x.k_len = min(g.K, kb + g.k_per_split) - kb;
        x.nslabs = (x.k_len + BK - 1) / BK;
        x.rows_a = g.M - x.m0;
        x.rows_b = g.N - x.n0;
        x.A = static_cast<const T*>(g.a) + a_off + int64_t(x.m0) * g.a_ms + int64_t(kb) * g.a_ks;
        x.B = static_cast<const T*>(g.b) + b_off + int64_t(x.n0) * g.b_ns + int64_t(kb) * g.b_ks;
        x.c_off = c_off;
        return x;
    };

    const typename OA::LaneOff loa = OA::lane_off(lane, wm * WM);
    const typename OB::LaneOff lob = OB::lane_off(lane, wn * WN);

    TileWalk walk(g.total_blocks);
    uint32_t cbid = walk.next;
    if (cbid >= walk.end) return;
    Tile ct = locate(cbid);  // tile being computed
    int cs = 0;              // its next slab
    Tile lt = ct;            // tile of the next load
    uint32_t lbid = cbid;
    int ls = 0;              // its next slab to load
    bool lvalid = true;

    // Per-lane byte offsets of the load tile's full slabs (computed once per
    // tile; the slab's base advances in scalar registers).
    uint32_t lofa = 0, lofb = 0;
    auto set_lo = [&]() {
        if (g.off32) {
            lofa = OA::full_off(g.a_ms, g.a_ks, lt.rows_a, lane, wave);
            lofb = OB::full_off(g.b_ns, g.b_ks, lt.rows_b, lane, wave);
        }
    };
    set_lo();
    const uint32_t la0 = lds_addr(sa0), la1 = lds_addr(sa1), lb0 = lds_addr(sb0), lb1 = lds_addr(sb1);
    auto issue = [&](uint32_t da, uint32_t db) {
        const int kl = lt.k_len - ls * BK;
        const T* pa = lt.A + int64_t(ls) * BK * g.a_ks;
        const T* pb = lt.B + int64_t(ls) * BK * g.b_ks;
        const bool full = g.off32 && kl >= BK;
        if (full && OA::full_ok(lt.rows_a))
            OA::load_full(pa, OA::chunk_step(g.a_ms, g.a_ks), lofa, da, wave);
        else
            OA::load(pa, g.a_ms, g.a_ks, lt.rows_a, kl, da, lane, wave);
        if (full && OB::full_ok(lt.rows_b))
            OB::load_full(pb, OB::chunk_step(g.b_ns, g.b_ks), lofb, db, wave);
        else
            OB::load(pb, g.b_ns, g.b_ks, lt.rows_b, kl, db, lane, wave);
        if (++ls == lt.nslabs) {
            lbid += walk.step;
            lvalid = lbid < walk.end;
            if (lvalid) {
                lt = locate(lbid);
                ls = 0;
                set_lo();
            }
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto epilogue = [&]() {
        float* __restrict__ C;
        int64_t cms, cns;
        const int ntm = g.store_nt;  // store flavour (nt_mode)
        if (g.nsplit > 1) {
            C = g.partial + ((int64_t(ct.split) * g.nbatch_total + ct.batch) * g.M) * int64_t(g.N);
            cms = g.N;
            cns = 1;
        } else {
            C = g.c + ct.c_off;
            cms = g.c_ms;
            cns = g.c_ns;
        }
        // The store assembly reads accumulators the MFMAs just wrote, a read
        // the compiler cannot see: keep every MFMA above this point and
        // leave the wait states an MFMA result needs before a vector-memory
        // instruction reads it (at most 20 on this target).
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
        // 32x32 accumulator layout: lane l, register r holds row
        // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of its block.
        const int wm0 = ct.m0 + wm * WM, wn0 = ct.n0 + wn * WN;
        const float* wbase = dl_uniform_base(C + int64_t(wm0) * cms + int64_t(wn0) * cns);
        uint32_t cms4 = uint32_t(cms) * 4u, cns4 = uint32_t(cns) * 4u, ln = uint32_t(lane);
        int rrem = g.M - wm0, crem = g.N - wn0;
        asm volatile("" : "+s"(cms4), "+s"(cns4), "+v"(ln), "+s"(rrem), "+s"(crem));
        const uint32_t lo = (ln >> 5) * 4u * cms4 + (ln & 31u) * cns4;
        if (ct.m0 + BM <= g.M && ct.n0 + BN <= g.N) {
            // The system-scope flavour only for float16 operands: a third
            // epilogue in the float32 kernel shifted its register allocation
            // (97 -> 96 VGPRs for 128x128 tiles), which let five blocks share
            // a CU and ran config 2 at 317 against 276 us.
            if (sizeof(T) == 2 && ntm == 2) dl_store_tile<2, false>(wbase, lo, cms4, cns4, 0, 0, acc);
            else if (ntm != 0) dl_store_tile<1, false>(wbase, lo, cms4, cns4, 0, 0, acc);
            else dl_store_tile<0, false>(wbase, lo, cms4, cns4, 0, 0, acc);
        } else {
            const int rr = rrem - 4 * int(ln >> 5), cr = crem - int(ln & 31u);
            // (partial tiles: the system-scope flavour is not instantiated)
            if (ntm != 0) dl_store_tile<1, true>(wbase, lo, cms4, cns4, rr, cr, acc);
            else dl_store_tile<0, true>(wbase, lo, cms4, cns4, rr, cr, acc);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    };

    // One slab: wait for its loads, start the next slab's loads into the
    // other stage, then the MFMAs.  Returns true when the block is done.
    auto step = [&](const T* sa, const T* sb, uint32_t na, uint32_t nb) -> bool {
        // This wave's loads of the slab have landed; after the barrier every
        // wave's have, and every wave is done reading the other stage.
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (lvalid) issue(na, nb);
        const int k_left = ct.k_len - cs * BK;
        if (k_left < BK) {
            OA::zero_tail(const_cast<T*>(sa), k_left, tid);
            OB::zero_tail(const_cast<T*>(sb), k_left, tid);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        typename M::Frag fa[FM][OA::RING], fb[FN][OB::RING];
        // Raised wave priority for the slab's fragment reads and MFMAs: the
        // SIMD then issues this wave's MFMAs ahead of other waves' loads and
        // address work (4096^3 float32 -3 %, 8192^3 float16 -1.5 % on one box).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < FM; ++i) OA::frag(sa, loa, wm * WM, i, 0, fa[i]);
#pragma unroll
        for (int j = 0; j < FN; ++j) OB::frag(sb, lob, wn * WN, j, 0, fb[j]);
#pragma unroll
        for (int st = 0; st < M::STEPS; ++st) {
            if (st + 1 < M::STEPS) {
#pragma unroll
                for (int i = 0; i < FM; ++i) OA::frag(sa, loa, wm * WM, i, st + 1, fa[i]);
#pragma unroll
                for (int j = 0; j < FN; ++j) OB::frag(sb, lob, wn * WN, j, st + 1, fb[j]);
            }
            // Keep the next step's reads ahead of this step's MFMAs (the
            // scheduler would otherwise sink them to save registers and wait
            // on each read in turn).
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = M::mfma(fa[i][st % OA::RING], fb[j][st % OB::RING], acc[i][j]);
        }
        __builtin_amdgcn_s_setprio(0);
        if (++cs == ct.nslabs) {
            epilogue();
            cbid += walk.step;
            if (cbid >= walk.end) return true;
            ct = locate(cbid);
            cs = 0;
        }
        return false;
    };

    issue(la0, lb0);
    for (;;) {
        if (step(sa0, sb0, la1, lb1)) break;
        if (step(sa1, sb1, la0, lb0)) break;
    }
}

// Short-K variant: every k slab of the tile resident in LDS at once.  One
// block per output tile (no split, no persistent walk); each wave issues the
// loads of all NS slabs into NS LDS stages up front and then computes slab by
// slab, waiting only until its own loads of that slab have landed (vmcnt
// counts the later slabs' loads still in flight) and for the other waves'
// (one barrier per slab).  For K in ((NS - 1) BK, NS BK]: the two-stage ring
// of gemm_dl_kernel keeps one slab of loads ahead of the MFMAs, and where a
// slab's MFMAs take far less than a load's latency (float16, 128 x 128
// tiles: 8 MFMAs of 32 cycles per wave and slab) its NS slabs cost NS load
// latencies in a row; here they cost one.  LDS: NS x (BM + BN) x 64 bytes
// (48 KB for the 64 x 128 float16 tiles at K = 128, three blocks per CU; a
// block keeps them until its output stores complete, and the other resident
// blocks load and multiply meanwhile).  Measured on MI355X: config 5.1
// (tn,sn->ts, 4096^2 x 128 float16, float32 out) with its output stores
// removed ran 9.5 us of its 17.8 (two-stage kernel); float32 short K
// (the GDN chunk products, K = 128 in eight slabs) ran slower than the
// two-stage kernel both as 128 x 128 tiles at one block per CU (22 against
// 20 us at 256 x 128^3, 68 against 54 us at 1024 x 128^3) and as 64 x 64
// tiles at two per CU (21-22 against 19.5-21 us at 256 x 128^3): float32
// MFMAs per slab take about as long as a load, so the two-stage ring at four
// blocks per CU already hides the latency, and fewer resident waves issue
// them less densely.
template <typename E, int BM, int BN, int AL, int BL, int NS, int MINB>
__global__ __launch_bounds__(kGemmThreads, MINB) void gemm_res_kernel(GemmArgs g) {
    using T = typename E::T;
    using M = DlMath<E>;
    using OA = DlOperand<E, BM, AL, true>;
    using OB = DlOperand<E, BN, BL, true>;
    constexpr int BK = M::BK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int PER_SLAB = OA::NI + OB::NI;  // load instructions per wave per slab
    static_assert((NS - 1) * PER_SLAB <= 63, "vmcnt counts at most 63 loads");
    __shared__ __attribute__((aligned(16))) T sa[NS][OA::ELEMS];
    __shared__ __attribute__((aligned(16))) T sb[NS][OB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    uint32_t t = blockIdx.x;
    const uint32_t batch = t / g.tiles_per_batch;
    t -= batch * g.tiles_per_batch;
    const int tm = int(t / uint32_t(g.tiles_n));
    const int tn = int(t - uint32_t(tm) * uint32_t(g.tiles_n));
    int64_t a_off = 0, b_off = 0, c_off = 0;
    uint32_t rem = batch;
    for (int d = g.nbatch - 1; d >= 0; --d) {
        uint32_t q, r;
        g.batch_div[d].divmod(rem, q, r);
        a_off += int64_t(r) * g.a_bs[d];
        b_off += int64_t(r) * g.b_bs[d];
        c_off += int64_t(r) * g.c_bs[d];
        rem = q;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const T* A = static_cast<const T*>(g.a) + a_off + int64_t(m0) * g.a_ms;
    const T* B = static_cast<const T*>(g.b) + b_off + int64_t(n0) * g.b_ns;
    const int rows_a = g.M - m0, rows_b = g.N - n0;

    // Every slab's loads, in slab order (loads complete in issue order, so
    // vmcnt(n) means all but this wave's last n loads have landed).  Full
    // slabs load from per-lane 32-bit offsets as in gemm_dl_kernel.
    const uint32_t lofa = g.off32 ? OA::full_off(g.a_ms, g.a_ks, rows_a, lane, wave) : 0u;
    const uint32_t lofb = g.off32 ? OB::full_off(g.b_ns, g.b_ks, rows_b, lane, wave) : 0u;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int kl = g.K - s * BK;
        const T* pa = A + int64_t(s) * BK * g.a_ks;
        const T* pb = B + int64_t(s) * BK * g.b_ks;
        const bool full = g.off32 && kl >= BK;
        if (full && OA::full_ok(rows_a))
            OA::load_full(pa, OA::chunk_step(g.a_ms, g.a_ks), lofa, lds_addr(sa[s]), wave);
        else
            OA::load(pa, g.a_ms, g.a_ks, rows_a, kl, sa[s], lane, wave);
        if (full && OB::full_ok(rows_b))
            OB::load_full(pb, OB::chunk_step(g.b_ns, g.b_ks), lofb, lds_addr(sb[s]), wave);
        else
            OB::load(pb, g.b_ns, g.b_ks, rows_b, kl, sb[s], lane, wave);
    }

    const typename OA::LaneOff loa = OA::lane_off(lane, wm * WM);
    const typename OB::LaneOff lob = OB::lane_off(lane, wn * WN);
    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
    for (int s = 0; s < NS; ++s) {
        // This wave's loads of slab s have landed (those of the later slabs
        // may still be in flight); after the barrier, every wave's have.
        switch (NS - 1 - s) {
#define PE_RES_WAIT(n) \
    case n: asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((n) * PER_SLAB) : "memory"); break;
            PE_RES_WAIT(0) PE_RES_WAIT(1) PE_RES_WAIT(2) PE_RES_WAIT(3)
            PE_RES_WAIT(4) PE_RES_WAIT(5) PE_RES_WAIT(6) PE_RES_WAIT(7)
#undef PE_RES_WAIT
        }
        const int k_left = g.K - s * BK;
        if (k_left < BK) {
            OA::zero_tail(sa[s], k_left, tid);
            OB::zero_tail(sb[s], k_left, tid);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        typename M::Frag fa[FM][OA::RING], fb[FN][OB::RING];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < FM; ++i) OA::frag(sa[s], loa, wm * WM, i, 0, fa[i]);
#pragma unroll
        for (int j = 0; j < FN; ++j) OB::frag(sb[s], lob, wn * WN, j, 0, fb[j]);
#pragma unroll
        for (int st = 0; st < M::STEPS; ++st) {
            if (st + 1 < M::STEPS) {
#pragma unroll
                for (int i = 0; i < FM; ++i) OA::frag(sa[s], loa, wm * WM, i, st + 1, fa[i]);
#pragma unroll
                for (int j = 0; j < FN; ++j) OB::frag(sb[s], lob, wn * WN, j, st + 1, fb[j]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = M::mfma(fa[i][st % OA::RING], fb[j][st % OB::RING], acc[i][j]);
        }
        __builtin_amdgcn_s_setprio(0);
    }

    // Epilogue, as gemm_dl_kernel's (no split).
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    const int wm0 = m0 + wm * WM, wn0 = n0 + wn * WN;
    const float* wbase = dl_uniform_base(g.c + c_off + int64_t(wm0) * g.c_ms + int64_t(wn0) * g.c_ns);
    uint32_t cms4 = uint32_t(g.c_ms) * 4u, cns4 = uint32_t(g.c_ns) * 4u, ln = uint32_t(lane);
    int rrem = g.M - wm0, crem = g.N - wn0;
    asm volatile("" : "+s"(cms4), "+s"(cns4), "+v"(ln), "+s"(rrem), "+s"(crem));
    const uint32_t lo = (ln >> 5) * 4u * cms4 + (ln & 31u) * cns4;
    const int ntm = g.store_nt;  // store flavour (nt_mode)
    if (m0 + BM <= g.M && n0 + BN <= g.N) {
        if (sizeof(T) == 2 && ntm == 2) dl_store_tile<2, false>(wbase, lo, cms4, cns4, 0, 0, acc);
        else if (ntm != 0) dl_store_tile<1, false>(wbase, lo, cms4, cns4, 0, 0, acc);
        else dl_store_tile<0, false>(wbase, lo, cms4, cns4, 0, 0, acc);
    } else {
        const int rr = rrem - 4 * int(ln >> 5), cr = crem - int(ln & 31u);
        // (partial tiles: the system-scope flavour is not instantiated)
        if (ntm != 0) dl_store_tile<1, true>(wbase, lo, cms4, cns4, rr, cr, acc);
        else dl_store_tile<0, true>(wbase, lo, cms4, cns4, rr, cr, acc);
    }
}

}  // namespace pe
