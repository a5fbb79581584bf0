// Float32 batched GEMM with direct global -> LDS operand loads (gfx950).
//
// Same contract and tile walk as gemm_kernel (pe_gemm_kernel.h), for the
// float32 operands whose 16-byte vectors run along M / N (L_MN) or along K
// (L_K).  What differs is how a slab reaches LDS:
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
// LDS layouts per stage (one 16-deep slab):
//   L_MN: [16][ROWS]  k-major; a chunk holds 256 / ROWS whole k rows; a
//         fragment is one 32-lane contiguous read per k.
//   L_K : [ROWS][16]  k contiguous, 16-byte groups XOR-swizzled by
//         (row / 4) % 4, so the 16 lanes of one ds_read_b64 phase (rows
//         r .. r+15 at one k) hit 16 distinct bank pairs.  A lane's load
//         fetches the global group that its swizzled slot holds.
// Both operands use the same k order inside a slab: lane half h = lane / 32
// of MFMA step st consumes k = 8 h + st.
//
// Boundaries: rows past M / N load a clamped (in-bounds) vector and only
// feed outputs that are never stored.  The K tail of a tile's last slab
// loads clamped (in-bounds) data and is then overwritten with zeros in LDS
// before any MFMA reads it, so no value from outside the operand reaches a
// stored sum.  Host-side conditions (see gemm_dl_eligible): L_MN operands
// need M (resp. N) % 4 == 0, L_K operands need K % 4 == 0 (and so every
// split's k extent), both need 16-byte aligned vectors.
#pragma once

#include "pe_gemm_kernel.h"

namespace pe {

constexpr int kDlBK = 16;

// Output stores as inline assembly as well: a compiler-issued store would be
// a tracked vector-memory operation, and the compiler then waits for the
// whole vector-memory counter (in-flight slab loads included) before
// reusing any register the store read.
__device__ __forceinline__ void dl_store(float* p, float v, bool nt) {
    if (nt) asm volatile("global_store_dword %0, %1, off nt" : : "v"(p), "v"(v));
    else asm volatile("global_store_dword %0, %1, off" : : "v"(p), "v"(v));
}

// 16 bytes per lane from global memory into LDS at lds + 16 * lane.  Written
// as inline assembly so the compiler does not treat the in-flight load as a
// pending write to every LDS array: it would otherwise wait for it before the
// first read of the other stage, serialising loads and MFMAs.  Completion is
// awaited explicitly (s_waitcnt vmcnt(0) before the barrier of the slab that
// reads it).
__device__ __forceinline__ void dma16(const float* gptr, const float* lds) {
    // The LDS address is wave-uniform (M0 takes a scalar register).
    const uint32_t l = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) float*)(lds))));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(l) : "memory", "m0");
}

// One operand's share of a slab: ROWS rows (m or n) x 16 k.  Stateless:
// per-lane offsets are recomputed from the lane index at each use, so no
// register stays live across slabs for them.
template <int ROWS, int LAYOUT>
struct DlOperand {
    static_assert(LAYOUT == L_MN || LAYOUT == L_K, "direct loads need 16-byte vectors");
    static constexpr int ELEMS = ROWS * kDlBK;   // floats per stage
    static constexpr int NCHUNK = ELEMS / 256;   // 1 KB chunks, one wave instruction each
    static constexpr int NI = NCHUNK / 4;        // instructions per wave per slab
    static_assert(NI >= 1 && NCHUNK % 4 == 0, "every wave issues whole chunks");
    static constexpr int LPR = ROWS / 4;         // L_MN: lanes per k row
    // Fragment ring: values of the current and the next MFMA step (L_MN
    // reads one k per step; L_K reads k pairs, so two pairs are held).
    static constexpr int RING = LAYOUT == L_MN ? 2 : 4;

    // Issues the slab's loads into `stage`.  base: operand at (batch, tile
    // row 0, slab k 0); rows_left / k_left: valid extent from there.
    __device__ __forceinline__ static void load(const float* base, int64_t rs, int64_t ks, int rows_left,
                                                int k_left, float* stage, int lane, int wave) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c = i * 4 + wave;
            int r, k;
            if constexpr (LAYOUT == L_MN) {
                k = min(c * (256 / ROWS) + lane / LPR, k_left - 1);
                r = min((lane % LPR) * 4, rows_left - 4);
            } else {
                r = min(c * 16 + lane / 4, rows_left - 1);
                k = min(4 * ((lane % 4) ^ (lane / 16)), k_left - 4);
            }
            dma16(base + int64_t(r) * rs + int64_t(k) * ks, stage + c * 256);
        }
    }

    // Zeroes every k >= k_left of a stage (0 < k_left < 16).
    __device__ __forceinline__ static void zero_tail(float* stage, int k_left, int tid) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (LAYOUT == L_MN) {
            const int n = (kDlBK - k_left) * LPR;
            for (int idx = tid; idx < n; idx += kGemmThreads) {
                const int k = k_left + idx / LPR, c = (idx % LPR) * 4;
                *reinterpret_cast<f32x4*>(stage + k * ROWS + c) = z;
            }
        } else {
            for (int idx = tid; idx < ROWS * 4; idx += kGemmThreads) {
                const int r = idx / 4, pc = idx % 4;
                const int lc = pc ^ ((r >> 2) & 3);
                if (4 * lc >= k_left) *reinterpret_cast<f32x4*>(stage + r * 16 + pc * 4) = z;
            }
        }
    }

    // Per-lane fragment offsets (floats from the stage origin) for a wave
    // whose fragment rows start at wrow0: L_MN needs one, L_K one per half
    // slab (the swizzled group of k = 8 h + 4 q differs per lane).
    struct LaneOff {
        int o[2];
    };
    __device__ __forceinline__ static LaneOff lane_off(int lane, int wrow0) {
        const int h = lane >> 5, r = wrow0 + (lane & 31);
        LaneOff x;
        if constexpr (LAYOUT == L_MN) {
            x.o[0] = 8 * h * ROWS + r;
            x.o[1] = 0;
        } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) x.o[q] = r * 16 + (((2 * h + q) ^ ((r >> 2) & 3)) * 4);
        }
        return x;
    }

    // Reads what MFMA step st needs (lane half h consumes k = 8 h + st) for
    // fragment block i (rows 32 i .. 32 i + 31 of the wave) into ring slot
    // st % RING; L_K reads k pairs, at even steps only (slots st % 4 and
    // (st + 1) % 4).  All offsets but the lane's are compile-time constants.
    __device__ __forceinline__ static void frag(const float* stage, const LaneOff& lo, int i, int st,
                                                float (&v)[RING]) {
        if constexpr (LAYOUT == L_MN) {
            v[st % 2] = stage[lo.o[0] + st * ROWS + i * 32];
        } else if (st % 2 == 0) {
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            const f32x2 x = *reinterpret_cast<const f32x2*>(stage + lo.o[st / 4] + i * 32 * 16 + st % 4);
            v[st % 4] = x[0];
            v[(st + 1) % 4] = x[1];
        }
    }
};

// MINB: resident blocks per CU the register allocation is held to (four
// waves per block, one per SIMD, so MINB waves per SIMD).
template <int BM, int BN, int AL, int BL, int MINB>
__global__ __launch_bounds__(kGemmThreads, MINB) void gemm_dl_kernel(GemmArgs g) {
    using OA = DlOperand<BM, AL>;
    using OB = DlOperand<BN, BL>;
    constexpr int BK = kDlBK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    __shared__ __attribute__((aligned(16))) float sa0[OA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sa1[OA::ELEMS];
    __shared__ __attribute__((aligned(16))) float sb0[OB::ELEMS];
    __shared__ __attribute__((aligned(16))) float sb1[OB::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5;
    const uint32_t tiles_all = g.tiles_per_batch * g.nbatch_total;

    struct Tile {
        const float* A;
        const float* B;
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
        x.A = static_cast<const float*>(g.a) + a_off + int64_t(x.m0) * g.a_ms + int64_t(kb) * g.a_ks;
        x.B = static_cast<const float*>(g.b) + b_off + int64_t(x.n0) * g.b_ns + int64_t(kb) * g.b_ks;
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

    auto issue = [&](float* da, float* db) {
        const int kl = lt.k_len - ls * BK;
        OA::load(lt.A + int64_t(ls) * BK * g.a_ks, g.a_ms, g.a_ks, lt.rows_a, kl, da, lane, wave);
        OB::load(lt.B + int64_t(ls) * BK * g.b_ks, g.b_ns, g.b_ks, lt.rows_b, kl, db, lane, wave);
        if (++ls == lt.nslabs) {
            lbid += walk.step;
            lvalid = lbid < walk.end;
            if (lvalid) {
                lt = locate(lbid);
                ls = 0;
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
        const bool nt = g.store_nt != 0;
        if (g.nsplit > 1) {
            C = g.partial + ((int64_t(ct.split) * g.nbatch_total + ct.batch) * g.M) * int64_t(g.N);
            cms = g.N;
            cns = 1;
        } else {
            C = g.c + ct.c_off;
            cms = g.c_ms;
            cns = g.c_ns;
        }
        // 32x32 accumulator layout: lane l, register r holds row
        // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of its block.
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int n = ct.n0 + wn * WN + j * 32 + (lane & 31);
                if (n < g.N) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = ct.m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (m < g.M) dl_store(C + int64_t(m) * cms + int64_t(n) * cns, acc[i][j][r], nt);
                    }
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
            }
        }
    };

    // One slab: wait for its loads, start the next slab's loads into the
    // other stage, then the MFMAs.  Returns true when the block is done.
    auto step = [&](const float* sa, const float* sb, float* na, float* nb) -> bool {
        // This wave's loads of the slab have landed; after the barrier every
        // wave's have, and every wave is done reading the other stage.
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (lvalid) issue(na, nb);
        const int k_left = ct.k_len - cs * BK;
        if (k_left < BK) {
            OA::zero_tail(const_cast<float*>(sa), k_left, tid);
            OB::zero_tail(const_cast<float*>(sb), k_left, tid);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        float fa[FM][OA::RING], fb[FN][OB::RING];
#pragma unroll
        for (int i = 0; i < FM; ++i) OA::frag(sa, loa, i, 0, fa[i]);
#pragma unroll
        for (int j = 0; j < FN; ++j) OB::frag(sb, lob, j, 0, fb[j]);
#pragma unroll
        for (int st = 0; st < BK / 2; ++st) {
            if (st + 1 < BK / 2) {
#pragma unroll
                for (int i = 0; i < FM; ++i) OA::frag(sa, loa, i, st + 1, fa[i]);
#pragma unroll
                for (int j = 0; j < FN; ++j) OB::frag(sb, lob, j, st + 1, fb[j]);
            }
            // Keep the next step's reads ahead of this step's MFMAs (the
            // scheduler would otherwise sink them to save registers and wait
            // on each read in turn).
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][st % OA::RING], fb[j][st % OB::RING],
                                                                     acc[i][j], 0, 0, 0);
        }
        if (++cs == ct.nslabs) {
            epilogue();
            cbid += walk.step;
            if (cbid >= walk.end) return true;
            ct = locate(cbid);
            cs = 0;
        }
        return false;
    };

    issue(sa0, sb0);
    for (;;) {
        if (step(sa0, sb0, sa1, sb1)) break;
        if (step(sa1, sb1, sa0, sb0)) break;
    }
}

}  // namespace pe
