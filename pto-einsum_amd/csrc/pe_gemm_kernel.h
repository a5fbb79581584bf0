// Device side of the batched MFMA GEMM (see pe_gemm.h for the design).
#pragma once

#include "pe_gemm.h"

namespace pe {

constexpr int kGemmThreads = 256;

// Tile geometry for one instantiation.
//   KC = true : LDS rows are m (A) / n (B) with k contiguous, [rows][BK + pad];
//               each lane's MFMA fragments for a whole slab are 16-byte reads.
//   KC = false: LDS rows are k, [BK][rows + 4]; each float32 fragment is one
//               32-lane contiguous read (float32 only).
// The k padding makes a 16-lane group of 16-byte reads at one column hit
// 16 distinct 4-bank groups (row stride = 4 mod 64 words).
template <typename E, int BM_, int BN_, int BK_, bool KC_, int NBUF_ = 2>
struct GemmGeom {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr bool KC = KC_;
    static constexpr int NBUF = NBUF_;  // LDS stages: 2 = double buffer, 1 = single
    static constexpr bool kF32 = E::kBytes == 4;
    static_assert(kF32 || KC, "float16 operands are always staged k-contiguous");
    static constexpr int KSTEP = kF32 ? 2 : 16;          // k per MFMA
    static constexpr int WM = BM / 2, WN = BN / 2;       // wave tile (2x2 waves)
    static constexpr int FM = WM / 32, FN = WN / 32;     // 32x32 blocks per wave
    static constexpr int VEC = 16 / E::kBytes;           // elements per 16-byte load
    static constexpr int KPAD = 16 / E::kBytes;          // one 16-byte group
    static constexpr int A_LD = KC ? BK + KPAD : BM + 4;
    static constexpr int B_LD = KC ? BK + KPAD : BN + 4;
    static constexpr int A_ELEMS = KC ? BM * A_LD : BK * A_LD;
    static constexpr int B_ELEMS = KC ? BN * B_LD : BK * B_LD;
    static constexpr int A_VECS = BM * BK / VEC / kGemmThreads;
    static constexpr int B_VECS = BN * BK / VEC / kGemmThreads;
    static constexpr int LDS_BYTES = NBUF * (A_ELEMS + B_ELEMS) * E::kBytes;
    static_assert(A_VECS >= 1 && B_VECS >= 1, "tile too small for one vector per thread");
    static_assert(BK % (2 * KSTEP) == 0 || !kF32, "float32 slab splits evenly over the two lane groups");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget per block (gfx950: 160 KB per CU)");
};

template <int N, typename T>
struct Pack;
template <typename T>
struct Pack<1, T> { using type = T; };
template <>
struct Pack<2, float> { typedef float type __attribute__((ext_vector_type(2))); };
template <>
struct Pack<4, float> { typedef float type __attribute__((ext_vector_type(4))); };
template <>
struct Pack<2, _Float16> { typedef _Float16 type __attribute__((ext_vector_type(2))); };
template <>
struct Pack<4, _Float16> { typedef _Float16 type __attribute__((ext_vector_type(4))); };
template <>
struct Pack<8, _Float16> { typedef _Float16 type __attribute__((ext_vector_type(8))); };

// Loader for one operand tile (OPND rows = m for A, n for B).  Staged values
// live in registers between the global load and the LDS store, so the load of
// slab s+1 is in flight while slab s feeds the MFMAs.
//   L_MN:      a thread loads NV vectors of VEC consecutive rows at NV
//              consecutive k (one row chunk), so a k-contiguous LDS store
//              packs NV values per row;
//   L_K:       a thread loads vectors of VEC consecutive k at one row;
//   L_GENERIC: as L_K with element loads at arbitrary strides.
template <typename E, int ROWS, int BK, int LD, bool KC, int LAYOUT, int NV>
struct TileLoader {
    using T = typename E::T;
    static constexpr int VEC = 16 / E::kBytes;
    // L_MN: whole row chunks per thread when the threads split evenly over
    // the vectors of one k row; else a strided vector walk (k-major LDS only).
    static constexpr bool kRowChunks = kGemmThreads % (ROWS / VEC) == 0;
    static_assert(LAYOUT != L_MN || kRowChunks || !KC, "strided L_MN walk needs k-major LDS");
    T stage[NV][VEC];

    __device__ __forceinline__ static void vload(const T* p, T (&d)[VEC]) {
        using V = typename Pack<VEC, T>::type;
        V x = *reinterpret_cast<const V*>(p);
#pragma unroll
        for (int j = 0; j < VEC; ++j) d[j] = x[j];
    }

    // base: operand at (batch, row0, k0); rs/ks: row and k strides;
    // rows_left/k_left: valid extent from the tile origin.
    __device__ __forceinline__ void load(const T* __restrict__ base, int64_t rs, int64_t ks,
                                         int rows_left, int k_left, int tid) {
        if constexpr (LAYOUT == L_MN && !kRowChunks) {
            // Rows that do not divide the block: vector idx = tid + v*threads
            // covers (k = idx / VPR, rows (idx % VPR)*VEC ..).
            constexpr int VPR = ROWS / VEC;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int idx = tid + v * kGemmThreads;
                const int k = idx / VPR, r = (idx % VPR) * VEC;
                if (k >= k_left) {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) stage[v][j] = T(0);
                } else if (r + VEC <= rows_left) {
                    vload(base + int64_t(k) * ks + r, stage[v]);
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j)
                        stage[v][j] = base[int64_t(k) * ks + min(r + j, rows_left - 1)];
                }
            }
        } else if constexpr (LAYOUT == L_MN) {
            constexpr int VPR = ROWS / VEC;
            const int r = (tid % VPR) * VEC;
            const int k0 = (tid / VPR) * NV;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int k = k0 + v;
                if (k >= k_left) {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) stage[v][j] = T(0);
                } else if (r + VEC <= rows_left) {
                    vload(base + int64_t(k) * ks + r, stage[v]);
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j)
                        stage[v][j] = base[int64_t(k) * ks + min(r + j, rows_left - 1)];
                }
            }
        } else {
            constexpr int VPK = BK / VEC;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int idx = tid + v * kGemmThreads;
                const int r = min(idx / VPK, rows_left - 1);
                const int k = (idx % VPK) * VEC;
                if constexpr (LAYOUT == L_K) {
                    const T* p = base + int64_t(r) * rs + k;
                    if (k + VEC <= k_left) {
                        vload(p, stage[v]);
                    } else {
#pragma unroll
                        for (int j = 0; j < VEC; ++j) stage[v][j] = (k + j < k_left) ? p[j] : T(0);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j)
                        stage[v][j] = (k + j < k_left) ? base[int64_t(r) * rs + int64_t(k + j) * ks] : T(0);
                }
            }
        }
    }

    __device__ __forceinline__ void store(T* lds, int tid) const {
        if constexpr (LAYOUT == L_MN && !kRowChunks) {
            constexpr int VPR = ROWS / VEC;
            using V = typename Pack<VEC, T>::type;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int idx = tid + v * kGemmThreads;
                const int k = idx / VPR, r = (idx % VPR) * VEC;
                V x;
#pragma unroll
                for (int j = 0; j < VEC; ++j) x[j] = stage[v][j];
                *reinterpret_cast<V*>(lds + k * LD + r) = x;
            }
        } else if constexpr (LAYOUT == L_MN) {
            constexpr int VPR = ROWS / VEC;
            const int r = (tid % VPR) * VEC;
            const int k0 = (tid / VPR) * NV;
            if constexpr (KC) {
                // Row r+j receives NV consecutive k values.
                using P = typename Pack<NV, T>::type;
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    P x;
                    if constexpr (NV == 1) {
                        x = stage[0][j];
                    } else {
#pragma unroll
                        for (int v = 0; v < NV; ++v) x[v] = stage[v][j];
                    }
                    *reinterpret_cast<P*>(lds + (r + j) * LD + k0) = x;
                }
            } else {
                using V = typename Pack<VEC, T>::type;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    V x;
#pragma unroll
                    for (int j = 0; j < VEC; ++j) x[j] = stage[v][j];
                    *reinterpret_cast<V*>(lds + (k0 + v) * LD + r) = x;
                }
            }
        } else {
            constexpr int VPK = BK / VEC;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int idx = tid + v * kGemmThreads;
                const int r = idx / VPK;
                const int k = (idx % VPK) * VEC;
                if constexpr (KC) {
                    using V = typename Pack<VEC, T>::type;
                    V x;
#pragma unroll
                    for (int j = 0; j < VEC; ++j) x[j] = stage[v][j];
                    *reinterpret_cast<V*>(lds + r * LD + k) = x;
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) lds[(k + j) * LD + r] = stage[v][j];
                }
            }
        }
    }
};

// Maps the block's n-th tile to (split, batch, tm, tn).  Blocks are dealt to
// the 8 XCDs round-robin by block id, so XCD x = blockIdx % 8 runs
// q + (x < r) of the G blocks (q = G / 8, r = G % 8) and is given a
// contiguous logical range of the T tiles in proportion -- tiles that share A
// rows and B columns then meet in the same L2, and with one block per tile
// every block gets exactly one (equal ranges of T / 8 had left some blocks
// two tiles and others none whenever G was not a multiple of 8: twice the
// time for, e.g., 540 blocks).  With fewer than 8 blocks, a plain
// grid-stride order is used.  Every logical tile is visited exactly once
// whatever XCD actually runs the block.
#ifndef PE_GEMM_XCD_WALK
#define PE_GEMM_XCD_WALK 1
#endif
struct TileWalk {
    uint32_t next, end, step;
    __device__ __forceinline__ TileWalk(uint32_t total) {
        const uint32_t G = gridDim.x, b = blockIdx.x;
        if (G < 8 || !PE_GEMM_XCD_WALK) {
            next = b; end = total; step = G;
        } else {
            const uint32_t x = b % 8, j = b / 8, q = G / 8, r = G % 8;
            // first tile of XCD y: its share of T after the blocks of XCDs 0 .. y-1
            auto first = [&](uint32_t y) {
                return uint32_t(uint64_t(total) * (uint64_t(y) * q + (y < r ? y : r)) / G);
            };
            next = first(x) + j; end = first(x + 1); step = q + (x < r ? 1u : 0u);
        }
    }
};

// Fragment schedule for float32 k-major slabs: 0 = read each k-step's
// fragments just before its MFMAs (few registers, high occupancy);
// 1 = read the whole slab first (more registers, one wait per slab).
// -1 picks per tile: whole-slab reads for the 256x128 / 128x256 tiles, whose
// accumulators already bound occupancy to two waves per SIMD.
#ifndef PE_GEMM_PRELOAD
#define PE_GEMM_PRELOAD -1
#endif
#ifndef PE_GEMM_PRELOAD_MIN
#define PE_GEMM_PRELOAD_MIN (256 * 128)
#endif


template <typename E, int BM, int BN, int BK, bool KC, int NBUF, int ALAYOUT, int BLAYOUT>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_kernel(GemmArgs g) {
    using G = GemmGeom<E, BM, BN, BK, KC, NBUF>;
    using T = typename E::T;
    constexpr int PRELOAD = PE_GEMM_PRELOAD >= 0 ? PE_GEMM_PRELOAD : (BM * BN >= PE_GEMM_PRELOAD_MIN ? 1 : 0);
    __shared__ __attribute__((aligned(16))) T lds_a[NBUF][G::A_ELEMS];
    __shared__ __attribute__((aligned(16))) T lds_b[NBUF][G::B_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t tiles_all = g.tiles_per_batch * g.nbatch_total;

    // Operand origins and extents of one tile (split, batch, tm, tn).
    struct Tile {
        const T* A;
        const T* B;
        int64_t c_off;
        uint32_t split, batch;
        int m0, n0, rows_a, rows_b, k_len;
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
        x.rows_a = g.M - x.m0;
        x.rows_b = g.N - x.n0;
        x.A = static_cast<const T*>(g.a) + a_off + int64_t(x.m0) * g.a_ms + int64_t(kb) * g.a_ks;
        x.B = static_cast<const T*>(g.b) + b_off + int64_t(x.n0) * g.b_ns + int64_t(kb) * g.b_ks;
        x.c_off = c_off;
        return x;
    };

    TileLoader<E, BM, BK, G::A_LD, KC, ALAYOUT, G::A_VECS> la;
    TileLoader<E, BN, BK, G::B_LD, KC, BLAYOUT, G::B_VECS> lb;

    TileWalk walk(g.total_blocks);
    uint32_t bid = walk.next;
    if (bid >= walk.end) return;
    Tile cur_t = locate(bid);
    la.load(cur_t.A, g.a_ms, g.a_ks, cur_t.rows_a, cur_t.k_len, tid);
    lb.load(cur_t.B, g.b_ns, g.b_ks, cur_t.rows_b, cur_t.k_len, tid);
    for (;;) {
        const T* __restrict__ A = cur_t.A;
        const T* __restrict__ B = cur_t.B;
        const int m0 = cur_t.m0, n0 = cur_t.n0;
        const int rows_a = cur_t.rows_a, rows_b = cur_t.rows_b;
        const uint32_t split = cur_t.split, batch = cur_t.batch;
        const int64_t c_off = cur_t.c_off;

        f32x16 acc[G::FM][G::FN];
#pragma unroll
        for (int i = 0; i < G::FM; ++i)
#pragma unroll
            for (int j = 0; j < G::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

        const int nslabs = (cur_t.k_len + BK - 1) / BK;
        int k_left = cur_t.k_len;
        la.store(lds_a[0], tid);
        lb.store(lds_b[0], tid);
        __syncthreads();

        for (int s = 0; s < nslabs; ++s) {
            const int cur = NBUF == 2 ? (s & 1) : 0;
            if (s + 1 < nslabs) {
                A += int64_t(BK) * g.a_ks;
                B += int64_t(BK) * g.b_ks;
                la.load(A, g.a_ms, g.a_ks, rows_a, k_left - BK, tid);
                lb.load(B, g.b_ns, g.b_ks, rows_b, k_left - BK, tid);
            }
            const T* sa = lds_a[cur];
            const T* sb = lds_b[cur];
            if constexpr (G::kF32 && !KC && PRELOAD) {
                // All of the slab's fragments first (distinct registers), so the
                // LDS latency is paid once per slab rather than once per k-step.
                constexpr int H = BK / 2;
                float fa[H][G::FM], fb[H][G::FN];
#pragma unroll
                for (int st = 0; st < H; ++st) {
                    const int kr = 2 * st + (lane >> 5);
#pragma unroll
                    for (int i = 0; i < G::FM; ++i) fa[st][i] = sa[kr * G::A_LD + wm * G::WM + i * 32 + (lane & 31)];
#pragma unroll
                    for (int j = 0; j < G::FN; ++j) fb[st][j] = sb[kr * G::B_LD + wn * G::WN + j * 32 + (lane & 31)];
                }
                // Keep every read ahead of the MFMAs: the scheduler would
                // otherwise reuse one register pair per step and wait on
                // each read in turn.
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int st = 0; st < H; ++st)
#pragma unroll
                    for (int i = 0; i < G::FM; ++i)
#pragma unroll
                        for (int j = 0; j < G::FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[st][i], fb[st][j], acc[i][j], 0, 0, 0);
            } else if constexpr (G::kF32 && !KC) {
#pragma unroll
                for (int kk = 0; kk < BK; kk += 2) {
                    float fa[G::FM], fb[G::FN];
                    const int kr = kk + (lane >> 5);
#pragma unroll
                    for (int i = 0; i < G::FM; ++i) fa[i] = sa[kr * G::A_LD + wm * G::WM + i * 32 + (lane & 31)];
#pragma unroll
                    for (int j = 0; j < G::FN; ++j) fb[j] = sb[kr * G::B_LD + wn * G::WN + j * 32 + (lane & 31)];
#pragma unroll
                    for (int i = 0; i < G::FM; ++i)
#pragma unroll
                        for (int j = 0; j < G::FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            } else if constexpr (G::kF32) {
                // Lane group g = lane/32 owns k in [g*BK/2, (g+1)*BK/2); step s
                // feeds k = g*BK/2 + s from both operands.
                constexpr int H = BK / 2;
                float fa[G::FM][H], fb[G::FN][H];
                const int kc = (lane >> 5) * H;
#pragma unroll
                for (int i = 0; i < G::FM; ++i) {
                    const float* p = sa + (wm * G::WM + i * 32 + (lane & 31)) * G::A_LD + kc;
#pragma unroll
                    for (int q = 0; q < H; q += 4) {
                        f32x4 x = *reinterpret_cast<const f32x4*>(p + q);
                        fa[i][q] = x[0]; fa[i][q + 1] = x[1]; fa[i][q + 2] = x[2]; fa[i][q + 3] = x[3];
                    }
                }
#pragma unroll
                for (int j = 0; j < G::FN; ++j) {
                    const float* p = sb + (wn * G::WN + j * 32 + (lane & 31)) * G::B_LD + kc;
#pragma unroll
                    for (int q = 0; q < H; q += 4) {
                        f32x4 x = *reinterpret_cast<const f32x4*>(p + q);
                        fb[j][q] = x[0]; fb[j][q + 1] = x[1]; fb[j][q + 2] = x[2]; fb[j][q + 3] = x[3];
                    }
                }
#pragma unroll
                for (int s2 = 0; s2 < H; ++s2)
#pragma unroll
                    for (int i = 0; i < G::FM; ++i)
#pragma unroll
                        for (int j = 0; j < G::FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s2], fb[j][s2], acc[i][j], 0, 0, 0);
            } else {
#pragma unroll
                for (int kk = 0; kk < BK; kk += 16) {
                    f16x8 fa[G::FM], fb[G::FN];
                    const int kc = kk + 8 * (lane >> 5);
#pragma unroll
                    for (int i = 0; i < G::FM; ++i)
                        fa[i] = *reinterpret_cast<const f16x8*>(sa + (wm * G::WM + i * 32 + (lane & 31)) * G::A_LD + kc);
#pragma unroll
                    for (int j = 0; j < G::FN; ++j)
                        fb[j] = *reinterpret_cast<const f16x8*>(sb + (wn * G::WN + j * 32 + (lane & 31)) * G::B_LD + kc);
#pragma unroll
                    for (int i = 0; i < G::FM; ++i)
#pragma unroll
                        for (int j = 0; j < G::FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
            if constexpr (NBUF == 1) __syncthreads();  // every wave is done reading the stage
            if (s + 1 < nslabs) {
                la.store(lds_a[NBUF == 2 ? (cur ^ 1) : 0], tid);
                lb.store(lds_b[NBUF == 2 ? (cur ^ 1) : 0], tid);
                k_left -= BK;
            }
            __syncthreads();
        }

        // Epilogue.  32x32 accumulator layout: lane l, register r holds row
        // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of its block.
        float* __restrict__ C;
        int64_t cms, cns;
        const int nt = g.store_nt;  // store flavour (nt_mode)
        if (g.nsplit > 1) {
            C = g.partial + ((int64_t(split) * g.nbatch_total + batch) * g.M) * int64_t(g.N);
            cms = g.N;
            cns = 1;
        } else {
            C = g.c + c_off;
            cms = g.c_ms;
            cns = g.c_ns;
        }
#pragma unroll
        for (int i = 0; i < G::FM; ++i) {
#pragma unroll
            for (int j = 0; j < G::FN; ++j) {
                const int n = n0 + wn * G::WN + j * 32 + (lane & 31);
                if (n >= g.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * G::WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < g.M) store_f(C + int64_t(m) * cms + int64_t(n) * cns, acc[i][j][r], nt);
                }
            }
        }
        // Next tile of a persistent block.  (Loading its first slab before
        // this epilogue instead measured slower: the extra live registers
        // cost a resident block per CU.)
        bid += walk.step;
        if (bid >= walk.end) break;
        cur_t = locate(bid);
        la.load(cur_t.A, g.a_ms, g.a_ks, cur_t.rows_a, cur_t.k_len, tid);
        lb.load(cur_t.B, g.b_ns, g.b_ks, cur_t.rows_b, cur_t.k_len, tid);
    }
}

}  // namespace pe
