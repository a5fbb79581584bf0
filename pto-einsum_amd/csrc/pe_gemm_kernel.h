// Device side of the batched MFMA GEMM (see pe_gemm.h for the design).
#pragma once

#include "pe_gemm.h"

namespace pe {

constexpr int kGemmThreads = 256;

// Tile geometry for one instantiation.
template <typename E, int BM_, int BN_>
struct GemmGeom {
    static constexpr int BM = BM_;
    static constexpr int BN = BN_;
    static constexpr bool kF32 = E::kBytes == 4;
    static constexpr int BK = kF32 ? 16 : 32;           // k per LDS slab
    static constexpr int KSTEP = kF32 ? 2 : 16;         // k per MFMA
    static constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
    static constexpr int FM = WM / 32, FN = WN / 32;    // 32x32 blocks per wave
    static constexpr int VEC = 16 / E::kBytes;          // elements per 16-byte load
    // LDS: float32 [BK][BM + 4] (m contiguous); float16 [BM][BK + 8] (k contiguous).
    static constexpr int A_LD = kF32 ? (BM + 4) : (BK + 8);
    static constexpr int B_LD = kF32 ? (BN + 4) : (BK + 8);
    static constexpr int A_ELEMS = kF32 ? BK * A_LD : BM * A_LD;
    static constexpr int B_ELEMS = kF32 ? BK * B_LD : BN * B_LD;
    // Global loads per thread per slab (16-byte vectors or single elements).
    static constexpr int A_VECS = BM * BK / VEC / kGemmThreads;
    static constexpr int B_VECS = BN * BK / VEC / kGemmThreads;
    static_assert(A_VECS >= 1 && B_VECS >= 1, "tile too small for one vector per thread");
};

// Store one staged vector into LDS.  `row`/`col` are in the global view of the
// tile: for A, rows are m and cols are k; for B (passed transposed), rows are
// n and cols are k.  float32 LDS is k-major ([k][mn]); float16 is mn-major.
template <typename E, int LD>
__device__ __forceinline__ void lds_put(typename E::T* lds, int mn, int k, typename E::T v) {
    if constexpr (E::kBytes == 4) lds[k * LD + mn] = v;
    else lds[mn * LD + k] = v;
}

// Loader for one operand tile.  OPND 0 = A (rows m), 1 = B (rows n); the
// template LAYOUT selects the vectorisation axis.  Staged values live in
// registers between the global load and the LDS store so the load of slab
// s+1 overlaps the MFMAs of slab s.
template <typename E, int ROWS, int BK, int LD, int LAYOUT, int NV>
struct TileLoader {
    using T = typename E::T;
    static constexpr int VEC = 16 / E::kBytes;
    T stage[NV][VEC];

    // base: operand pointer already offset to (batch, row0, k0); rs/ks: row
    // and k strides; rows_left/k_left: valid extent from the tile origin.
    __device__ __forceinline__ void load(const T* __restrict__ base, int64_t rs, int64_t ks,
                                         int rows_left, int k_left, int tid) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if constexpr (LAYOUT == L_MN) {
                // Rows (m/n) contiguous: a vector spans VEC consecutive rows at one k.
                constexpr int VPR = ROWS / VEC;             // vectors per k-row
                const int idx = tid + v * kGemmThreads;
                const int k = idx / VPR;
                const int r = (idx % VPR) * VEC;
                if (k >= k_left) {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) stage[v][j] = T(0);
                } else if (r + VEC <= rows_left) {
                    const T* p = base + int64_t(k) * ks + r;
                    if constexpr (VEC == 4) {
                        f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
                        for (int j = 0; j < 4; ++j) stage[v][j] = x[j];
                    } else {
                        f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
                        for (int j = 0; j < 8; ++j) stage[v][j] = x[j];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) {
                        int rr = min(r + j, rows_left - 1);
                        stage[v][j] = base[int64_t(k) * ks + rr];
                    }
                }
            } else if constexpr (LAYOUT == L_K) {
                // k contiguous: a vector spans VEC consecutive k at one row.
                constexpr int VPK = BK / VEC;                 // vectors per row
                const int idx = tid + v * kGemmThreads;
                const int r = min(idx / VPK, rows_left - 1);
                const int k = (idx % VPK) * VEC;
                const T* p = base + int64_t(r) * rs + k;
                if (k + VEC <= k_left) {
                    if constexpr (VEC == 4) {
                        f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
                        for (int j = 0; j < 4; ++j) stage[v][j] = x[j];
                    } else {
                        f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
                        for (int j = 0; j < 8; ++j) stage[v][j] = x[j];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) stage[v][j] = (k + j < k_left) ? p[j] : T(0);
                }
            } else {
                // Generic strides: VEC single elements along k of one row.
                constexpr int VPK = BK / VEC;
                const int idx = tid + v * kGemmThreads;
                const int r = min(idx / VPK, rows_left - 1);
                const int k = (idx % VPK) * VEC;
#pragma unroll
                for (int j = 0; j < VEC; ++j)
                    stage[v][j] = (k + j < k_left) ? base[int64_t(r) * rs + int64_t(k + j) * ks] : T(0);
            }
        }
    }

    __device__ __forceinline__ void store(T* lds, int tid) const {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int idx = tid + v * kGemmThreads;
            if constexpr (LAYOUT == L_MN) {
                constexpr int VPR = ROWS / VEC;
                const int k = idx / VPR;
                const int r = (idx % VPR) * VEC;
                if constexpr (E::kBytes == 4) {
                    f32x4 x = {stage[v][0], stage[v][1], stage[v][2], stage[v][3]};
                    *reinterpret_cast<f32x4*>(lds + k * LD + r) = x;
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) lds_put<E, LD>(lds, r + j, k, stage[v][j]);
                }
            } else {
                constexpr int VPK = BK / VEC;
                const int r = idx / VPK;
                const int k = (idx % VPK) * VEC;
                if constexpr (E::kBytes == 2) {
                    f16x8 x;
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] = stage[v][j];
                    *reinterpret_cast<f16x8*>(lds + r * LD + k) = x;
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) lds_put<E, LD>(lds, r, k + j, stage[v][j]);
                }
            }
        }
    }
};

template <typename E, int BM, int BN, int ALAYOUT, int BLAYOUT>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_kernel(GemmArgs g) {
    using G = GemmGeom<E, BM, BN>;
    using T = typename E::T;
    constexpr int BK = G::BK;
    __shared__ __attribute__((aligned(16))) T lds_a[2][G::A_ELEMS];
    __shared__ __attribute__((aligned(16))) T lds_b[2][G::B_ELEMS];

    // XCD-aware block order: the dispatcher deals consecutive block ids to
    // the 8 XCDs in turn; give each XCD a contiguous run of logical tiles so
    // the tiles sharing A rows / B columns meet in the same L2.
    uint32_t bid = blockIdx.x;
    {
        const uint32_t per = g.total_blocks / 8;
        if (bid < per * 8) bid = (bid % 8) * per + bid / 8;
    }
    const uint32_t tiles_all = g.tiles_per_batch * g.nbatch_total;
    const uint32_t split = bid / tiles_all;
    uint32_t t = bid - split * tiles_all;
    uint32_t batch = t / g.tiles_per_batch;
    t -= batch * g.tiles_per_batch;
    const int tm = int(t / uint32_t(g.tiles_n));
    const int tn = int(t - uint32_t(tm) * uint32_t(g.tiles_n));

    int64_t a_off = 0, b_off = 0, c_off = 0;
    {
        uint32_t rem = batch;
        for (int d = g.nbatch - 1; d >= 0; --d) {
            uint32_t q, r;
            g.batch_div[d].divmod(rem, q, r);
            a_off += int64_t(r) * g.a_bs[d];
            b_off += int64_t(r) * g.b_bs[d];
            c_off += int64_t(r) * g.c_bs[d];
            rem = q;
        }
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int kb = int(split) * g.k_per_split;
    const int ke = min(g.K, kb + g.k_per_split);
    const int rows_a = g.M - m0, rows_b = g.N - n0;

    const T* __restrict__ A = static_cast<const T*>(g.a) + a_off + int64_t(m0) * g.a_ms + int64_t(kb) * g.a_ks;
    const T* __restrict__ B = static_cast<const T*>(g.b) + b_off + int64_t(n0) * g.b_ns + int64_t(kb) * g.b_ks;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    TileLoader<E, BM, BK, G::A_LD, ALAYOUT, G::A_VECS> la;
    TileLoader<E, BN, BK, G::B_LD, BLAYOUT, G::B_VECS> lb;

    f32x16 acc[G::FM][G::FN];
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
        for (int j = 0; j < G::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nslabs = (ke - kb + BK - 1) / BK;
    int k_left = ke - kb;
    la.load(A, g.a_ms, g.a_ks, rows_a, k_left, tid);
    lb.load(B, g.b_ns, g.b_ks, rows_b, k_left, tid);
    la.store(lds_a[0], tid);
    lb.store(lds_b[0], tid);
    __syncthreads();

    for (int s = 0; s < nslabs; ++s) {
        const int cur = s & 1;
        if (s + 1 < nslabs) {
            A += int64_t(BK) * g.a_ks;
            B += int64_t(BK) * g.b_ks;
            la.load(A, g.a_ms, g.a_ks, rows_a, k_left - BK, tid);
            lb.load(B, g.b_ns, g.b_ks, rows_b, k_left - BK, tid);
        }
        const T* sa = lds_a[cur];
        const T* sb = lds_b[cur];
#pragma unroll
        for (int kk = 0; kk < BK; kk += G::KSTEP) {
            if constexpr (G::kF32) {
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
            } else {
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
        if (s + 1 < nslabs) {
            la.store(lds_a[cur ^ 1], tid);
            lb.store(lds_b[cur ^ 1], tid);
            k_left -= BK;
        }
        __syncthreads();
    }

    // Epilogue.  32x32 accumulator layout: lane l, register r holds row
    // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of its block.
    float* __restrict__ C;
    int64_t cms, cns;
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
                if (m < g.M) store_nt(C + int64_t(m) * cms + int64_t(n) * cns, acc[i][j][r]);
            }
        }
    }
}

// Deterministic split-K reduction: C = sum over splits in ascending order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs r);

}  // namespace pe
