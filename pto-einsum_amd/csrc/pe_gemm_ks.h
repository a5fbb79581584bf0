// Batched GEMM whose four waves split every slab's k four ways (gfx950):
// one block per small output tile, no K split across blocks.
//
// Grids with fewer 128 x 128 tiles than CUs split K over blocks, and a
// second kernel sums the split partials in order (pe_gemm.hip).  Where K is
// short (<= 1024) that costs a second launch and a round trip of the
// partials for a few microseconds of MFMA work; unsplit grids of one 64 x 64
// tile per CU leave one wave per SIMD walking all of K.  Here the tiles are
// 32 x 32 (or 64 x 64 where those still give each CU about one), and each
// block's four waves walk K together: a stage holds
// 4 x SPW sub-slabs, each laid out exactly as a direct-load kernel's slab
// (pe_gemm_dl.h: 64 bytes of k per row, the same swizzles and fragment
// reads); wave w accumulates the whole tile over sub-slabs q * 4 + w of every
// stage, into ILP accumulator sets taken in turn by the MFMA steps (so that
// consecutive MFMAs do not wait for one another).  At the end each wave adds
// its sets in order, the four waves' sums meet in LDS and are added in wave
// order, ((w0 + w1) + w2) + w3, each wave adding and storing a quarter of the
// tile.  The sum is deterministic; it groups the k terms differently from the
// split-K path (float32 rounding only).
//
// Loads: global_load_lds_dwordx4 through an NS-stage ring, NS - 1 stages in
// flight ahead of the one the MFMAs read.  A full stage's loads are spread
// over the MFMA steps of the stage before (per-lane addresses computed once);
// the last, partial stage's are clamped in-bounds and its k tail zeroed in
// LDS afterwards, as in the direct-load kernel.  Every wave issues the same
// number of loads per stage and loads complete in issue order, so s_waitcnt
// vmcnt(ahead x loads per stage) waits for exactly the stage about to be read.
// Measured on MI355X: float32 faster than the split-K path up to K = 1024
// (256^3 7.4 -> 4.9 us, 512^2 x 1024 15.5 -> 10.8), no faster beyond (512^2 x
// 4096 34.6 against 34.5, 1024 x 128 x 2048 16.9 against 18.7); float16 64 x
// 64 tiles faster up to K = 8192 where they fill the CUs (1024^3 19.9 -> 9.6
// us); the grids it takes are chosen in pe_gemm.hip.
#pragma once

#include "pe_gemm_dl.h"

namespace pe {

template <typename E, int BM, int BN, int AL, int BL, int NS, int SPW>
struct KsGeom {
    using T = typename E::T;
    using M = DlMath<E>;
    using OA = DlOperand<E, BM, AL, true>;
    using OB = DlOperand<E, BN, BL, true>;
    static constexpr int BK = M::BK;                 // k per sub-slab
    static constexpr int NSUB = 4 * SPW;             // sub-slabs per stage, SPW per wave
    static constexpr int SK = NSUB * BK;             // k per stage
    static constexpr int FM = BM / 32, FN = BN / 32;
    static constexpr int A_STAGE = NSUB * OA::ELEMS; // elements per stage
    static constexpr int B_STAGE = NSUB * OB::ELEMS;
    static constexpr int STAGE_BYTES = (A_STAGE + B_STAGE) * E::kBytes;
    static constexpr int LA = SPW * OA::NCHUNK;      // loads per wave per stage
    static constexpr int LB = SPW * OB::NCHUNK;
    static constexpr int LOADS = LA + LB;
    // Wave partial sums at the end: 4 waves x FM x FN blocks x 16 registers x 64 lanes.
    static constexpr int RED_BYTES = 4 * FM * FN * 16 * 64 * 4;
    static constexpr int LDS_BYTES = NS * STAGE_BYTES > RED_BYTES ? NS * STAGE_BYTES : RED_BYTES;
    static_assert(BM % 32 == 0 && BN % 32 == 0, "32 x 32 MFMA blocks");
    static_assert(NS >= 2 && NS <= 4, "ring depth");
    static_assert(LOADS * (NS - 2) <= 63, "vmcnt immediate");
    static_assert((FM * FN * 16) % 4 == 0, "each wave sums a quarter of the tile");
};

template <int N>
__device__ __forceinline__ void ks_wait_barrier() {
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <typename E, int BM, int BN, int AL, int BL, int NS, int SPW, int ILP>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_ks_kernel(GemmArgs g) {
    using G = KsGeom<E, BM, BN, AL, BL, NS, SPW>;
    using T = typename E::T;
    using M = typename G::M;
    using OA = typename G::OA;
    using OB = typename G::OB;
    constexpr int BK = G::BK, SK = G::SK, FM = G::FM, FN = G::FN;
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::LDS_BYTES];
    T* const ring = reinterpret_cast<T*>(lds);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Tile of this block (no K split: one block per tile and batch).
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
    const int rows_a = g.M - m0, rows_b = g.N - n0;
    const int K = g.K;
    const int nst = (K + SK - 1) / SK;
    const T* const A = static_cast<const T*>(g.a) + a_off + int64_t(m0) * g.a_ms;
    const T* const B = static_cast<const T*>(g.b) + b_off + int64_t(n0) * g.b_ns;

    auto a_stage = [&](int s) { return ring + (s % NS) * (G::A_STAGE + G::B_STAGE); };
    auto b_stage = [&](int s) { return a_stage(s) + G::A_STAGE; };

    // Per-lane addresses of this wave's chunks of stage 0 (chunk i * 4 +
    // wave of the stage's 4 x NCHUNK: sub-slab j, chunk c of it); a full
    // stage s reads them s * SK k further on.
    const T* pa[G::LA];
    const T* pb[G::LB];
#pragma unroll
    for (int i = 0; i < G::LA; ++i) {
        const int cc = i * 4 + wave, j = cc / OA::NCHUNK, c = cc % OA::NCHUNK;
        int r, k;
        OA::chunk_rk(lane, c, rows_a, BK, r, k);
        pa[i] = A + int64_t(r) * g.a_ms + int64_t(j * BK + k) * g.a_ks;
    }
#pragma unroll
    for (int i = 0; i < G::LB; ++i) {
        const int cc = i * 4 + wave, j = cc / OB::NCHUNK, c = cc % OB::NCHUNK;
        int r, k;
        OB::chunk_rk(lane, c, rows_b, BK, r, k);
        pb[i] = B + int64_t(r) * g.b_ns + int64_t(j * BK + k) * g.b_ks;
    }

    // Stage s's loads, LA + LB per wave.  In the last, partial stage a
    // sub-slab past K loads the first sub-slab's (in-bounds) data instead;
    // it is zeroed before use.
    auto issue = [&](int s) {
        T* sa = a_stage(s);
        T* sb = b_stage(s);
        if ((s + 1) * SK <= K) {
            const int64_t ka = int64_t(s) * SK * g.a_ks, kb = int64_t(s) * SK * g.b_ks;
#pragma unroll
            for (int i = 0; i < G::LA; ++i) {
                const int cc = i * 4 + wave;
                dma16(reinterpret_cast<const float*>(pa[i] + ka),
                      reinterpret_cast<const float*>(sa + cc * (1024 / E::kBytes)));
            }
#pragma unroll
            for (int i = 0; i < G::LB; ++i) {
                const int cc = i * 4 + wave;
                dma16(reinterpret_cast<const float*>(pb[i] + kb),
                      reinterpret_cast<const float*>(sb + cc * (1024 / E::kBytes)));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < G::LA; ++i) {
            const int cc = i * 4 + wave, j = cc / OA::NCHUNK, c = cc % OA::NCHUNK;
            int k0 = s * SK + j * BK;
            if (k0 >= K) k0 = 0;
            OA::load_chunk(A + int64_t(k0) * g.a_ks, g.a_ms, g.a_ks, rows_a, min(K - k0, BK),
                           sa + j * OA::ELEMS, lane, c);
        }
#pragma unroll
        for (int i = 0; i < G::LB; ++i) {
            const int cc = i * 4 + wave, j = cc / OB::NCHUNK, c = cc % OB::NCHUNK;
            int k0 = s * SK + j * BK;
            if (k0 >= K) k0 = 0;
            OB::load_chunk(B + int64_t(k0) * g.b_ks, g.b_ns, g.b_ks, rows_b, min(K - k0, BK),
                           sb + j * OB::ELEMS, lane, c);
        }
    };

    // NSET independent accumulator sets: set q * ILP + st % ILP takes the
    // wave's q-th sub-slab of a stage at MFMA step st.
    constexpr int NSET = SPW * ILP;
    f32x16 acc[NSET][FM][FN];
#pragma unroll
    for (int q = 0; q < NSET; ++q)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[q][i][j][r] = 0.0f;

    const typename OA::LaneOff loa = OA::lane_off(lane, 0);
    const typename OB::LaneOff lob = OB::lane_off(lane, 0);

#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < nst) issue(p);

    for (int s = 0; s < nst; ++s) {
        // Stages issued after s: min(nst - 1, s + NS - 2) - s.
        const int ahead = min(nst - 1, s + NS - 2) - s;
        if (NS >= 4 && ahead >= 2) ks_wait_barrier<G::LOADS * 2 * (NS >= 4)>();
        else if (NS >= 3 && ahead >= 1) ks_wait_barrier<G::LOADS * (NS >= 3)>();
        else ks_wait_barrier<0>();
        // Every wave is past stage s - 1's reads: its slot takes stage
        // s + NS - 1.  A full stage's loads are spread over this stage's
        // MFMA steps (issued all at once they queue behind one another in
        // the address unit, and the wave issues no MFMA meanwhile); a
        // partial last stage's are issued here.
        const int ls = s + NS - 1;
        const bool spread = ls < nst && (ls + 1) * SK <= K;
        if (ls < nst && !spread) issue(ls);
        const int64_t lka = int64_t(ls) * SK * g.a_ks, lkb = int64_t(ls) * SK * g.b_ks;
        T* const lsa = a_stage(ls);
        T* const lsb = b_stage(ls);
        const int k_left = K - s * SK;
        if (k_left < SK) {
#pragma unroll
            for (int j = 0; j < G::NSUB; ++j) {
                const int kl = k_left - j * BK;
                if (kl < BK) {
                    OA::zero_tail(a_stage(s) + j * OA::ELEMS, max(kl, 0), tid);
                    OB::zero_tail(b_stage(s) + j * OB::ELEMS, max(kl, 0), tid);
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int q = 0; q < SPW; ++q) {
            // Sub-slab q * 4 + wave: the four waves read consecutive k runs.
            const T* sa = a_stage(s) + (q * 4 + wave) * OA::ELEMS;
            const T* sb = b_stage(s) + (q * 4 + wave) * OB::ELEMS;
            typename M::Frag fa[FM][OA::RING], fb[FN][OB::RING];
#pragma unroll
            for (int i = 0; i < FM; ++i) OA::frag(sa, loa, 0, i, 0, fa[i]);
#pragma unroll
            for (int j = 0; j < FN; ++j) OB::frag(sb, lob, 0, j, 0, fb[j]);
#pragma unroll
            for (int st = 0; st < M::STEPS; ++st) {
                if (st + 1 < M::STEPS) {
#pragma unroll
                    for (int i = 0; i < FM; ++i) OA::frag(sa, loa, 0, i, st + 1, fa[i]);
#pragma unroll
                    for (int j = 0; j < FN; ++j) OB::frag(sb, lob, 0, j, st + 1, fb[j]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        f32x16& a = acc[q * ILP + st % ILP][i][j];
                        a = M::mfma(fa[i][st % OA::RING], fb[j][st % OB::RING], a);
                    }
                // Load l of the stage goes out after step l * TS / LOADS.
                constexpr int TS = SPW * M::STEPS;
                const int gst = q * M::STEPS + st;
                if (spread) {
#pragma unroll
                    for (int l = 0; l < G::LOADS; ++l) {
                        if (l * TS / G::LOADS != gst) continue;
                        if (l < G::LA)
                            dma16(reinterpret_cast<const float*>(pa[l] + lka),
                                  reinterpret_cast<const float*>(lsa + (l * 4 + wave) * (1024 / E::kBytes)));
                        else
                            dma16(reinterpret_cast<const float*>(pb[l - G::LA] + lkb),
                                  reinterpret_cast<const float*>(lsb + ((l - G::LA) * 4 + wave) * (1024 / E::kBytes)));
                    }
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
    }
    // The wave's sets in order: acc[0] = ((set 0 + set 1) + ...).
#pragma unroll
    for (int q = 1; q < NSET; ++q)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[0][i][j][r] = acc[0][i][j][r] + acc[q][i][j][r];

    // Every wave's MFMAs and fragment reads are done (and no load is in
    // flight: the last stage waited for vmcnt(0)) before the ring is reused.
    __syncthreads();
    constexpr int NREG = FM * FN * 16;
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[(wave * NREG + (i * FN + j) * 16 + r) * 64 + lane] = acc[0][i][j][r];
    __syncthreads();

    // Wave w sums and stores registers w * Q .. w * Q + Q - 1 of every lane.
    // 32x32 accumulator layout: lane l, register r of block (i, j) holds row
    // 32 i + 8 (r / 4) + 4 (l / 32) + r % 4 and column 32 j + l % 32.
    constexpr int Q = NREG / 4;
    float* const C = g.c + c_off;
    const bool nt = g.store_nt != 0;
#pragma unroll
    for (int e = 0; e < Q; ++e) {
        const int idx = wave * Q + e;
        const int blk = idx / 16, r = idx % 16;
        const int i = blk / FN, j = blk % FN;
        float v = red[idx * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) v = v + red[(w * NREG + idx) * 64 + lane];
        const int row = 32 * i + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
        const int col = 32 * j + (lane & 31);
        if (row < rows_a && col < rows_b) {
            float* p = C + int64_t(m0 + row) * g.c_ms + int64_t(n0 + col) * g.c_ns;
            if (nt) __builtin_nontemporal_store(v, p);
            else *p = v;
        }
    }
}

}  // namespace pe
