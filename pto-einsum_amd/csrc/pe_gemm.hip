// Host side of the batched MFMA GEMM: descriptor validation, operand layout
// classification, tile / split-K choice and the deterministic split-K
// reduction kernel.
#include "pe_gemm_kernel.h"

#include <algorithm>

// Blocks per CU of the persistent tile loop: 0 launches one block per tile,
// -1 as many blocks as the launched kernel keeps resident per CU.
#ifndef PE_GEMM_PERSIST
#define PE_GEMM_PERSIST -1
#endif
// float16 GEMMs launch one block per tile: blocks dispatched in tile order
// keep the output rows being written in a compact window of HBM, where
// persistent blocks drift apart (config 3, whose 2.15 GB output dominates:
// 458 -> 427 us on one MI355X; 5.1 unchanged).
#ifndef PE_GEMM_F16_PERSIST
#define PE_GEMM_F16_PERSIST 0
#endif
// 256x128 / 128x256 tiles (wave tile 128x64) for grids that still fill the
// GPU, with their own persistent block count.
#ifndef PE_GEMM_BIG
#define PE_GEMM_BIG 1
#endif
// 128x128 tiles per CU at or below which 64x64 tiles are used instead.
#ifndef PE_GEMM_SMALL_TILE_CUS
#define PE_GEMM_SMALL_TILE_CUS 2
#endif
#ifndef PE_GEMM_BIG_PERSIST
#define PE_GEMM_BIG_PERSIST -1
#endif
// Smallest slot fill (tiles / (rounds * resident slots)) at which the
// 256-wide float32 tiles are taken.
#ifndef PE_GEMM_BIG_MIN_FILL
#define PE_GEMM_BIG_MIN_FILL 0.95
#endif

// float32 GEMMs with a K of at most this length whose tile choice splits K
// over blocks, or leaves at most two 64x64 tiles per CU, run the k-split
// kernel (pe_gemm_ks.h) instead: one launch, no partials, four waves per
// tile walking K together.
#ifndef PE_GEMM_KS_MAX_K
#define PE_GEMM_KS_MAX_K 1024
#endif
// Unsplit float32 grids of at most this many 64x64 tiles per CU, with K of at
// least PE_GEMM_KS_MIN_K, take the k-split kernel too; its 64x64 instantiation
// serves grids of at most PE_GEMM_KS_TILE64_PER_CU such tiles per CU (else
// 32x32 tiles).  Widening the rule to the GDN chunk products (256 x 128^3,
// K = 128, four 64x64 tiles per CU) measured 30-32 us against 20 us on the
// direct-load kernel's 64x64 tiles.
#ifndef PE_GEMM_KS_TILES_PER_CU
#define PE_GEMM_KS_TILES_PER_CU 2
#endif
#ifndef PE_GEMM_KS_MIN_K
#define PE_GEMM_KS_MIN_K 256
#endif
#ifndef PE_GEMM_KS_TILE64_PER_CU
#define PE_GEMM_KS_TILE64_PER_CU 1
#endif

// float16 products with K in (96, 128] take the short-K kernel (all of K
// resident in LDS) on grids of at most this many 128x128 tiles per CU (the
// kernel itself runs 64x128 tiles, pe_gemm_dl.hip).  Measured on MI355X
// against the two-stage direct-load kernel (float32 output, cold operands and
// outputs), first with 128x128 short-K tiles: 4096^2 x 128 (config 5.1, 4
// tiles per CU) 18.0 -> 16.2 us, 4096 x 8192 x 128 (8) 31.0 -> 26.9, 8192^2
// x 128 (16) 51.6 -> 48.2, 8192 x 16384 x 128 (32) 117.9 -> 92.8; config 3
// (128 tiles per CU, its 2.15 GB output the bound) 403-412 -> 439 us with
// 128x128 and 482 us with 64x128 short-K tiles, and 4 x 8192^2 x 128 (64
// per CU) 184-185 -> 188 us, so those keep the two-stage kernel, whose four
// blocks per CU keep more stores in flight.
// The float32 variant (eight 16-k slabs, one block per CU; pe_gemm_desc.tile
// = 2) is not chosen automatically: on the GDN 16x16 contractions (256 x
// 128^3, one 128x128 tile per CU) it took 20.8-22.6 us against 18.9-19.6 us
// for 64x64 tiles of the two-stage kernel at four blocks per CU.
#ifndef PE_GEMM_RES
#define PE_GEMM_RES 1
#endif
#ifndef PE_GEMM_RES_MAX_TILES_PER_CU
#define PE_GEMM_RES_MAX_TILES_PER_CU 32
#endif


// float16 GEMMs bound by matrix-core issue take 256x256 tiles (pe_gemm_big.h)
// when those fill at least one round of CUs.
#ifndef PE_GEMM_BIG_F16
#define PE_GEMM_BIG_F16 1
#endif

namespace pe {

// Deterministic split reduction.  Each thread owns VEC consecutive outputs
// and sums their nsplit partials in ascending split order, from +0, exactly
// as a sequential loop would; the partial loads are issued U splits at a time
// so their latencies overlap instead of adding up (U = 16 covers the 16
// splits of the fused chain in one round).  VST: the VEC outputs are
// consecutive elements of one output row, 16-byte aligned, stored as one
// vector.
template <int VEC, int U, bool VST>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs r) {
    using V = typename Pack<VEC, float>::type;
    const uint32_t nv = r.per_split / VEC;
    const uint32_t stride = gridDim.x * 256;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < nv; i += stride) {
        float acc[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
        for (int s0 = 0; s0 < r.nsplit; s0 += U) {
            V x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int sp = min(s0 + u, r.nsplit - 1);
                x[u] = *reinterpret_cast<const V*>(r.partial + int64_t(sp) * r.per_split + int64_t(i) * VEC);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s0 + u < r.nsplit) {
                    if constexpr (VEC == 1) {
                        acc[0] = acc[0] + x[u];
                    } else {
#pragma unroll
                        for (int e = 0; e < VEC; ++e) acc[e] = acc[e] + x[u][e];
                    }
                }
            }
        }
        auto offset = [&](uint32_t idx) {
            uint32_t rest, n, batch, m;
            r.n_div.divmod(idx, rest, n);
            r.m_div.divmod(rest, batch, m);
            int64_t off = int64_t(m) * r.c_ms + int64_t(n) * r.c_ns;
            for (int d = r.nbatch - 1; d >= 0; --d) {
                uint32_t q, rr;
                r.batch_div[d].divmod(batch, q, rr);
                off += int64_t(rr) * r.c_bs[d];
                batch = q;
            }
            return off;
        };
        if constexpr (VST) {
            const f32x4 v = {acc[0], acc[1], acc[2], acc[3]};
            store_f(reinterpret_cast<f32x4*>(r.c + offset(i * VEC)), v, r.store_nt);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) store_f(r.c + offset(i * VEC + e), acc[e], r.store_nt);
        }
    }
}

hipError_t launch_splitk_reduce(const ReduceArgs& r, hipStream_t s) {
    const bool vec = r.per_split % 4 == 0 && (r.nsplit == 0 || aligned(r.partial, 16));
    // Four consecutive outputs form one aligned vector of one output row.
    bool vst = vec && r.c_ns == 1 && r.n_div.d % 4 == 0 && r.c_ms % 4 == 0 && aligned(r.c, 16);
    for (int d = 0; d < r.nbatch; ++d) vst = vst && r.c_bs[d] % 4 == 0;
    const int64_t items = vec ? r.per_split / 4 : r.per_split;
    const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(items, 256), cu_count() * 8)));
    const bool wide = r.nsplit > 8;
    const void* k = vst ? (wide ? reinterpret_cast<const void*>(&splitk_reduce_kernel<4, 16, true>)
                                : reinterpret_cast<const void*>(&splitk_reduce_kernel<4, 8, true>))
                  : vec ? (wide ? reinterpret_cast<const void*>(&splitk_reduce_kernel<4, 16, false>)
                                : reinterpret_cast<const void*>(&splitk_reduce_kernel<4, 8, false>))
                        : reinterpret_cast<const void*>(&splitk_reduce_kernel<1, 8, false>);
    ReduceArgs a = r;
    void* args[] = {&a};
    return hipLaunchKernel(k, dim3(grid), dim3(256), args, 0, s);
}

namespace {

struct GemmChoice {
    int bm, bn;    // tile: 64x64, 128x128, 256x128 or 128x256
    int minb;      // direct-load kernel: register budget (resident blocks per CU) of 256-wide tiles
    int persist;   // blocks per CU of a persistent grid (0: one block per tile, -1: resident count)
    int nsplit;    // K splits (1 = direct store)
    int k_per_split;
    int64_t nbatch_total;
    int64_t ws_bytes;
};

int64_t batch_total(const pe_gemm_desc& d) {
    int64_t n = 1;
    for (int k = 0; k < d.nbatch; ++k) n *= d.batch_shape[k];
    return n;
}

// True when the GEMM's compulsory HBM traffic (operands once, float32 output
// once, at 8 TB/s) takes longer than its MFMA work at the dtype's dense peak
// (157.3 TFLOP/s float32, 2516.6 float16): the output write then sets the
// time, and blocks are launched one per tile in tile order (a compact window
// of output rows in flight) rather than as a persistent grid.
bool hbm_bound(const pe_gemm_desc& d) {
    const double nb = double(batch_total(d));
    const double eb = d.dtype == PE_F32 ? 4.0 : 2.0;
    const double bytes = nb * (double(d.M) * d.N * 4.0 + (double(d.M) + d.N) * d.K * eb);
    const double flops = 2.0 * nb * double(d.M) * d.N * d.K;
    const double peak = d.dtype == PE_F32 ? 157.3e12 : 2516.6e12;
    return bytes / 8.0e12 > flops / peak;
}

// The 256x256 float16 kernel: for direct-load float16 operands of GEMMs
// whose MFMA work outweighs their compulsory traffic, when it has tiles for
// at least a quarter of the CUs (one block per CU) and they cover no more
// padding than 128x128 tiles would.  Below a full round it still beats the
// 128x128 tiles over every CU (settled clocks: 2048^2 x 4096, 64 tiles, 85
// against 93 us; 2048 x 4096 x 2048, 128 tiles, 48 against 55; 3072^2 x
// 2048, 144 tiles, 51 against 58; 3584^2 x 2048, 196 tiles, 59 against
// 77).  tile == 1 asks for it explicitly.
bool big_f16(const pe_gemm_desc& d, bool dl, int al, int bl) {
    if (!PE_GEMM_BIG_F16 || d.dtype != PE_F16 || !dl || d.split_k > 1) return false;
    if (gemm_big_resident(al, bl) < 1) return false;
    // Its full-slab loads address each 16-byte vector by a 32-bit byte offset
    // from the slab's base (256 rows, 32 k): operands whose strides reach
    // past 2^32 bytes within a slab take the direct-load kernel (64-bit
    // addresses) instead.
    auto slab_span = [](int64_t rs, int64_t ks) { return (255 * rs + 31 * ks + 8) * 2; };
    if (slab_span(d.a_ms, d.a_ks) >= (int64_t(1) << 32) || slab_span(d.b_ns, d.b_ks) >= (int64_t(1) << 32))
        return false;
    if (d.tile == 1) return true;
    if (d.tile != 0 || d.split_k != 0 || hbm_bound(d) || d.K < 128) return false;
    const int64_t tm = ceil_div(d.M, 256), tn = ceil_div(d.N, 256);
    if (4 * batch_total(d) * tm * tn < cu_count()) return false;
    return tm * 256 * tn * 256 <= ceil_div(d.M, 128) * 128 * ceil_div(d.N, 128) * 128;
}

// The descriptor with adjacent batch axes merged where all three operands
// address them as one axis (outer stride = inner extent x inner stride);
// extent-1 axes are dropped.
pe_gemm_desc merged_batch(const pe_gemm_desc& d) {
    pe_gemm_desc m = d;
    m.nbatch = 0;
    for (int i = 0; i < d.nbatch; ++i) {
        if (d.batch_shape[i] == 1) continue;
        const int k = m.nbatch - 1;
        if (k >= 0 && m.a_bstride[k] == d.batch_shape[i] * d.a_bstride[i] &&
            m.b_bstride[k] == d.batch_shape[i] * d.b_bstride[i] &&
            m.c_bstride[k] == d.batch_shape[i] * d.c_bstride[i]) {
            m.batch_shape[k] *= d.batch_shape[i];
            m.a_bstride[k] = d.a_bstride[i];
            m.b_bstride[k] = d.b_bstride[i];
            m.c_bstride[k] = d.c_bstride[i];
            continue;
        }
        m.batch_shape[m.nbatch] = d.batch_shape[i];
        m.a_bstride[m.nbatch] = d.a_bstride[i];
        m.b_bstride[m.nbatch] = d.b_bstride[i];
        m.c_bstride[m.nbatch] = d.c_bstride[i];
        ++m.nbatch;
    }
    return m;
}

// Orientation of a 256-wide tile: along the longer output axis; for equal
// extents along the output's contiguous axis, so each tile row written is
// 1 KB of contiguous memory rather than 512 B.
bool wide_along_m(const pe_gemm_desc& d) {
    if (d.M != d.N) return d.M > d.N;
    return d.c_ms < d.c_ns;
}

// Direct-load operand layouts (dl = true) switch the 256-wide candidates to
// the direct-load kernel's own instantiations.  The split-K decision and the
// workspace size do not depend on it (256-wide tiles are only taken on grids
// that need no split).
GemmChoice choose(const pe_gemm_desc& d, bool dl = false, int al = L_MN, int bl = L_MN) {
    GemmChoice c{};
    int64_t long_k_split = 0;
    c.minb = 3;
    c.nbatch_total = batch_total(d);
    if (c.nbatch_total == 0 || d.M == 0 || d.N == 0) {
        // An empty output: nothing is launched (the tile and split counts
        // below would divide by its zero tiles).
        c.bm = c.bn = 128;
        c.nsplit = 1;
        c.k_per_split = int(std::max<int64_t>(d.K, 1));
        return c;
    }
    const int bk = gemm_bk(d.dtype);
    const int64_t cus = cu_count();
    c.persist = PE_GEMM_PERSIST;
    if (d.tile == 2) {  // the short-K kernel: 128x128 tiles, all of K in one block
        c.bm = c.bn = 128;
        c.nsplit = 1;
        c.k_per_split = int(d.K);
        return c;
    }
    if (d.tile == 64 || d.tile == 128) {
        c.bm = c.bn = d.tile;
    } else if (d.tile == 192 || d.tile == 256) {
        const bool tall = wide_along_m(d);
        c.bm = tall ? d.tile : 128;
        c.bn = tall ? 128 : d.tile;
        c.persist = PE_GEMM_BIG_PERSIST;
        if (dl && gemm_dl_resident(d.dtype, c.bm, c.bn, 3, al, bl) < 3) c.minb = 2;
        if (dl && gemm_dl_resident(d.dtype, c.bm, c.bn, c.minb, al, bl) < 1) c.bm = c.bn = 128;
    } else {
        // 64x64 unless 128x128 tiles give every CU more than two: with two
        // or fewer per CU the smaller tiles' extra parallelism hides more
        // load latency than their lower MFMA density costs (measured on
        // MI355X for batched 128^3 blocks and 2048^2 outputs at K = 128..512).
        c.bm = (d.M > 64 && d.N > 64) ? 128 : 64;
        const int64_t tiles128 = c.nbatch_total * ceil_div(d.M, 128) * ceil_div(d.N, 128);
        // (float32 only: the float16 64x64 tiles measured 1.1-3x slower than
        // 128x128 on such grids, e.g. 1024^2 at K = 128: 17.2 against 5.5 us.)
        // Nor where 128x128 tiles already give every CU one and K > 512
        // (2048^2 float32 at K = 4096: 372 -> 344 us; at K = 1024: 95.5 -> 91.8).
        if (c.bm == 128 && d.dtype == PE_F32 && tiles128 <= PE_GEMM_SMALL_TILE_CUS * cus &&
            !(tiles128 >= cus && d.K > 512))
            c.bm = 64;
        // Long-K grids that need a K split with either tile: 128x128 tiles
        // split to about two blocks per CU, each split at least 16 slabs
        // deep, beat 64x64 tiles (config 5.3, ts,sp->tp float32 with K = 4096:
        // 52.5 us against 57.1 us on one MI355X).  The split count is the one
        // whose busiest CU does the least k work: blocks reach each XCD's
        // cus / 8 CUs round robin, so its CUs run up to ceil(ceil(tiles * s /
        // 8) / (cus / 8)) blocks of K / s (k rounded to slabs), a CU running
        // one block at about 0.9 of the rate of two; ties go to fewer splits
        // (fewer partials).  Against two blocks per CU, one MI355X: 768^2 x
        // 4096 74.3 -> 55.0 us (14 splits), 1024 x 1536 x 4096 155.8 -> 116.9
        // (8 splits).
        if (d.M > 64 && d.N > 64 && tiles128 < cus && d.split_k == 0 &&
            c.nbatch_total * d.M * d.N < (int64_t(1) << 32)) {
            const int64_t s2 = std::min<int64_t>(32, ceil_div(2 * cus, tiles128));
            if (d.K >= 16 * bk * s2) {
                c.bm = 128;
                const int64_t cpx = std::max<int64_t>(1, cus / 8);
                double best_cost = 0.0;
                for (int64_t sc = 2; sc <= std::min<int64_t>(32, d.K / (16 * bk)); ++sc) {
                    const int64_t kps = ceil_div(ceil_div(d.K, sc), bk) * bk;
                    const int64_t per_cu = ceil_div(ceil_div(tiles128 * ceil_div(d.K, kps), 8), cpx);
                    const double cost = double(per_cu * kps) / (per_cu == 1 ? 0.9 : 1.0);
                    if (long_k_split == 0 || cost < best_cost) {
                        long_k_split = sc;
                        best_cost = cost;
                    }
                }
            }
        }
        c.bn = c.bm;
        if (PE_GEMM_BIG && dl && c.bm == 128 && !hbm_bound(d) && d.dtype == PE_F16) {
            // Direct-load float16 256x128 / 128x256 tiles come in two
            // register budgets, three or two resident blocks per CU, and
            // pay off in whole rounds (4096^2 x 1024: 512 tiles, one round
            // at two per CU, 43.5 us against 47.5 for 128x128; 4 x 2048^2 x
            // 2048 84 against 97; 3072^2 x 2048 51.7 against 54.6, steady
            // clocks).  Float32 keeps the direct-load 128x128 tiles (four
            // blocks per CU): at steady clocks they beat the 256-wide ones
            // on every MFMA-bound shape measured (config 2 278 against 292
            // us, 8 x 2048^2 x 512 245 against 262, 4096^3 919 against 928,
            // 4096 x 6144 x 1024 356 against 362; 4 x 2048^2 x 2048 with
            // both operands k-contiguous 483 against 480).  Both
            // orientations are candidates, the one along the longer output
            // axis first (their register allocations differ; an
            // instantiation that spills reports no residency).
            double best = PE_GEMM_BIG_MIN_FILL;
            bool taken = false;
            const bool tall = wide_along_m(d);
            for (int o = 0; o < 2; ++o) {
                const bool wide_m = (o == 0) == tall;
                const int bbm = wide_m ? 256 : 128, bbn = wide_m ? 128 : 256;
                const int64_t bt = c.nbatch_total * ceil_div(d.M, bbm) * ceil_div(d.N, bbn);
                const bool no_waste = ceil_div(d.M, bbm) * bbm * ceil_div(d.N, bbn) * bbn <=
                                      ceil_div(d.M, 128) * 128 * ceil_div(d.N, 128) * 128;
                for (int minb = 3; minb >= 2 && bt >= cus && no_waste; --minb) {
                    // A budget whose blocks do not all fit (LDS) gives up
                    // registers for nothing: skip it for the next one.
                    const int res = gemm_dl_resident(d.dtype, bbm, bbn, minb, al, bl);
                    if (res < minb) continue;
                    const int64_t slots = cus * res;
                    const double fill = double(bt) / double(ceil_div(bt, slots) * slots);
                    if (fill >= best + 1e-9 || (fill >= best && !taken)) {
                        best = fill;
                        taken = true;
                        c.bm = bbm;
                        c.bn = bbn;
                        c.minb = minb;
                    }
                }
            }
        } else if (PE_GEMM_BIG && !dl && c.bm == 128 && d.dtype == PE_F32) {
            // 256x128 / 128x256 tiles (wave tile 128x64) read fewer LDS
            // fragments per MFMA but hold two waves per SIMD.  Measured on
            // MI355X: they beat 128x128 by 10-25 % when their tiles fill the
            // resident block slots in whole rounds (4096^2 at K = 512..4096),
            // and lose by 5-35 % when a round is left part-filled (config 2:
            // 1.5 rounds, where the last round runs one block per CU).  So
            // take them only for (nearly) whole rounds.
            auto fill = [&](int bm, int bn) {
                const int64_t t = c.nbatch_total * ceil_div(d.M, bm) * ceil_div(d.N, bn);
                const int64_t slots = cus * gemm_occupancy_f32(bm, bn);
                const int64_t rounds = ceil_div(t, slots);
                return double(t) / double(rounds * slots);
            };
            const bool tall = wide_along_m(d);
            const int bbm = tall ? 256 : 128, bbn = tall ? 128 : 256;
            const int64_t bt = c.nbatch_total * ceil_div(d.M, bbm) * ceil_div(d.N, bbn);
            // ... and only when they cover no more padding than 128x128
            // tiles (a 128-row batch in a 256-row tile doubles the MFMAs).
            const bool no_waste = ceil_div(d.M, bbm) * bbm * ceil_div(d.N, bbn) * bbn <=
                                  ceil_div(d.M, 128) * 128 * ceil_div(d.N, 128) * 128;
            if (bt >= cus && no_waste && fill(bbm, bbn) >= PE_GEMM_BIG_MIN_FILL) {
                c.bm = bbm;
                c.bn = bbn;
                c.persist = PE_GEMM_BIG_PERSIST;
            }
        }
    }
    const int64_t tiles = c.nbatch_total * ceil_div(d.M, c.bm) * ceil_div(d.N, c.bn);
    int64_t split = 1;
    if (d.split_k > 0) {
        split = d.split_k;
    } else if (long_k_split > 0) {
        split = long_k_split;
    } else if (tiles < cus && c.nbatch_total * d.M * d.N < (int64_t(1) << 32)) {
        // At most about four blocks per CU and at least four K slabs per
        // split; beyond one block per CU, split further only while each split
        // keeps 16 slabs (the reduction reads every split's partial output
        // back: 512^2 at K = 1024, 16 splits of 4 slabs 19.3 us, 4 of 16
        // slabs 15.3 us; 256^3, 4 splits of 4 slabs, 7.4 us either way).
        split = std::min<int64_t>(ceil_div(4 * cus, tiles), std::max<int64_t>(1, d.K / (4 * bk)));
        split = std::min<int64_t>(split, std::max<int64_t>(ceil_div(cus, tiles), d.K / (16 * bk)));
        split = std::max<int64_t>(1, std::min<int64_t>(split, 32));
    }
    if (d.dtype == PE_F32 && d.split_k == 0 && d.tile == 0 && c.bm == c.bn && (c.bm == 64 || c.bm == 128) &&
        c.nbatch_total * d.M * d.N < (int64_t(1) << 32)) {
        // Rebalance float32 square-tile grids the rules above leave uneven.
        // Blocks reach each XCD's cus / 8 CUs round robin, so the busiest CU
        // runs P = ceil(ceil(blocks / 8) / (cus / 8)) blocks; its time is
        // modelled as P x (tile area) x (k per split), at 0.9 of the rate for
        // 64x64 tiles and for a CU with one block, plus the split partials'
        // round trip (0.01 per output element and split, per CU, in the same
        // units: fitted to eight measured shapes, within 1 % of the best of
        // their measured options on average).  Another tile or split count is
        // taken only where the model gives it 20 % less time: 2304^2 x 6144
        // 827.7 -> 580.4 us (128x128, 8 splits, against 1.27 unsplit tiles per
        // CU), 384 x 2816 x 1536 74.5 -> 47.8 us (128x128, 6 splits, against
        // 64x64 tiles unsplit) on one MI355X.
        const int64_t cpx = std::max<int64_t>(1, cus / 8);
        auto model = [&](int tile, int64_t sc) {
            const int64_t kp = ceil_div(ceil_div(d.K, sc), bk) * bk;
            const int64_t sp = ceil_div(d.K, kp);
            const int64_t t = c.nbatch_total * ceil_div(d.M, tile) * ceil_div(d.N, tile);
            const int64_t per = ceil_div(ceil_div(t * sp, 8), cpx);
            const double eff = (tile == 64 ? 0.9 : 1.0) * (per == 1 ? 0.9 : 1.0);
            const double area = double(tile / 64) * double(tile / 64);
            const double part = sp > 1 ? 0.01 * double(sp) * double(c.nbatch_total * d.M * d.N) / double(cus) : 0.0;
            return double(per) * area * double(kp) / eff + part;
        };
        const double now = model(c.bm, split);
        double best = now;
        int best_tile = c.bm;
        int64_t best_split = split;
        for (int tile : {64, 128}) {
            if (tile == 128 && (d.M <= 64 || d.N <= 64)) continue;
            for (int64_t sc = 1; sc <= std::min<int64_t>(32, std::max<int64_t>(1, d.K / (16 * bk))); ++sc) {
                const double m = model(tile, sc);
                if (m < best) {
                    best = m;
                    best_tile = tile;
                    best_split = sc;
                }
            }
        }
        if (best < 0.8 * now) {
            c.bm = c.bn = best_tile;
            split = best_split;
        }
    } else if (d.dtype == PE_F16 && d.split_k == 0 && d.tile == 0 && c.bm == 128 && c.bn == 128 && split == 1 &&
               c.nbatch_total * d.M * d.N < (int64_t(1) << 32)) {
        // float16 128x128 grids of one to four tiles per CU, unsplit: the
        // same model with float16's own constants (a CU with one block at 0.8
        // of the rate of two, partials 0.04 per output element and split:
        // float16 MFMAs make the partials' round trip weigh more; fitted to
        // twenty measured shapes) may split them where one round is left
        // part-filled: 2816 x 1664 x 3072 68.9 -> 60.5 us with 4 splits.
        const int64_t t = c.nbatch_total * ceil_div(d.M, 128) * ceil_div(d.N, 128);
        if (t >= cus && t < 4 * cus) {
            const int64_t cpx = std::max<int64_t>(1, cus / 8);
            auto model = [&](int64_t sc) {
                const int64_t kp = ceil_div(ceil_div(d.K, sc), bk) * bk;
                const int64_t sp = ceil_div(d.K, kp);
                const int64_t per = ceil_div(ceil_div(t * sp, 8), cpx);
                const double part = sp > 1 ? 0.04 * double(sp) * double(c.nbatch_total * d.M * d.N) / double(cus) : 0.0;
                return double(per) * 4.0 * double(kp) / (per == 1 ? 0.8 : 1.0) + part;
            };
            const double now = model(1);
            double best = now;
            int64_t best_split = 1;
            for (int64_t sc = 2; sc <= std::min<int64_t>(32, d.K / (16 * bk)); ++sc) {
                const double m = model(sc);
                if (m < best) {
                    best = m;
                    best_split = sc;
                }
            }
            if (best < 0.8 * now) split = best_split;
        }
    }
    int64_t kps = ceil_div(ceil_div(d.K, split), bk) * bk;
    split = std::max<int64_t>(1, ceil_div(d.K, kps));
    c.nsplit = int(split);
    c.k_per_split = int(kps);
    c.ws_bytes = split > 1 ? split * c.nbatch_total * d.M * d.N * int64_t(sizeof(float)) : 0;
    return c;
}

// Direct-load full slabs address each operand vector by a 32-bit byte offset
// from the slab's base: (256 rows, 64 bytes of k) of both operands within
// 2^32 bytes.
bool dl_off32(const pe_gemm_desc& d) {
    const int64_t elem = d.dtype == PE_F32 ? 4 : 2;
    auto span_ok = [&](int64_t rs, int64_t ks) {
        return rs >= 0 && ks >= 0 && (256 * rs + (64 / elem) * ks + 8) * elem < (int64_t(1) << 32);
    };
    return span_ok(d.a_ms, d.a_ks) && span_ok(d.b_ns, d.b_ks);
}

// float16 products with K in (96, 128] (four 32-k slabs) that the tile
// choice leaves unsplit on 128x128 tiles, at most
// PE_GEMM_RES_MAX_TILES_PER_CU of those per CU: the short-K kernel, all of K
// in flight at once.
bool res_auto(const pe_gemm_desc& d, const GemmChoice& ch, bool dl, int al, int bl) {
    return PE_GEMM_RES && dl && d.dtype == PE_F16 && d.split_k == 0 && d.tile == 0 && ch.nsplit == 1 &&
           ch.bm == 128 && ch.bn == 128 && d.K > 96 && d.K <= 128 &&
           batch_total(d) * ceil_div(d.M, 128) * ceil_div(d.N, 128) <= PE_GEMM_RES_MAX_TILES_PER_CU * cu_count() &&
           gemm_res_resident(d.dtype, al, bl) >= 1;
}

// Launch of the short-K kernel (gemm_res_kernel) for descriptor d.
hipError_t launch_res(const pe_gemm_desc& d, const void* a, const void* b, float* c, int64_t nb, int al, int bl,
                      hipStream_t s) {
    GemmArgs g{};
    g.a = a; g.b = b; g.c = c;
    g.partial = nullptr;
    g.M = int32_t(d.M); g.N = int32_t(d.N); g.K = int32_t(d.K);
    g.nsplit = 1;
    g.k_per_split = int32_t(d.K);
    g.tiles_m = int32_t(ceil_div(d.M, gemm_res_tile_m(d.dtype)));
    g.tiles_n = int32_t(ceil_div(d.N, gemm_res_tile_n(d.dtype)));
    g.tiles_per_batch = uint32_t(g.tiles_m) * uint32_t(g.tiles_n);
    g.nbatch_total = uint32_t(nb);
    g.total_blocks = g.tiles_per_batch * g.nbatch_total;
    g.grid = g.total_blocks;
    g.store_nt = nt_mode(nb * d.M * d.N * 4);
    g.off32 = dl_off32(d);
    g.a_ms = d.a_ms; g.a_ks = d.a_ks; g.b_ks = d.b_ks; g.b_ns = d.b_ns;
    g.c_ms = d.c_ms; g.c_ns = d.c_ns;
    g.nbatch = d.nbatch;
    for (int i = 0; i < d.nbatch; ++i) {
        g.batch_div[i].init(uint32_t(d.batch_shape[i]));
        g.a_bs[i] = d.a_bstride[i];
        g.b_bs[i] = d.b_bstride[i];
        g.c_bs[i] = d.c_bstride[i];
    }
    return launch_gemm_res(d.dtype, al, bl, g, s);
}

int classify(int64_t rows, int64_t k, int64_t rs, int64_t ks, const int64_t* bs, int nb,
             const void* p, int vec) {
    // Extent-1 axes carry no stride; treat them as absent.
    if (rows == 1) rs = 0;
    if (k == 1) ks = 0;
    bool batch_ok = true;
    for (int i = 0; i < nb; ++i) batch_ok = batch_ok && (bs[i] % vec == 0);
    const bool al = aligned(p, 16) && batch_ok;
    if (rs == 1 && ks % vec == 0 && al) return L_MN;
    if (ks == 1 && rs % vec == 0 && al) return L_K;
    return L_GENERIC;
}

}  // namespace

int validate_gemm(const pe_gemm_desc& d) {
    if (d.dtype != PE_F32 && d.dtype != PE_F16)
        return fail(PE_ERR_UNSUPPORTED, "gemm: dtype must be PE_F32 or PE_F16");
    if (d.nbatch < 0 || d.nbatch > PE_MAX_DIMS) return fail(PE_ERR_INVALID, "gemm: nbatch out of range");
    if (d.tile != 0 && d.tile != 1 && d.tile != 2 && d.tile != 64 && d.tile != 128 && d.tile != 192 && d.tile != 256)
        return fail(PE_ERR_INVALID, "gemm: tile must be 0, 1, 2, 64, 128, 192 or 256");
    if (d.tile == 2 && (d.split_k > 1 || d.K > 128 || d.K <= (d.dtype == PE_F16 ? 96 : 112)))
        return fail(PE_ERR_UNSUPPORTED,
                    "gemm: the short-K kernel (tile 2) takes K in (96, 128] (float16) or (112, 128] (float32), no split");
    if (d.tile == 1 && (d.dtype != PE_F16 || d.split_k > 1))
        return fail(PE_ERR_UNSUPPORTED, "gemm: the 256x256 tile (1) is float16 only, without a K split");
    if (d.tile == 192 && d.dtype != PE_F32)
        return fail(PE_ERR_UNSUPPORTED, "gemm: the 192 tile is float32 only");
    if (d.split_k < 0) return fail(PE_ERR_INVALID, "gemm: split_k must be >= 0");
    if (d.M < 0 || d.N < 0 || d.K < 0) return fail(PE_ERR_INVALID, "gemm: negative extent");
    if (d.M >= (int64_t(1) << 31) || d.N >= (int64_t(1) << 31) || d.K >= (int64_t(1) << 31))
        return fail(PE_ERR_UNSUPPORTED, "gemm: M, N and K must each be below 2^31");
    int64_t amax = 0, bmax = 0, cmax = 0, nb = 1;
    for (int i = 0; i < d.nbatch; ++i) {
        if (d.batch_shape[i] < 0 || d.a_bstride[i] < 0 || d.b_bstride[i] < 0 || d.c_bstride[i] < 0)
            return fail(PE_ERR_INVALID, "gemm: negative batch extent or stride");
        nb *= d.batch_shape[i];
        if (d.batch_shape[i] > 0) {
            amax += (d.batch_shape[i] - 1) * d.a_bstride[i];
            bmax += (d.batch_shape[i] - 1) * d.b_bstride[i];
            cmax += (d.batch_shape[i] - 1) * d.c_bstride[i];
        }
    }
    if (nb >= (int64_t(1) << 31)) return fail(PE_ERR_UNSUPPORTED, "gemm: batch count must be below 2^31");
    if (d.a_ms < 0 || d.a_ks < 0 || d.b_ks < 0 || d.b_ns < 0 || d.c_ms < 0 || d.c_ns < 0)
        return fail(PE_ERR_INVALID, "gemm: negative stride");
    if (nb == 0 || d.M == 0 || d.N == 0) return PE_OK;
    cmax += (d.M - 1) * d.c_ms + (d.N - 1) * d.c_ns;
    if (cmax >= d.c_numel) return fail(PE_ERR_BOUNDS, "gemm: C strides address past the output");
    if (d.K > 0) {
        amax += (d.M - 1) * d.a_ms + (d.K - 1) * d.a_ks;
        bmax += (d.N - 1) * d.b_ns + (d.K - 1) * d.b_ks;
        if (amax >= d.a_numel) return fail(PE_ERR_BOUNDS, "gemm: A strides address past operand 0");
        if (bmax >= d.b_numel) return fail(PE_ERR_BOUNDS, "gemm: B strides address past operand 1");
    }
    const int64_t tiles = nb * ceil_div(d.M, 64) * ceil_div(d.N, 64) * 32;
    if (tiles >= (int64_t(1) << 32)) return fail(PE_ERR_UNSUPPORTED, "gemm: too many tiles");
    return PE_OK;
}

}  // namespace pe

extern "C" int pe_gemm_choice(const pe_gemm_desc* d, int64_t* info) {
    if (!d || !info) return pe::fail(PE_ERR_INVALID, "gemm_choice: null argument");
    const int st = pe::validate_gemm(*d);
    if (st != PE_OK) return st;
    // As pe_gemm chooses for these strides, operand pointers taken as
    // 16-byte aligned (the split is the same for every layout).
    const int vec = d->dtype == PE_F32 ? 4 : 8;
    const int al = pe::classify(d->M, d->K, d->a_ms, d->a_ks, d->a_bstride, d->nbatch, nullptr, vec);
    const int bl = pe::classify(d->N, d->K, d->b_ns, d->b_ks, d->b_bstride, d->nbatch, nullptr, vec);
    const bool dl = d->tile != 192 && pe::gemm_dl_eligible(d->dtype, al, bl, d->M, d->N, d->K, d->c_ms, d->c_ns);
    if (d->tile == 1 || (d->tile != 2 && pe::big_f16(*d, dl, al, bl) && pe::merged_batch(*d).nbatch <= 1)) {
        info[0] = info[1] = 256;
        info[2] = 1;
        info[3] = d->K;
        return PE_OK;
    }
    const pe::GemmChoice c = pe::choose(*d, dl, al, bl);
    if (d->tile == 2 || pe::res_auto(*d, c, dl, al, bl)) {
        info[0] = pe::gemm_res_tile_m(d->dtype);
        info[1] = pe::gemm_res_tile_n(d->dtype);
        info[2] = 1;
        info[3] = d->K;
        return PE_OK;
    }
    info[0] = c.bm;
    info[1] = c.bn;
    info[2] = c.nsplit;
    info[3] = c.k_per_split;
    return PE_OK;
}

extern "C" int64_t pe_gemm_workspace_bytes(const pe_gemm_desc* d) {
    if (!d || pe::validate_gemm(*d) != PE_OK) return 0;
    if (d->K == 0 || d->M == 0 || d->N == 0 || pe::batch_total(*d) == 0) return 0;
    return pe::choose(*d).ws_bytes;
}

extern "C" int pe_gemm(const pe_gemm_desc* d, const void* a, const void* b, float* c, void* ws,
                       int64_t ws_bytes, void* stream) {
    using namespace pe;
    if (!d) return fail(PE_ERR_INVALID, "gemm: null descriptor");
    int st = validate_gemm(*d);
    if (st != PE_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = batch_total(*d);
    if (nb == 0 || d->M == 0 || d->N == 0) return PE_OK;

    ReduceArgs r{};
    r.c = c;
    r.per_split = uint32_t(nb * d->M * d->N);
    r.n_div.init(uint32_t(d->N));
    r.m_div.init(uint32_t(d->M));
    r.c_ms = d->c_ms;
    r.c_ns = d->c_ns;
    r.nbatch = d->nbatch;
    for (int i = 0; i < d->nbatch; ++i) {
        r.batch_div[i].init(uint32_t(d->batch_shape[i]));
        r.c_bs[i] = d->c_bstride[i];
    }
    if (d->K == 0) {  // empty contraction: every output is the empty sum, +0
        if (nb * d->M * d->N >= (int64_t(1) << 32)) return fail(PE_ERR_UNSUPPORTED, "gemm: output too large");
        r.nsplit = 0;
        r.partial = nullptr;
        PE_CHECK_HIP(launch_splitk_reduce(r, s));
        return PE_OK;
    }

    const int vec = d->dtype == PE_F32 ? 4 : 8;
    const int al = classify(d->M, d->K, d->a_ms, d->a_ks, d->a_bstride, d->nbatch, a, vec);
    const int bl = classify(d->N, d->K, d->b_ns, d->b_ks, d->b_bstride, d->nbatch, b, vec);
    bool dl = d->tile != 192 && gemm_dl_eligible(d->dtype, al, bl, d->M, d->N, d->K, d->c_ms, d->c_ns);
    if (big_f16(*d, dl, al, bl) && merged_batch(*d).nbatch <= 1) {
        const pe_gemm_desc md = merged_batch(*d);
        GemmArgs g{};
        g.a = a; g.b = b; g.c = c;
        g.partial = nullptr;
        g.M = int32_t(d->M); g.N = int32_t(d->N); g.K = int32_t(d->K);
        g.nsplit = 1;
        g.k_per_split = int32_t(d->K);
        g.tiles_m = int32_t(ceil_div(d->M, 256));
        g.tiles_n = int32_t(ceil_div(d->N, 256));
        g.tiles_per_batch = uint32_t(g.tiles_m) * uint32_t(g.tiles_n);
        g.nbatch_total = uint32_t(nb);
        g.total_blocks = g.tiles_per_batch * g.nbatch_total;
        g.grid = g.total_blocks;
        g.store_nt = nt_mode(nb * d->M * d->N * 4);
        g.a_ms = d->a_ms; g.a_ks = d->a_ks; g.b_ks = d->b_ks; g.b_ns = d->b_ns;
        g.c_ms = d->c_ms; g.c_ns = d->c_ns;
        g.nbatch = md.nbatch;
        g.batch_div[0].init(uint32_t(md.nbatch ? md.batch_shape[0] : 1));
        g.a_bs[0] = md.nbatch ? md.a_bstride[0] : 0;
        g.b_bs[0] = md.nbatch ? md.b_bstride[0] : 0;
        g.c_bs[0] = md.nbatch ? md.c_bstride[0] : 0;
        PE_CHECK_HIP(launch_gemm_big(al, bl, g, s));
        return PE_OK;
    }
    if (d->tile == 1)
        return fail(PE_ERR_UNSUPPORTED,
                    "gemm: the 256x256 tile needs 16-byte vector operands and batch axes that merge into one");
    if (d->tile == 2) {
        if (!dl || gemm_res_resident(d->dtype, al, bl) < 1)
            return fail(PE_ERR_UNSUPPORTED, "gemm: the short-K kernel (tile 2) needs 16-byte vector operands");
        PE_CHECK_HIP(launch_res(*d, a, b, c, nb, al, bl, s));
        return PE_OK;
    }
    GemmChoice ch = choose(*d, dl, al, bl);
    if (dl && gemm_dl_resident(d->dtype, ch.bm, ch.bn, ch.minb, al, bl) < 1) {
        // the chosen direct-load instantiation spills: the staged kernel
        dl = false;
        ch = choose(*d, false, al, bl);
    }
    if (ch.nsplit > 1) {
        if (!ws || ws_bytes < ch.ws_bytes) return fail(PE_ERR_WORKSPACE, "gemm: split-K workspace missing or too small");
        if (nb * d->M * d->N >= (int64_t(1) << 32))
            return fail(PE_ERR_UNSUPPORTED, "gemm: split-K output too large");
    }
    // A short K that the tile choice would split, or (K >= 256) whose 64x64
    // tiles give each CU at most two: the k-split kernel, one block per 64x64
    // tile where those give each CU between three quarters of one and one,
    // else per 32x32 tile (at most 16x the split grid's 64x64 or 128x128
    // tiles, fewer than 2^31 blocks).  Measured on one MI355X against the
    // split or unsplit grid: 256^3 7.4 -> 4.9 us, 512^2 x 1024 15.5 -> 10.8,
    // 1024^3 36.2 -> 25.5, 1024^2 x 512 19.5 -> 15.9, 1024 x 1536 x 1024
    // 51.2 -> 36.2, 1280^2 x 768 39.4 -> 33.4, 2048 x 1024 x 512 28.4 ->
    // 27.4; more 64x64 tiles per CU stay on them (2048 x 1536 x 256, three
    // per CU: 21.6 against 25.3; 1536^2 x 1024, 2.25 per CU: 52.2 against
    // 53.3), and 64x64 k-split tiles lost where they left CUs idle (768^2 x
    // 1024: 24.6 against 19.2 us on 32x32 ones).
    // Split grids with K up to twice that length take it too when its 32x32
    // tiles give every CU one (1024 x 1536 x 2048 83.9 -> 66.9 us, 1536^2 x
    // 2048 113.7 -> 98.8, 512^2 x 2048 23.0 -> 18.8; 2048 x 1024 x 2048 84.6
    // against 88.1; fewer tiles lost: 1024 x 128 x 2048 16.9 against 18.7).
    // float16 split grids take its 64x64 tiles (float16 MFMAs are 16x the
    // float32 rate, so the split's partial round trip weighs more) when those
    // give every CU one to three (K <= 8192) or a quarter of the CUs one (K <=
    // 2048): 1024^3 19.9 -> 9.8 us, 768^2 x 2048 21.7 -> 12.6, 1024^2 x 8192
    // 44.8 -> 37.6, 512^2 x 1024 12.7 -> 8.7, 2048 x 1024 x 1024 24.7 ->
    // 17.0, 1152 x 2304 x 512 (2.5 per CU) 23.6 -> 19.3; fewer tiles, more
    // tiles or longer K lost (256^2 x 2048 9.6 against 12.1, 4096 x 128 x
    // 4096 22.6 against 26.4, 1664 x 2304 x 3072 with 3.7 tiles per CU 48.8
    // against 60.1).
    const int64_t cus = cu_count();
    if (res_auto(*d, ch, dl, al, bl)) {
        PE_CHECK_HIP(launch_res(*d, a, b, c, nb, al, bl, s));
        return PE_OK;
    }

    const int64_t tiles64 = nb * ceil_div(d->M, 64) * ceil_div(d->N, 64);
    const int64_t tiles32 = nb * ceil_div(d->M, 32) * ceil_div(d->N, 32);
    int ks_tile = (4 * tiles64 >= 3 * cus && tiles64 <= PE_GEMM_KS_TILE64_PER_CU * cus) ? 64 : 32;
    bool ks_k;
    if (d->dtype == PE_F32) {
        ks_k = d->K <= PE_GEMM_KS_MAX_K ? (ch.nsplit > 1 || (tiles64 <= PE_GEMM_KS_TILES_PER_CU * cus &&
                                                             d->K >= PE_GEMM_KS_MIN_K))
                                        : (d->K <= 2 * PE_GEMM_KS_MAX_K && ch.nsplit > 1 && tiles32 >= cus);
    } else {
        ks_tile = 64;
        ks_k = ch.nsplit > 1 && tiles64 <= 3 * cus &&
               ((tiles64 >= cus && d->K <= 8 * PE_GEMM_KS_MAX_K) || (4 * tiles64 >= cus && d->K <= 2 * PE_GEMM_KS_MAX_K));
    }
    if (ks_k && dl && d->split_k == 0 && d->tile == 0 && gemm_ks_resident(d->dtype, al, bl, ks_tile) >= 1) {
        GemmArgs g{};
        g.a = a; g.b = b; g.c = c;
        g.partial = nullptr;
        g.M = int32_t(d->M); g.N = int32_t(d->N); g.K = int32_t(d->K);
        g.nsplit = 1;
        g.k_per_split = int32_t(d->K);
        g.tiles_m = int32_t(ceil_div(d->M, ks_tile));
        g.tiles_n = int32_t(ceil_div(d->N, ks_tile));
        g.tiles_per_batch = uint32_t(g.tiles_m) * uint32_t(g.tiles_n);
        g.nbatch_total = uint32_t(nb);
        g.total_blocks = g.tiles_per_batch * g.nbatch_total;
        g.grid = g.total_blocks;
        g.store_nt = nt_mode(nb * d->M * d->N * 4);
        g.a_ms = d->a_ms; g.a_ks = d->a_ks; g.b_ks = d->b_ks; g.b_ns = d->b_ns;
        g.c_ms = d->c_ms; g.c_ns = d->c_ns;
        g.nbatch = d->nbatch;
        for (int i = 0; i < d->nbatch; ++i) {
            g.batch_div[i].init(uint32_t(d->batch_shape[i]));
            g.a_bs[i] = d->a_bstride[i];
            g.b_bs[i] = d->b_bstride[i];
            g.c_bs[i] = d->c_bstride[i];
        }
        PE_CHECK_HIP(launch_gemm_ks(d->dtype, al, bl, ks_tile, g, s));
        return PE_OK;
    }
    GemmArgs g{};
    g.a = a; g.b = b; g.c = c;
    g.partial = static_cast<float*>(ws);
    g.M = int32_t(d->M); g.N = int32_t(d->N); g.K = int32_t(d->K);
    g.nsplit = ch.nsplit;
    g.k_per_split = ch.k_per_split;
    g.tiles_m = int32_t(ceil_div(d->M, ch.bm));
    g.tiles_n = int32_t(ceil_div(d->N, ch.bn));
    g.tiles_per_batch = uint32_t(g.tiles_m) * uint32_t(g.tiles_n);
    g.nbatch_total = uint32_t(nb);
    g.total_blocks = g.tiles_per_batch * g.nbatch_total * uint32_t(ch.nsplit);
    g.grid = g.total_blocks;
    g.store_nt = ch.nsplit > 1 ? int(ch.ws_bytes >= PE_NT_PARTIAL_MIN_BYTES) : nt_mode(nb * d->M * d->N * 4);
    g.a_ms = d->a_ms; g.a_ks = d->a_ks; g.b_ks = d->b_ks; g.b_ns = d->b_ns;
    g.c_ms = d->c_ms; g.c_ns = d->c_ns;
    g.nbatch = d->nbatch;
    for (int i = 0; i < d->nbatch; ++i) {
        g.batch_div[i].init(uint32_t(d->batch_shape[i]));
        g.a_bs[i] = d->a_bstride[i];
        g.b_bs[i] = d->b_bstride[i];
        g.c_bs[i] = d->c_bstride[i];
    }
    g.off32 = dl && dl_off32(*d);
    hipError_t e = dl                   ? launch_gemm_dl(d->dtype, ch.bm, ch.bn, ch.minb, al, bl, !hbm_bound(*d), g, s)
                   : d->dtype == PE_F32 ? launch_gemm_f32(ch.bm, ch.bn, al, bl, ch.persist, g, s)
                                        : launch_gemm_f16(ch.bm, ch.bn, al, bl, PE_GEMM_F16_PERSIST, g, s);
    PE_CHECK_HIP(e);
    if (ch.nsplit > 1) {
        r.nsplit = ch.nsplit;
        r.partial = static_cast<const float*>(ws);
        r.store_nt = nt_mode(nb * d->M * d->N * 4);
        PE_CHECK_HIP(launch_splitk_reduce(r, s));
    }
    return PE_OK;
}
