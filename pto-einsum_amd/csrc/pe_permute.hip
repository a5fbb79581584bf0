// Permutation copies (bit-exact) of 2- and 4-byte elements.
//
// Reference counterpart: transpose_inline and its bodies
// (pto_einsum_transpose.h:27-660): identity copy, N-D gather with the
// innermost axis kept, and 2D / batched-2D TTRANS when the innermost axis
// moves.  The destination is row-major over `shape`; destination axis d reads
// the source with stride src_stride[d] -- the transfer_idx map of
// cpu_einsum.h:35-43.
//
// After merging axes that stay adjacent (and dropping extent-1 axes) there
// are two cases, both HBM-bound (one read and one write per element):
//  * the innermost destination axis is also source-contiguous: a streamed
//    gather of contiguous runs with 16-byte vectors where the run length and
//    strides allow it;
//  * otherwise a 64x64 LDS-tiled transpose (32x32 for float32 destination
//    rows that are not whole 16-byte vectors, 32x64 where those rows are
//    33 to 64 elements long: [16, 777, 1000] -> (0, 2, 1)
//    26.9 -> 24.0 us, while aligned rows measured equal or slower with the
//    smaller tile) between the destination's innermost axis and the axis
//    that is contiguous in the source, with the remaining axes decoded from
//    blockIdx.  Both global sides are coalesced;
//    the LDS tile has one padding column so the transposed read is free of
//    bank conflicts.
#include "pe_common.h"

#include <algorithm>
#include <vector>

namespace pe {
namespace {

constexpr int kThreads = 256;

// Gather stream shape of the persistent grid (many resident waves, two
// 16-byte vectors in flight per lane), used for unaligned gathers; aligned
// ones take a flat launch, one vector per thread (PE_GATHER_FLAT, see run()),
// with non-temporal stores for outputs beyond the Infinity Cache.
#ifndef PE_GATHER_GRID_PER_CU
#define PE_GATHER_GRID_PER_CU 64
#endif
#ifndef PE_GATHER_UNROLL
#define PE_GATHER_UNROLL 2
#endif
#ifndef PE_GATHER_FLAT
#define PE_GATHER_FLAT 1
#endif

struct GatherArgs {
    const void* src;
    void* dst;
    uint32_t nvec;           // destination vectors (32-bit path)
    FastDiv inner_vecs;      // innermost extent / VEC
    int32_t nouter;
    FastDiv outer_div[PE_MAX_DIMS];
    int64_t outer_stride[PE_MAX_DIMS];
    int64_t inner_stride;    // source stride of the innermost destination axis
    int32_t nt;              // output store flavour (nt_mode)
};

template <typename W, int VEC>
struct Chunk {
    W v[VEC];
};

// A 16-byte store of flavour `mode` (nt_mode).
__device__ __forceinline__ void put(u32x4* p, const u32x4& v, int mode) { store_f(p, v, mode); }

// Streamed gather: VEC elements of type W per vector (16 bytes when VEC > 1),
// U vectors per lane in flight.  Every source vector is read once, with the
// non-temporal hint (measured on MI355X: config 3 in0, 134 MB, 26.4-26.6 ->
// 25.1-25.3 us; config 3's output permutation 715-718 -> 704-707 us; the
// tiled transposes, whose neighbouring tiles share source lines, ran the
// same or slower with it: config 2 in0 24.7-25.0 -> 27.8-28.0 us).
template <typename W, int VEC, bool HAS_OUTER, int U>
__global__ __launch_bounds__(kThreads) void gather_kernel(GatherArgs p) {
    const W* __restrict__ src = static_cast<const W*>(p.src);
    W* __restrict__ dst = static_cast<W*>(p.dst);
    const uint32_t stride = gridDim.x * kThreads;
    for (uint32_t v0 = blockIdx.x * kThreads + threadIdx.x; v0 < p.nvec; v0 += stride * U) {
        int64_t off[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t v = v0 + u * stride;
            if constexpr (HAS_OUTER) {
                uint32_t row, colv;
                p.inner_vecs.divmod(v, row, colv);
                off[u] = int64_t(colv) * VEC * p.inner_stride;
                for (int d = p.nouter - 1; d >= 0; --d) {
                    uint32_t q, r;
                    p.outer_div[d].divmod(row, q, r);
                    off[u] += int64_t(r) * p.outer_stride[d];
                    row = q;
                }
            } else {
                off[u] = int64_t(v) * VEC * p.inner_stride;
            }
        }
        if constexpr (VEC > 1) {
            u32x4 x[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (v0 + u * stride < p.nvec)
                    x[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + off[u]));
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (v0 + u * stride < p.nvec)
                    put(reinterpret_cast<u32x4*>(dst + int64_t(v0 + u * stride) * VEC), x[u], p.nt);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (v0 + u * stride < p.nvec) dst[v0 + u * stride] = src[off[u]];
        }
    }
}

struct TileArgs {
    const void* src;
    void* dst;
    int64_t P, Q;            // extents of the source-contiguous axis p and the
                             // destination-innermost axis q
    int64_t src_q_stride;    // source stride of q (p has source stride 1)
    int64_t dst_p_stride;    // destination stride of p (q has destination stride 1)
    uint32_t tiles_p, tiles_q;
    int32_t nbatch;          // remaining axes, decoded from the batch index
    FastDiv batch_div[PE_MAX_DIMS];
    int64_t batch_src[PE_MAX_DIMS];
    int64_t batch_dst[PE_MAX_DIMS];
    uint32_t nbatch_total;
    int32_t nt;
};

// Tile edge: 64 elements, or 32 for float32 where the rule below picks it
// (PE_TILE_SMALL_F32: 0 never, 1 when destination rows are not 16-byte
// vectors, 2 always).
#ifndef PE_TILE_SMALL_F32
#define PE_TILE_SMALL_F32 1
#endif

// Float16 tile extents along p and q.
#ifndef PE_TILE_F16_P
#define PE_TILE_F16_P 64
#endif
#ifndef PE_TILE_F16_Q
#define PE_TILE_F16_Q 64
#endif
template <typename W>
int tile_edge(bool vstore) {
    if (sizeof(W) != 4) return 64;
    return (PE_TILE_SMALL_F32 == 2 || (PE_TILE_SMALL_F32 == 1 && !vstore)) ? 32 : 64;
}

// Permutation outputs from this size on are written with non-temporal
// stores.  Lower than the GEMM / product threshold: a 67 MB gather ran 6 %
// faster with them and a 67 MB tile transpose 3 % (cold operands), while a
// 64 MB GEMM output or product ran 7-13 % slower; a staged einsum whose GEMM
// reads the gathered operand right after was unchanged.
#ifndef PE_PERMUTE_NT_MIN_BYTES
#define PE_PERMUTE_NT_MIN_BYTES (32ll << 20)
#endif

// Tile-transpose blocks per CU in the grid (each walks tiles beyond that):
// one tile per block up to 64 per CU, so a block's next tile never waits
// for its last tile's stores (memory counters complete in issue order).
// Config 2 in0 (12,800 32x32 tiles, one MI355X): 24.5-24.7 us at 32 per CU,
// 24.2-24.3 at 64, 24.1-24.2 at 128; config 3 in1 unchanged.
#ifndef PE_TILE_GRID_PER_CU
#define PE_TILE_GRID_PER_CU 64
#endif

// One 64x64 tile per block iteration.  With VLOAD the reads are 16-byte
// vectors along p (source-contiguous), else one element per lane with the
// lanes along p; with VSTORE the writes are 16-byte vectors along q
// (destination-contiguous), else one element per lane with the lanes along q.
// The LDS tile has one padding element per row, so the row-wise accesses of
// one side and the column-wise accesses of the other both spread over all
// banks.  Tiles are walked diagonally (the q-tile index is offset by the
// p-tile index), so concurrently running blocks do not all write rows that
// are a large power of two apart in the same column range.
template <typename W, bool VLOAD, bool VSTORE, int TP = 64, int TQ = TP>
__global__ __launch_bounds__(kThreads) void tile_transpose_kernel(TileArgs p) {
    constexpr int VEC = 16 / sizeof(W);
    constexpr int LVPR = VLOAD ? TP / VEC : TP;   // lanes per tile row, read side
    constexpr int LW = VLOAD ? VEC : 1;                  // elements per lane access, read
    constexpr int SVPR = VSTORE ? TQ / VEC : TQ;  // lanes per tile row, write side
    constexpr int SW = VSTORE ? VEC : 1;
    static_assert(TQ % (kThreads / LVPR) == 0 && TP % (kThreads / SVPR) == 0 && TQ >= kThreads / LVPR &&
                  TP >= kThreads / SVPR, "tile rows must split evenly over the block's passes");
    __shared__ W tile[TQ][TP + 1];  // tile[q][p]
    const W* __restrict__ src = static_cast<const W*>(p.src);
    W* __restrict__ dst = static_cast<W*>(p.dst);
    const uint32_t tiles_per_batch = p.tiles_p * p.tiles_q;
    const uint32_t total = tiles_per_batch * p.nbatch_total;
    const int lc = threadIdx.x % LVPR, lr = threadIdx.x / LVPR;
    const int sc = threadIdx.x % SVPR, sr = threadIdx.x / SVPR;
    for (uint32_t t = blockIdx.x; t < total; t += gridDim.x) {
        uint32_t bidx = t / tiles_per_batch;
        const uint32_t rem = t - bidx * tiles_per_batch;
        const uint32_t tp = rem % p.tiles_p;
        uint32_t tq = rem / p.tiles_p + tp;
        tq = tq % p.tiles_q;
        int64_t sbase = 0, dbase = 0;
        for (int d = p.nbatch - 1; d >= 0; --d) {
            uint32_t q, r;
            p.batch_div[d].divmod(bidx, q, r);
            sbase += int64_t(r) * p.batch_src[d];
            dbase += int64_t(r) * p.batch_dst[d];
            bidx = q;
        }
        const int64_t p0 = int64_t(tp) * TP, q0 = int64_t(tq) * TQ;
        // Read: tile rows are q, each lane covers LW consecutive p.
#pragma unroll
        for (int it = 0; it < TQ / (kThreads / LVPR); ++it) {
            const int r = lr + it * (kThreads / LVPR);
            const int64_t gq = q0 + r, gp = p0 + lc * LW;
            if (gq >= p.Q) continue;
            const W* s = src + sbase + gq * p.src_q_stride + gp;
            if (VLOAD && gp + LW <= p.P) {
                Chunk<W, LW> x = *reinterpret_cast<const Chunk<W, LW>*>(s);
#pragma unroll
                for (int j = 0; j < LW; ++j) tile[r][lc * LW + j] = x.v[j];
            } else {
#pragma unroll
                for (int j = 0; j < LW; ++j)
                    if (gp + j < p.P) tile[r][lc * LW + j] = s[j];
            }
        }
        __syncthreads();
        // Write: destination rows are p, each lane covers SW consecutive q.
#pragma unroll
        for (int it = 0; it < TP / (kThreads / SVPR); ++it) {
            const int r = sr + it * (kThreads / SVPR);
            const int64_t gp = p0 + r, gq = q0 + sc * SW;
            if (gp >= p.P) continue;
            W* d = dst + dbase + gp * p.dst_p_stride + gq;
            if (VSTORE && gq + SW <= p.Q) {
                Chunk<W, SW> x;
#pragma unroll
                for (int j = 0; j < SW; ++j) x.v[j] = tile[sc * SW + j][r];
                if constexpr (VSTORE)
                    put(reinterpret_cast<u32x4*>(d), *reinterpret_cast<const u32x4*>(&x), p.nt);
            } else {
#pragma unroll
                for (int j = 0; j < SW; ++j)
                    if (gq + j < p.Q) d[j] = tile[sc * SW + j][r];
            }
        }
        __syncthreads();
    }
}

// Wide fallback (2^31+ elements): one element per thread, 64-bit decode.
template <typename W>
__global__ __launch_bounds__(kThreads) void gather_wide_kernel(const W* __restrict__ src,
                                                               W* __restrict__ dst, int64_t n,
                                                               pe_permute_desc d) {
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    for (int64_t o = int64_t(blockIdx.x) * kThreads + threadIdx.x; o < n; o += stride) {
        int64_t rem = o, off = 0;
        for (int k = d.ndims - 1; k >= 0; --k) {
            off += (rem % d.shape[k]) * d.src_stride[k];
            rem /= d.shape[k];
        }
        dst[o] = src[off];
    }
}

int grid_cap(int64_t blocks, int per_cu = 16) {
    int64_t cap = int64_t(cu_count()) * per_cu;
    return int(std::max<int64_t>(1, std::min(blocks, cap)));
}

template <typename W, int TP, int TQ>
void launch_tile(bool vload, bool vstore, dim3 grid, hipStream_t s, const TileArgs& t) {
    if (vload && vstore) hipLaunchKernelGGL((tile_transpose_kernel<W, true, true, TP, TQ>), grid, dim3(kThreads), 0, s, t);
    else if (vload) hipLaunchKernelGGL((tile_transpose_kernel<W, true, false, TP, TQ>), grid, dim3(kThreads), 0, s, t);
    else if (vstore) hipLaunchKernelGGL((tile_transpose_kernel<W, false, true, TP, TQ>), grid, dim3(kThreads), 0, s, t);
    else hipLaunchKernelGGL((tile_transpose_kernel<W, false, false, TP, TQ>), grid, dim3(kThreads), 0, s, t);
}

template <typename W>
int run(const pe_permute_desc& d, const void* src, void* dst, hipStream_t s) {
    // Merge destination-adjacent axes that are also source-adjacent.
    std::vector<int64_t> shape, sst;
    for (int k = 0; k < d.ndims; ++k) {
        if (d.shape[k] == 1) continue;
        if (!shape.empty() && sst.back() == d.shape[k] * d.src_stride[k]) {
            shape.back() *= d.shape[k];
            sst.back() = d.src_stride[k];
        } else {
            shape.push_back(d.shape[k]);
            sst.push_back(d.src_stride[k]);
        }
    }
    int64_t n = 1;
    for (int64_t x : shape) n *= x;
    if (n == 0) return PE_OK;
    const int nd = int(shape.size());
    if (n >= (int64_t(1) << 31)) {
        pe_permute_desc m = d;
        m.ndims = nd;
        for (int k = 0; k < nd; ++k) { m.shape[k] = shape[k]; m.src_stride[k] = sst[k]; }
        hipLaunchKernelGGL((gather_wide_kernel<W>), dim3(grid_cap(ceil_div(n, kThreads))),
                           dim3(kThreads), 0, s, (const W*)src, (W*)dst, n, m);
        PE_CHECK_HIP(hipGetLastError());
        return PE_OK;
    }
    // Destination row-major strides of the merged axes.
    std::vector<int64_t> dst_stride(nd, 1);
    for (int k = nd - 2; k >= 0; --k) dst_stride[k] = dst_stride[k + 1] * shape[k + 1];

    int pax = -1;  // merged axis with source stride 1
    for (int k = 0; k < nd; ++k)
        if (sst[k] == 1) pax = k;
    const bool inner_kept = nd == 0 || sst[nd - 1] == 1;

    if (inner_kept || pax < 0) {
        GatherArgs a{};
        a.src = src; a.dst = dst;
        const int64_t inner = nd ? shape[nd - 1] : 1;
        a.inner_stride = nd ? sst[nd - 1] : 0;
        a.nouter = std::max(0, nd - 1);
        for (int k = 0; k < a.nouter; ++k) {
            a.outer_div[k].init(uint32_t(shape[k]));
            a.outer_stride[k] = sst[k];
        }
        constexpr int VEC = 16 / sizeof(W);
        constexpr int U = PE_GATHER_UNROLL;
        a.nt = nt_mode(n * int64_t(sizeof(W)), PE_PERMUTE_NT_MIN_BYTES);
        bool vec = inner_kept && nd > 0 && inner % VEC == 0 && aligned(src, 16) && aligned(dst, 16);
        for (int k = 0; k < a.nouter && vec; ++k) vec = sst[k] % VEC == 0;
        const bool outer = a.nouter > 0;
        const int per_cu = PE_GATHER_GRID_PER_CU;
        if (vec && (a.nt || PE_GATHER_FLAT)) {
            // One vector per thread in a grid of blocks dispatched in address
            // order, so the blocks in flight read and write one compact
            // window of HBM.  Measured on MI355X: 1 GiB copy 4.99 -> 6.37
            // TB/s, config 3's output permutation (2.15 GB) 923 -> 714 us,
            // against the persistent grid-stride stream below, whose
            // drifting blocks scatter their writes over many DRAM pages.
            a.nvec = uint32_t(n / VEC);
            a.inner_vecs.init(uint32_t(inner / VEC));
            const int grid = int(ceil_div(a.nvec, kThreads));
            if (outer) hipLaunchKernelGGL((gather_kernel<W, VEC, true, 1>), dim3(grid), dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((gather_kernel<W, VEC, false, 1>), dim3(grid), dim3(kThreads), 0, s, a);
        } else if (vec) {
            a.nvec = uint32_t(n / VEC);
            a.inner_vecs.init(uint32_t(inner / VEC));
            int grid = grid_cap(ceil_div(ceil_div(a.nvec, U), kThreads), per_cu);
            if (outer) hipLaunchKernelGGL((gather_kernel<W, VEC, true, U>), dim3(grid), dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((gather_kernel<W, VEC, false, U>), dim3(grid), dim3(kThreads), 0, s, a);
        } else {
            a.nvec = uint32_t(n);
            a.inner_vecs.init(uint32_t(inner));
            int grid = grid_cap(ceil_div(ceil_div(a.nvec, 4), kThreads), per_cu);
            if (outer) hipLaunchKernelGGL((gather_kernel<W, 1, true, 4>), dim3(grid), dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((gather_kernel<W, 1, false, 4>), dim3(grid), dim3(kThreads), 0, s, a);
        }
        PE_CHECK_HIP(hipGetLastError());
        return PE_OK;
    }

    // Tiled transpose between axis q = nd-1 (destination-contiguous) and pax.
    const int qax = nd - 1;
    TileArgs t{};
    t.src = src; t.dst = dst;
    t.P = shape[pax]; t.Q = shape[qax];
    t.src_q_stride = sst[qax];
    t.dst_p_stride = dst_stride[pax];
    const int edge = tile_edge<W>(aligned(dst, 16) && t.dst_p_stride % (16 / int(sizeof(W))) == 0);
    // The small tile spans q with 64 where that covers q in one tile
    // ([64, 37, 4000] -> (0, 2, 1): 27.3 -> 19.1 us; 32 x 64 and 64 x 32
    // tiles were otherwise equal or slower than 32 x 32).
    const int tp = sizeof(W) == 2 ? PE_TILE_F16_P : edge;
    const int tq = sizeof(W) == 2 ? PE_TILE_F16_Q : (edge == 32 && t.Q > 32 && t.Q <= 64 ? 64 : edge);
    t.tiles_p = uint32_t(ceil_div(t.P, tp));
    t.tiles_q = uint32_t(ceil_div(t.Q, tq));
    int nb = 0;
    int64_t nbt = 1;
    for (int k = 0; k < nd; ++k) {
        if (k == pax || k == qax) continue;
        t.batch_div[nb].init(uint32_t(shape[k]));
        t.batch_src[nb] = sst[k];
        t.batch_dst[nb] = dst_stride[k];
        nbt *= shape[k];
        ++nb;
    }
    t.nbatch = nb;
    t.nbatch_total = uint32_t(nbt);
    t.nt = nt_mode(n * int64_t(sizeof(W)), PE_PERMUTE_NT_MIN_BYTES);
    constexpr int VEC = 16 / sizeof(W);
    bool vload = aligned(src, 16) && t.src_q_stride % VEC == 0;
    bool vstore = aligned(dst, 16) && t.dst_p_stride % VEC == 0;
    for (int k = 0; k < nb; ++k) {
        vload = vload && t.batch_src[k] % VEC == 0;
        vstore = vstore && t.batch_dst[k] % VEC == 0;
    }
    int64_t tiles = int64_t(t.tiles_p) * t.tiles_q * nbt;
    const dim3 grid(grid_cap(tiles, PE_TILE_GRID_PER_CU));
    if constexpr (sizeof(W) == 4) {
        if (tp == 32 && tq == 64) launch_tile<W, 32, 64>(vload, vstore, grid, s, t);
        else if (tp == 32) launch_tile<W, 32, 32>(vload, vstore, grid, s, t);
        else launch_tile<W, 64, 64>(vload, vstore, grid, s, t);
    } else {
        launch_tile<W, PE_TILE_F16_P, PE_TILE_F16_Q>(vload, vstore, grid, s, t);
    }
    PE_CHECK_HIP(hipGetLastError());
    return PE_OK;
}

}  // namespace

int validate_permute(const pe_permute_desc& d) {
    if (d.elem_bytes != 2 && d.elem_bytes != 4)
        return fail(PE_ERR_UNSUPPORTED, "permute: elem_bytes must be 2 or 4");
    if (d.ndims < 0 || d.ndims > PE_MAX_DIMS) return fail(PE_ERR_INVALID, "permute: ndims out of range");
    int64_t n = 1, smax = 0;
    for (int k = 0; k < d.ndims; ++k) {
        if (d.shape[k] < 0 || d.src_stride[k] < 0)
            return fail(PE_ERR_INVALID, "permute: negative extent or stride");
        n *= d.shape[k];
        if (d.shape[k] > 0) smax += (d.shape[k] - 1) * d.src_stride[k];
    }
    if (n > 0 && smax >= d.src_numel)
        return fail(PE_ERR_BOUNDS, "permute: strides address past the source extent");
    return PE_OK;
}

}  // namespace pe

extern "C" int pe_permute(const pe_permute_desc* d, const void* src, void* dst, void* stream) {
    if (!d) return pe::fail(PE_ERR_INVALID, "permute: null descriptor");
    int st = pe::validate_permute(*d);
    if (st != PE_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return d->elem_bytes == 4 ? pe::run<uint32_t>(*d, src, dst, s) : pe::run<uint16_t>(*d, src, dst, s);
}
