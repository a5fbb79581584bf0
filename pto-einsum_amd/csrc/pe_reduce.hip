// Sum over the solo axes of one einsum operand (an index found in that
// operand only and not in the output), into a contiguous float32 tensor over
// the remaining axes.
//
// The reference rejects equations with such axes (builder.py:218-229); its
// roadmap (IMPLEMENTATION.md:812-821, "Option A") reduces them on the owning
// operand before the transpose -> matmul pipeline, which is what this kernel
// is for: the reduced operand then enters the ordinary contraction.  With no
// axis to reduce it converts an operand to float32 (the other operand of a
// float16 einsum whose first operand was reduced to float32).
//
// Summation order.  It depends on the shapes, on whether the reduced axes
// form one contiguous run, on 16-byte alignment and on the dtype -- never on
// the launch or the device -- so results are deterministic.  With V, L and C
// as chosen below (pe_reduce_order reports them):
//   * the nterm terms of an output, row-major over the reduced index, form
//     G = ceil(nterm / V) groups of V consecutive terms (the last may be
//     shorter);
//   * the groups are cut into C contiguous chunks, the first G % C of them one
//     group longer;
//   * within a chunk, lane l of L sums the groups l, l + L, l + 2L, ... term
//     by term in order, from +0;
//   * the L lane sums, then the C chunk sums, are combined by a pairwise tree:
//     for s = 1, 2, 4, ...: p[i] = p[i] + p[i + s] for i a multiple of 2s with
//     i + s in range; the result is p[0].
// Two layouts of the work:
//   row mode (the reduced axes merge into one run of stride 1 with at least
//     kRowMinTerms terms): L lanes per (output, chunk), V = 16 bytes of
//     elements when every output's run starts 16-byte aligned, else 1; L = 64
//     halved (down to 4) while L x kLaneGroups > G, so that short runs share
//     a wave -- a lane reads V consecutive terms, its segment L x V;
//   column mode (all other cases): L = V = 1, one lane per output and chunk,
//     the 64 lanes of a wave on 64 consecutive outputs (coalesced when an
//     output axis is the contiguous one), the terms' offsets (the same for
//     every lane) advancing as a scalar odometer.
// C is chosen for about kTargetWaves waves, each chunk at least a few steps
// long; with C > 1 the chunk sums go through the caller's workspace and a
// second kernel combines them.  Both passes are HBM-bound.
#include "pe_common.h"

#include <algorithm>
#include <string>

namespace pe {
namespace {

constexpr int64_t kRowMinTerms = 32;    // shortest run read along the run
constexpr int64_t kLaneGroups = 4;      // row mode: L shrinks until each lane has this many groups
constexpr int64_t kTargetWaves = 4096;  // waves of the first pass (16 per CU)
constexpr int64_t kMaxChunks = 4096;    // chunk sums per output (LDS of the tree pass)

// Load type of one group of V elements.
template <typename T, int V> struct GroupOf { using type = T; };
template <> struct GroupOf<float, 4> { using type = f32x4; };
template <> struct GroupOf<_Float16, 8> { using type = f16x8; };

struct RedArgs {
    const void* src;
    float* dst;
    float* ws;                    // C x nout chunk sums when C > 1
    int64_t nout, nterm;
    int64_t G, C;                 // groups per output, chunks per output
    int32_t L;                    // row mode: lanes per (output, chunk), a power of two <= 64
    int32_t nkeep, nred;          // after merging
    int64_t keep_shape[PE_MAX_DIMS], keep_stride[PE_MAX_DIMS];
    int64_t red_shape[PE_MAX_DIMS], red_stride[PE_MAX_DIMS];
};

// Source offset of output element o: row-major decode over keep_shape.
__device__ __forceinline__ int64_t keep_offset(const RedArgs& a, int64_t o) {
    int64_t rem = o, base = 0;
#pragma unroll
    for (int d = PE_MAX_DIMS - 1; d >= 0; --d) {
        if (d < a.nkeep) {
            const int64_t q = rem / a.keep_shape[d];
            base += (rem - q * a.keep_shape[d]) * a.keep_stride[d];
            rem = q;
        }
    }
    return base;
}

__device__ __forceinline__ void chunk_range(int64_t n, int64_t C, int64_t c, int64_t& b, int64_t& e) {
    const int64_t q = n / C, r = n % C;
    b = c * q + (c < r ? c : r);
    e = b + q + (c < r ? 1 : 0);
}

__device__ __forceinline__ void put(const RedArgs& a, int64_t o, int64_t c, float v) {
    if (a.C == 1) a.dst[o] = v;
    else a.ws[c * a.nout + o] = v;
}

// Row mode: L consecutive lanes (an aligned segment of the wave) per
// (output, chunk); lane l of a segment sums groups l, l + L, ...  Every
// source element is read once.  NT: non-temporal loads, taken where one load
// of a segment covers whole 128-byte lines (L x V x element size >= 128);
// measured on MI355X: [64, 4000000] 177 -> 160 us, [1024, 250000] 177-179 ->
// 159-160, float16 [1024, 250000] 95-96 -> 85.5-86, [16384, 16000] 181-184
// -> 162-163, [262144, 1024] 180-181 -> 165-166, [1000000, 256] 169-173 ->
// 153.5 us; with segments of half a line ([8000000, 32]: 4 lanes x 16
// bytes) 215 -> 259 us, the line evicted between its two halves' loads.
template <typename E, int V, bool NT>
__global__ __launch_bounds__(256) void reduce_row_kernel(RedArgs a) {
    using T = typename E::T;
    const int L = a.L;
    const int64_t tid = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int lane = int(tid & (L - 1));
    const int64_t item = tid / L;
    // Segments past the end stay in step (their lanes take part in the
    // shuffles below) but read and write nothing.
    const bool live = item < a.nout * a.C;
    const int64_t o = live ? item / a.C : 0, c = live ? item - o * a.C : 0;
    int64_t g0 = 0, g1 = 0;
    if (live) chunk_range(a.G, a.C, c, g0, g1);
    const T* p = static_cast<const T*>(a.src) + keep_offset(a, o);
    float acc = 0.0f;
    int64_t g = g0 + lane;
    // Whole groups, four in flight per lane (loads first, then the adds in
    // order).
    using Vec = typename GroupOf<T, V>::type;
    constexpr int U = 4;
    for (; g + (U - 1) * L < g1 && (g + (U - 1) * L + 1) * V <= a.nterm; g += U * L) {
        Vec x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const Vec* q = reinterpret_cast<const Vec*>(p + (g + u * L) * V);
            if constexpr (NT) x[u] = __builtin_nontemporal_load(q);
            else x[u] = *q;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (V == 1) {
                acc = acc + E::to_f32(x[u]);
            } else {
#pragma unroll
                for (int v = 0; v < V; ++v) acc = acc + E::to_f32(x[u][v]);
            }
        }
    }
    // Whole groups one at a time, then the last (partial) group term by term.
    for (; g < g1 && (g + 1) * V <= a.nterm; g += L) {
        const Vec* q = reinterpret_cast<const Vec*>(p + g * V);
        Vec x;
        if constexpr (NT) x = __builtin_nontemporal_load(q);
        else x = *q;
        if constexpr (V == 1) {
            acc = acc + E::to_f32(x);
        } else {
#pragma unroll
            for (int v = 0; v < V; ++v) acc = acc + E::to_f32(x[v]);
        }
    }
    if (g < g1) {
        for (int64_t t = g * V; t < a.nterm; ++t) acc = acc + E::to_f32(p[t]);
    }
    // Pairwise tree over the segment's L lanes: after the step with offset s,
    // lane i holds the sum of the lanes of its aligned 2s block (addition is
    // commutative, so both partners hold the same value; s < L keeps every
    // exchange inside the segment).
    for (int s = 1; s < L; s <<= 1) acc = acc + __shfl_xor(acc, s, 64);
    if (live && lane == 0) put(a, o, c, acc);
}

// Column mode: one lane per (output, chunk), 64 consecutive outputs per wave;
// the unrolled loop's loads (a wave reads 64 consecutive elements per term)
// are non-temporal ([4000000, 64] summed over axis 0: 186-187 -> 167 us on
// MI355X).
template <typename E>
__global__ __launch_bounds__(256) void reduce_col_kernel(RedArgs a, int64_t ngroups) {
    using T = typename E::T;
    const int lane = threadIdx.x & 63;
    const int64_t item = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= ngroups * a.C) return;   // whole waves
    const int64_t c = item / ngroups, og = item - c * ngroups;
    const int64_t o = og * 64 + lane;
    const bool live = o < a.nout;
    int64_t t0, t1;
    chunk_range(a.nterm, a.C, c, t0, t1);
    const T* p = static_cast<const T*>(a.src) + (live ? keep_offset(a, o) : 0);
    float acc = 0.0f;
    if (a.nred == 1) {
        const int64_t rs = a.red_stride[0];
        int64_t t = t0;
        constexpr int U = 8;
        for (; t + U <= t1; t += U) {
            T x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = live ? __builtin_nontemporal_load(p + (t + u) * rs) : T(0);
#pragma unroll
            for (int u = 0; u < U; ++u) acc = acc + E::to_f32(x[u]);
        }
        for (; t < t1; ++t) acc = acc + E::to_f32(live ? p[t * rs] : T(0));
    } else if (t1 > t0) {
        // Odometer over the reduced axes (the same offsets for every lane).
        int64_t idx[PE_MAX_DIMS];
        int64_t off = 0, rem = t0;
#pragma unroll
        for (int e = PE_MAX_DIMS - 1; e >= 0; --e) {
            idx[e] = 0;
            if (e < a.nred) {
                const int64_t q = rem / a.red_shape[e];
                idx[e] = rem - q * a.red_shape[e];
                off += idx[e] * a.red_stride[e];
                rem = q;
            }
        }
        for (int64_t t = t0; t < t1; ++t) {
            acc = acc + E::to_f32(live ? p[off] : T(0));
#pragma unroll
            for (int e = PE_MAX_DIMS - 1; e >= 0; --e) {
                if (e < a.nred) {
                    if (++idx[e] < a.red_shape[e]) {
                        off += a.red_stride[e];
                        break;
                    }
                    off -= (a.red_shape[e] - 1) * a.red_stride[e];
                    idx[e] = 0;
                }
            }
        }
    }
    if (live) put(a, o, c, acc);
}

// Second pass: the C chunk sums of an output, combined by the pairwise tree
// in LDS (one block per output, grid-stride over outputs).
__global__ __launch_bounds__(256) void reduce_tree_kernel(const float* ws, float* dst, int64_t nout, int32_t C) {
    __shared__ float buf[kMaxChunks];
    for (int64_t o = blockIdx.x; o < nout; o += gridDim.x) {
        for (int i = threadIdx.x; i < C; i += 256) buf[i] = ws[int64_t(i) * nout + o];
        __syncthreads();
        for (int s = 1; s < C; s <<= 1) {
            for (int i = threadIdx.x * 2 * s; i < C; i += 256 * 2 * s)
                if (i + s < C) buf[i] = buf[i] + buf[i + s];
            __syncthreads();
        }
        if (threadIdx.x == 0) dst[o] = buf[0];
        __syncthreads();  // buf is rewritten for the next output
    }
}

// No reduced axis over one contiguous, 16-byte aligned run: a plain
// conversion, VEC elements per lane (each +0 + x, as the order prescribes
// for a one-term sum, so -0 becomes +0 exactly as on the general path).
template <typename E, int VEC>
__global__ __launch_bounds__(256) void convert_kernel(const typename E::T* __restrict__ src, float* __restrict__ dst,
                                                       int64_t n) {
    using Vec = typename GroupOf<typename E::T, VEC>::type;
    const int64_t nv = n / VEC;
    const int64_t step = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < nv; i += step) {
        const Vec x = *reinterpret_cast<const Vec*>(src + i * VEC);
#pragma unroll
        for (int v = 0; v < VEC; v += 4) {
            const f32x4 w = {0.0f + E::to_f32(x[v]), 0.0f + E::to_f32(x[v + 1]), 0.0f + E::to_f32(x[v + 2]),
                             0.0f + E::to_f32(x[v + 3])};
            *reinterpret_cast<f32x4*>(dst + i * VEC + v) = w;
        }
    }
    for (int64_t i = nv * VEC + int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += step)
        dst[i] = 0.0f + E::to_f32(src[i]);
}

__global__ __launch_bounds__(256) void zero_kernel(float* dst, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) dst[i] = 0.0f;
}

int validate(const pe_reduce_desc& d) {
    if (d.dtype != PE_F32 && d.dtype != PE_F16) return fail(PE_ERR_UNSUPPORTED, "reduce_axes: dtype must be PE_F32 or PE_F16");
    if (d.nkeep < 0 || d.nkeep > PE_MAX_DIMS || d.nred < 0 || d.nred > PE_MAX_DIMS)
        return fail(PE_ERR_INVALID, "reduce_axes: nkeep / nred outside 0.." + std::to_string(PE_MAX_DIMS));
    if (d.reserved != 0) return fail(PE_ERR_INVALID, "reduce_axes: reserved field must be 0");
    int64_t last = 0;  // largest source offset read
    bool empty = false;
    for (int i = 0; i < d.nkeep; ++i) {
        if (d.keep_shape[i] < 0 || d.keep_stride[i] < 0) return fail(PE_ERR_INVALID, "reduce_axes: negative extent or stride");
        if (d.keep_shape[i] == 0) empty = true;
        else last += (d.keep_shape[i] - 1) * d.keep_stride[i];
    }
    for (int i = 0; i < d.nred; ++i) {
        if (d.red_shape[i] < 0 || d.red_stride[i] < 0) return fail(PE_ERR_INVALID, "reduce_axes: negative extent or stride");
        if (d.red_shape[i] == 0) empty = true;
        else last += (d.red_shape[i] - 1) * d.red_stride[i];
    }
    if (!empty && last >= d.src_numel) return fail(PE_ERR_BOUNDS, "reduce_axes: strides address past the source");
    return PE_OK;
}

// Merges adjacent axes that address like one (outer stride = inner extent x
// inner stride) and drops extent-1 axes; the row-major index order over the
// axes is unchanged.
int merge_axes(const int64_t* shape, const int64_t* stride, int n, int64_t* mshape, int64_t* mstride) {
    int m = 0;
    for (int i = 0; i < n; ++i) {
        if (shape[i] == 1) continue;
        if (m > 0 && mstride[m - 1] == shape[i] * stride[i]) {
            mshape[m - 1] *= shape[i];
            mstride[m - 1] = stride[i];
        } else {
            mshape[m] = shape[i];
            mstride[m] = stride[i];
            ++m;
        }
    }
    return m;
}

struct RedPlan {
    RedArgs a;
    int mode;      // 0: zero fill (no terms), 1: row, 2: column, 3: contiguous conversion
    int V, L;
    int64_t ngroups;  // column mode: waves of outputs per chunk
};

RedPlan plan_reduce(const pe_reduce_desc& d, const void* src) {
    RedPlan p{};
    RedArgs& a = p.a;
    a.src = src;
    a.nkeep = merge_axes(d.keep_shape, d.keep_stride, d.nkeep, a.keep_shape, a.keep_stride);
    a.nred = merge_axes(d.red_shape, d.red_stride, d.nred, a.red_shape, a.red_stride);
    a.nout = 1;
    a.nterm = 1;
    for (int i = 0; i < d.nkeep; ++i) a.nout *= d.keep_shape[i];
    for (int i = 0; i < d.nred; ++i) a.nterm *= d.red_shape[i];
    const int64_t eb = d.dtype == PE_F16 ? 2 : 4;
    if (a.nterm == 0 || a.nout == 0) {
        // No terms (every output is +0) or no outputs (nothing to do).
        p.mode = 0;
        p.V = p.L = 1;
        a.G = 0;
        a.C = 1;
        return p;
    }
    if (a.nred == 1 && a.red_stride[0] == 1 && a.nterm >= kRowMinTerms) {
        p.mode = 1;
        p.L = 64;
        bool al = aligned(src, 16);
        for (int i = 0; i < a.nkeep; ++i) al = al && (a.keep_stride[i] * eb) % 16 == 0;
        p.V = al ? int(16 / eb) : 1;
        a.G = ceil_div(a.nterm, int64_t(p.V));
        while (p.L > 4 && p.L * kLaneGroups > a.G) p.L /= 2;
        a.L = p.L;
        const int64_t by_waves = ceil_div(kTargetWaves * (64 / p.L), a.nout);
        const int64_t by_len = std::max<int64_t>(1, a.G / (int64_t(p.L) * 8));  // each lane at least 8 groups
        a.C = std::max<int64_t>(1, std::min<int64_t>({by_waves, by_len, kMaxChunks}));
    } else if (a.nred == 0 && a.nkeep <= 1 && (a.nkeep == 0 || a.keep_stride[0] == 1) && aligned(src, 16)) {
        // Nothing to sum over one contiguous run: the conversion path (a
        // one-term sum, V = L = C = 1).
        p.mode = 3;
        p.V = p.L = 1;
        a.G = 1;
        a.C = 1;
    } else {
        p.mode = 2;
        p.V = p.L = 1;
        a.G = a.nterm;
        p.ngroups = ceil_div(a.nout, int64_t(64));
        const int64_t by_waves = ceil_div(kTargetWaves, p.ngroups);
        const int64_t by_len = std::max<int64_t>(1, a.nterm / 256);  // each chunk at least 256 terms
        a.C = std::max<int64_t>(1, std::min<int64_t>({by_waves, by_len, kMaxChunks}));
    }
    return p;
}

}  // namespace
}  // namespace pe

extern "C" int64_t pe_reduce_workspace_bytes(const pe_reduce_desc* d) {
    using namespace pe;
    if (!d || validate(*d) != PE_OK) return 0;
    // No source address here, so the size covers both alignments: a base that
    // is not 16-byte aligned takes one-element groups, hence more groups and
    // possibly more chunks than an aligned one.  (The planner only tests the
    // address for alignment; neither value is dereferenced.)
    int64_t bytes = 0;
    for (const void* src : {static_cast<const void*>(nullptr), reinterpret_cast<const void*>(uintptr_t(4))}) {
        const RedPlan p = plan_reduce(*d, src);
        if (p.a.C > 1) bytes = std::max<int64_t>(bytes, p.a.C * p.a.nout * int64_t(sizeof(float)));
    }
    return bytes;
}

extern "C" int pe_reduce_order(const pe_reduce_desc* d, const void* src, int64_t* order) {
    using namespace pe;
    if (!d || !order) return fail(PE_ERR_INVALID, "reduce_order: null argument");
    const int st = validate(*d);
    if (st != PE_OK) return st;
    const RedPlan p = plan_reduce(*d, src);
    order[0] = p.V;
    order[1] = p.L;
    order[2] = p.a.C;
    return PE_OK;
}

extern "C" int pe_reduce_axes(const pe_reduce_desc* d, const void* src, float* dst, void* ws, int64_t ws_bytes,
                              void* stream) {
    using namespace pe;
    if (!d) return fail(PE_ERR_INVALID, "reduce_axes: null descriptor");
    const int st = validate(*d);
    if (st != PE_OK) return st;
    RedPlan p = plan_reduce(*d, src);
    RedArgs& a = p.a;
    a.dst = dst;
    if (a.nout == 0) return PE_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int cus = cu_count();
    if (p.mode == 0) {
        // No terms: every output is the empty sum, +0 (a kernel, not a
        // memset, so the call stays capture-safe).
        const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(a.nout, 256), int64_t(cus) * 8)));
        hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(256), 0, s, dst, a.nout);
        PE_CHECK_HIP(hipGetLastError());
        return PE_OK;
    }
    if (a.C > 1) {
        if (!ws || ws_bytes < a.C * a.nout * int64_t(sizeof(float)))
            return fail(PE_ERR_WORKSPACE, "reduce_axes: workspace missing or smaller than pe_reduce_workspace_bytes");
        a.ws = static_cast<float*>(ws);
    }
    const bool f16 = d->dtype == PE_F16;
    if (p.mode == 3 && !aligned(dst, 16)) {
        // The same one-term sums through the lane-per-output path.
        p.mode = 2;
        p.ngroups = ceil_div(a.nout, int64_t(64));
    }
    if (p.mode == 3) {
        const int64_t nvec = ceil_div(a.nout, int64_t(8));
        const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(nvec, 256), int64_t(cus) * 16)));
        if (f16)
            hipLaunchKernelGGL((convert_kernel<F16, 8>), dim3(grid), dim3(256), 0, s,
                               static_cast<const _Float16*>(src), dst, a.nout);
        else
            hipLaunchKernelGGL((convert_kernel<F32, 4>), dim3(grid), dim3(256), 0, s, static_cast<const float*>(src),
                               dst, a.nout);
        PE_CHECK_HIP(hipGetLastError());
        return PE_OK;
    }
    if (p.mode == 1) {
        const int64_t blocks = ceil_div(a.nout * a.C * p.L, int64_t(256));
        if (blocks >= (int64_t(1) << 31)) return fail(PE_ERR_UNSUPPORTED, "reduce_axes: too many outputs");
        const dim3 grid{uint32_t(blocks)};
        const bool nt = int64_t(p.L) * p.V * (f16 ? 2 : 4) >= 128;
        if (f16) {
            if (p.V == 8) {
                if (nt) hipLaunchKernelGGL((reduce_row_kernel<F16, 8, true>), grid, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((reduce_row_kernel<F16, 8, false>), grid, dim3(256), 0, s, a);
            } else {
                if (nt) hipLaunchKernelGGL((reduce_row_kernel<F16, 1, true>), grid, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((reduce_row_kernel<F16, 1, false>), grid, dim3(256), 0, s, a);
            }
        } else {
            if (p.V == 4) {
                if (nt) hipLaunchKernelGGL((reduce_row_kernel<F32, 4, true>), grid, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((reduce_row_kernel<F32, 4, false>), grid, dim3(256), 0, s, a);
            } else {
                if (nt) hipLaunchKernelGGL((reduce_row_kernel<F32, 1, true>), grid, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((reduce_row_kernel<F32, 1, false>), grid, dim3(256), 0, s, a);
            }
        }
    } else {
        const int64_t blocks = ceil_div(p.ngroups * a.C, int64_t(4));
        if (blocks >= (int64_t(1) << 31)) return fail(PE_ERR_UNSUPPORTED, "reduce_axes: too many outputs");
        const dim3 grid{uint32_t(blocks)};
        if (f16) hipLaunchKernelGGL(reduce_col_kernel<F16>, grid, dim3(256), 0, s, a, p.ngroups);
        else hipLaunchKernelGGL(reduce_col_kernel<F32>, grid, dim3(256), 0, s, a, p.ngroups);
    }
    PE_CHECK_HIP(hipGetLastError());
    if (a.C > 1) {
        const int grid = int(std::max<int64_t>(1, std::min<int64_t>(a.nout, int64_t(cus) * 8)));
        hipLaunchKernelGGL(reduce_tree_kernel, dim3(grid), dim3(256), 0, s, a.ws, dst, a.nout, int32_t(a.C));
        PE_CHECK_HIP(hipGetLastError());
    }
    return PE_OK;
}
