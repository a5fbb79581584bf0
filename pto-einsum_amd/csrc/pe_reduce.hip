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
// Summation order, a function of (nout, nterm) only, so results are
// deterministic and independent of the launch shape and the device:
//   * the nterm terms of an output, in row-major order of the reduced index,
//     are cut into C contiguous chunks, the first nterm % C of them one term
//     longer than the rest;
//   * each chunk is summed in order from +0, then the C partial sums are added
//     in chunk order from +0;
//   * C = 1 (the plain sequential loop) when nterm <= kChunkTerms or
//     nout >= kWideOutputs, else min(kChunkThreads, ceil(nterm / kChunkTerms)).
// C = 1 runs one thread per output (coalesced over the output axes, enough
// threads to fill the chip); C > 1 runs one block per output, one thread per
// chunk, for reductions with few outputs and many terms.  Both are HBM-bound;
// the reduced index advances as an odometer (one add per term, a carry at each
// axis wrap).
#include "pe_common.h"

#include <algorithm>
#include <string>

namespace pe {
namespace {

constexpr int64_t kChunkTerms = 256;     // shortest chunk worth a thread of its own
constexpr int64_t kWideOutputs = 32768;  // outputs enough to fill the chip one thread each
constexpr int kChunkThreads = 256;       // chunks per output at most = block size

struct ReduceAxesArgs {
    const void* src;
    float* dst;
    int64_t nout;                 // product of keep_shape
    int64_t nterm;                // product of red_shape
    int32_t nkeep, nred;
    int64_t keep_shape[PE_MAX_DIMS], keep_stride[PE_MAX_DIMS];
    int64_t red_shape[PE_MAX_DIMS], red_stride[PE_MAX_DIMS];
};

// Source offset of output element o: row-major decode over keep_shape.
__device__ __forceinline__ int64_t keep_offset(const ReduceAxesArgs& a, int64_t o) {
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

// Sum of terms [t0, t1) of the output at source offset base, in order from +0.
template <typename E>
__device__ __forceinline__ float sum_terms(const ReduceAxesArgs& a, int64_t base, int64_t t0, int64_t t1) {
    const auto* src = static_cast<const typename E::T*>(a.src);
    int64_t idx[PE_MAX_DIMS];
    int64_t off = base, rem = t0;
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
    float acc = 0.0f;
    for (int64_t t = t0; t < t1; ++t) {
        acc = acc + E::to_f32(src[off]);
        // Next r in row-major order: the last axis moves fastest.
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
    return acc;
}

template <typename E>
__global__ __launch_bounds__(256) void reduce_axes_kernel(ReduceAxesArgs a) {
    const int64_t step = int64_t(gridDim.x) * 256;
    for (int64_t o = int64_t(blockIdx.x) * 256 + threadIdx.x; o < a.nout; o += step)
        a.dst[o] = sum_terms<E>(a, keep_offset(a, o), 0, a.nterm);
}

// One block per output (grid-stride over outputs), thread c sums chunk c.
template <typename E>
__global__ __launch_bounds__(kChunkThreads) void reduce_axes_chunked_kernel(ReduceAxesArgs a, int32_t nchunk) {
    __shared__ float part[kChunkThreads];
    const int c = threadIdx.x;
    const int64_t q = a.nterm / nchunk, r = a.nterm % nchunk;
    const int64_t t0 = c * q + std::min<int64_t>(c, r);
    const int64_t t1 = t0 + q + (c < r ? 1 : 0);
    for (int64_t o = blockIdx.x; o < a.nout; o += gridDim.x) {
        part[c] = c < nchunk ? sum_terms<E>(a, keep_offset(a, o), t0, t1) : 0.0f;
        __syncthreads();
        if (c == 0) {
            float s = 0.0f;
            for (int i = 0; i < nchunk; ++i) s = s + part[i];
            a.dst[o] = s;
        }
        __syncthreads();  // part[] is rewritten for the next output
    }
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

}  // namespace
}  // namespace pe

extern "C" int pe_reduce_axes(const pe_reduce_desc* d, const void* src, float* dst, void* stream) {
    using namespace pe;
    if (!d) return fail(PE_ERR_INVALID, "reduce_axes: null descriptor");
    const int st = validate(*d);
    if (st != PE_OK) return st;
    ReduceAxesArgs a{};
    a.src = src;
    a.dst = dst;
    a.nkeep = d->nkeep;
    a.nred = d->nred;
    a.nout = 1;
    a.nterm = 1;
    for (int i = 0; i < d->nkeep; ++i) {
        a.keep_shape[i] = d->keep_shape[i];
        a.keep_stride[i] = d->keep_stride[i];
        a.nout *= d->keep_shape[i];
    }
    for (int i = 0; i < d->nred; ++i) {
        a.red_shape[i] = d->red_shape[i];
        a.red_stride[i] = d->red_stride[i];
        a.nterm *= d->red_shape[i];
    }
    if (a.nout == 0) return PE_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f16 = d->dtype == PE_F16;
    if (a.nterm > kChunkTerms && a.nout < kWideOutputs) {
        const int32_t nchunk = int32_t(std::min<int64_t>(kChunkThreads, ceil_div(a.nterm, kChunkTerms)));
        const int grid = int(std::min<int64_t>(a.nout, int64_t(cu_count()) * 8));
        if (f16)
            hipLaunchKernelGGL(reduce_axes_chunked_kernel<F16>, dim3(grid), dim3(kChunkThreads), 0, s, a, nchunk);
        else
            hipLaunchKernelGGL(reduce_axes_chunked_kernel<F32>, dim3(grid), dim3(kChunkThreads), 0, s, a, nchunk);
    } else {
        const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(a.nout, 256), int64_t(cu_count()) * 16)));
        if (f16)
            hipLaunchKernelGGL(reduce_axes_kernel<F16>, dim3(grid), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(reduce_axes_kernel<F32>, dim3(grid), dim3(256), 0, s, a);
    }
    PE_CHECK_HIP(hipGetLastError());
    return PE_OK;
}
