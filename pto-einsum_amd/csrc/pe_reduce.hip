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
// One thread per output element, summing its terms in row-major order of the
// reduced index from +0: the sequential loop, so results are deterministic
// and independent of the launch shape.  The reduced index advances as an
// odometer (one add per term, a carry at each axis wrap).  HBM-bound for
// large outputs; a reduction over many terms with few outputs runs on few
// threads (the path is opt-in and not tuned for that shape).
#include "pe_common.h"

#include <algorithm>
#include <string>

namespace pe {
namespace {

struct ReduceAxesArgs {
    const void* src;
    float* dst;
    int64_t nout;                 // product of keep_shape
    int64_t nterm;                // product of red_shape
    int32_t nkeep, nred;
    int64_t keep_shape[PE_MAX_DIMS], keep_stride[PE_MAX_DIMS];
    int64_t red_shape[PE_MAX_DIMS], red_stride[PE_MAX_DIMS];
};

template <typename E>
__global__ __launch_bounds__(256) void reduce_axes_kernel(ReduceAxesArgs a) {
    const auto* src = static_cast<const typename E::T*>(a.src);
    const int64_t step = int64_t(gridDim.x) * 256;
    for (int64_t o = int64_t(blockIdx.x) * 256 + threadIdx.x; o < a.nout; o += step) {
        // Source offset of the output element: row-major decode of o.
        int64_t rem = o, base = 0;
#pragma unroll
        for (int d = PE_MAX_DIMS - 1; d >= 0; --d) {
            if (d < a.nkeep) {
                const int64_t q = rem / a.keep_shape[d];
                base += (rem - q * a.keep_shape[d]) * a.keep_stride[d];
                rem = q;
            }
        }
        int64_t idx[PE_MAX_DIMS];
#pragma unroll
        for (int e = 0; e < PE_MAX_DIMS; ++e) idx[e] = 0;
        float acc = 0.0f;
        int64_t off = base;
        for (int64_t t = 0; t < a.nterm; ++t) {
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
        a.dst[o] = acc;
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
    const int grid = int(std::max<int64_t>(1, std::min<int64_t>(ceil_div(a.nout, 256), int64_t(cu_count()) * 16)));
    if (d->dtype == PE_F16)
        hipLaunchKernelGGL(reduce_axes_kernel<F16>, dim3(grid), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(reduce_axes_kernel<F32>, dim3(grid), dim3(256), 0, s, a);
    PE_CHECK_HIP(hipGetLastError());
    return PE_OK;
}
