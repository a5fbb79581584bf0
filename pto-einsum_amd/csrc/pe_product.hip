// Contraction-free products: Hadamard, broadcast, outer and transposed
// elementwise einsums, streamed over a row-major float32 output.
//
// Reference counterparts: elementwise_mul (pto_einsum_elementwise.h:27-127)
// and broadcast_mul (pto_einsum_elementwise.h:152-370).  Both are one kernel
// here: every operand is addressed through per-axis strides (stride 0 where
// the operand lacks the axis), so the same launch covers the reference's
// Hadamard, column-expand and scalar broadcast modes and the outer products
// the reference sends to its matmul path.
//
// Numerics follow the reference CPU route (the parity oracle): the Hadamard
// route stores (float)a*(float)b (cpu_einsum.h:87-92); every other route is a
// C=1 matmul there and stores 0.0f + (float)a*(float)b (cpu_einsum.h:71-76),
// which differs from a*b only by turning -0 into +0.  Built with
// -ffp-contract=off so the multiply and the add round separately, and with
// denormals preserved.
//
// Memory: bandwidth bound (2-3 loads + 1 store per element, no reuse), so the
// kernel is a grid-stride stream of 16-byte loads and non-temporal 16-byte
// stores.  Axes are merged on the host first; the innermost merged axis is
// the vector axis and the outer axes are decoded with multiply-high division.
#include "pe_common.h"

#include <algorithm>
#include <type_traits>
#include <vector>

// Blocks per CU of the grid-stride stream and vectors per thread per
// iteration.  Measured on MI355X: a flat contiguous stream runs fastest with
// few long-lived waves (a compact moving window in HBM); streams that decode
// outer axes per vector need many more waves to hide that arithmetic.
#ifndef PE_PRODUCT_GRID_PER_CU_FLAT
#define PE_PRODUCT_GRID_PER_CU_FLAT 2
#endif
#ifndef PE_PRODUCT_GRID_PER_CU
#define PE_PRODUCT_GRID_PER_CU 64
#endif
#ifndef PE_PRODUCT_UNROLL
#define PE_PRODUCT_UNROLL 1
#endif
// Products with outer axes (a broadcast operand: configs 4b, 5.R) issue the
// next iteration's loads before this iteration's stores.  One MI355X, same
// box, cold operands and outputs: 5.R 41.7-42.2 -> 36.8-37.2 us, 4b
// 149.0-150.5 -> 146.1-147.2 us; flat products (4a, 5.2) measured 1-2 %
// slower that way and keep one iteration's loads and stores in turn.
#ifndef PE_PRODUCT_PIPE
#define PE_PRODUCT_PIPE 1
#endif
#ifndef PE_PRODUCT_VEC_F32
#define PE_PRODUCT_VEC_F32 4
#endif
#ifndef PE_PRODUCT_VEC_F16
#define PE_PRODUCT_VEC_F16 4
#endif

namespace pe {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxOuter = PE_MAX_DIMS - 1;

struct ProductArgs {
    const void* a;
    const void* b;
    float* out;
    uint32_t nvec;          // vectors in the output (32-bit path)
    uint32_t inner;         // extent of the innermost axis, in elements
    FastDiv inner_vecs;     // inner / VEC
    int32_t nouter;         // outer axes (outermost first)
    FastDiv outer_div[kMaxOuter];
    int64_t a_outer[kMaxOuter];
    int64_t b_outer[kMaxOuter];
    int64_t a_inner, b_inner;
    int32_t nt;             // output store flavour (nt_mode)
    int32_t a_flat;         // A's offset is the output's flat index (A laid out as the output)
    int32_t b_first;        // outer axes below this index have B stride 0 (their index is unused)
};

template <typename E, int VEC>
struct VecLoad;

// Vector load with the non-temporal hint (global_load ... nt), for the first
// operand of a flat stream (one merged axis: every element read once).  A
// compile-time choice: behind a runtime branch beside an ordinary load of the
// same address the compiler merges the two and drops the hint.  Measured on
// MI355X: config 4a 138-139 -> 132-134 us, 5.2 36.6 -> 34.6-34.8 us; with the
// second operand so loaded too, 4a went back to 138 us; for the broadcast
// streams (4b, 5.R, first operand laid out as the output) no change.
template <typename E, int VEC>
__device__ __forceinline__ void load_stream(const typename E::T* p, float (&v)[VEC]) {
    if constexpr (VEC == 4 && E::kBytes == 4) {
        const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = x[i];
    } else if constexpr (VEC == 4) {
        const f16x4 x = __builtin_nontemporal_load(reinterpret_cast<const f16x4*>(p));
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (float)x[i];
    } else {
        VecLoad<E, VEC>::load(p, v);
    }
}

template <>
struct VecLoad<F32, 4> {
    __device__ __forceinline__ static void load(const float* p, float (&v)[4]) {
        f32x4 x = *reinterpret_cast<const f32x4*>(p);
        v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
    }
};
template <>
struct VecLoad<F16, 8> {
    __device__ __forceinline__ static void load(const _Float16* p, float (&v)[8]) {
        f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
    }
};
template <>
struct VecLoad<F16, 4> {
    __device__ __forceinline__ static void load(const _Float16* p, float (&v)[4]) {
        f16x4 x = *reinterpret_cast<const f16x4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (float)x[i];
    }
};
template <typename E>
struct VecLoad<E, 1> {
    __device__ __forceinline__ static void load(const typename E::T* p, float (&v)[1]) {
        v[0] = E::to_f32(*p);
    }
};

// B operand per vector: contiguous (B_MODE 1), one broadcast scalar (0) or
// general per-element stride (2, scalar path only).
template <typename E, int VEC, int B_MODE>
__device__ __forceinline__ void load_b(const typename E::T* b, int64_t off, int64_t bstride,
                                       float (&v)[VEC]) {
    if constexpr (B_MODE == 1) {
        VecLoad<E, VEC>::load(b + off, v);
    } else if constexpr (B_MODE == 0) {
        float s = E::to_f32(b[off]);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] = s;
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] = E::to_f32(b[off + i * bstride]);
    }
}

template <int VEC>
__device__ __forceinline__ void store_out(float* out, const float (&r)[VEC], int nt) {
    if constexpr (VEC == 4) {
        f32x4 v = {r[0], r[1], r[2], r[3]};
        store_f(reinterpret_cast<f32x4*>(out), v, nt);
    } else if constexpr (VEC == 8) {
        f32x4 v0 = {r[0], r[1], r[2], r[3]};
        f32x4 v1 = {r[4], r[5], r[6], r[7]};
        store_f(reinterpret_cast<f32x4*>(out), v0, nt);
        store_f(reinterpret_cast<f32x4*>(out) + 1, v1, nt);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) store_f(out + i, r[i], nt);
    }
}

// As store_out with the store flavour fixed at compile time: the compiler's
// own non-temporal store (no branch for it to merge), which its
// memory-counter waits then count (an assembly store is invisible to them).
template <int VEC, bool NT>
__device__ __forceinline__ void store_out_fixed(float* out, const float (&r)[VEC]) {
    if constexpr (VEC == 4 || VEC == 8) {
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h) {
            const f32x4 v = {r[4 * h], r[4 * h + 1], r[4 * h + 2], r[4 * h + 3]};
            f32x4* q = reinterpret_cast<f32x4*>(out) + h;
            if constexpr (NT) __builtin_nontemporal_store(v, q);
            else *q = v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            if constexpr (NT) __builtin_nontemporal_store(r[i], out + i);
            else out[i] = r[i];
        }
    }
}

// One launch streams all output vectors.  UNROLL vectors per thread per
// iteration: all loads are issued before any store so several 16-byte loads
// are in flight per lane; with outer axes (PE_PRODUCT_PIPE) the next
// iteration's loads go out before this iteration's stores as well.
template <typename E, int VEC, int B_MODE, bool ADD_ZERO, bool HAS_OUTER, int UNROLL>
__global__ __launch_bounds__(kThreads) void product_kernel(ProductArgs p) {
    using T = typename E::T;
    const T* __restrict__ a = static_cast<const T*>(p.a);
    const T* __restrict__ b = static_cast<const T*>(p.b);
    float* __restrict__ out = p.out;
    const uint32_t stride = gridDim.x * kThreads;
    uint32_t v = blockIdx.x * kThreads + threadIdx.x;
    // Loads of the UNROLL vectors v0 + u * stride into (xa, xb); CHECK:
    // vectors past the end are skipped (lv false), else their index is
    // clamped to the last vector (loaded, never stored): no branch around a
    // load, so the compiler's memory-counter waits stay exact.
    auto fetch = [&](auto check, uint32_t v0, float (&xa)[UNROLL][VEC], float (&xb)[UNROLL][VEC],
                     bool (&lv)[UNROLL]) {
        constexpr bool CHECK = decltype(check)::value;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint32_t vv = v0 + u * stride;
            lv[u] = vv < p.nvec;
            if (CHECK) {
                if (!lv[u]) continue;
            } else {
                vv = min(vv, p.nvec - 1);
            }
            int64_t aoff, boff;
            if constexpr (HAS_OUTER) {
                uint32_t row, colv;
                p.inner_vecs.divmod(vv, row, colv);
                uint32_t col = colv * VEC;
                boff = int64_t(col) * p.b_inner;
                if (p.a_flat) {
                    // Only B's offset needs the outer indices, and only down
                    // to its outermost axis with a nonzero stride.
                    aoff = int64_t(vv) * VEC;
                    for (int d = p.nouter - 1; d >= p.b_first; --d) {
                        uint32_t q, r;
                        p.outer_div[d].divmod(row, q, r);
                        boff += int64_t(r) * p.b_outer[d];
                        row = q;
                    }
                } else {
                    aoff = int64_t(col) * p.a_inner;
                    for (int d = p.nouter - 1; d >= 0; --d) {
                        uint32_t q, r;
                        p.outer_div[d].divmod(row, q, r);
                        aoff += int64_t(r) * p.a_outer[d];
                        boff += int64_t(r) * p.b_outer[d];
                        row = q;
                    }
                }
            } else {
                aoff = int64_t(vv) * VEC * p.a_inner;
                boff = int64_t(vv) * VEC * p.b_inner;
            }
            if constexpr (VEC > 1 && !HAS_OUTER) {
                load_stream<E, VEC>(a + aoff, xa[u]);
            } else if constexpr (VEC > 1) {
                VecLoad<E, VEC>::load(a + aoff, xa[u]);
            } else {
                xa[u][0] = E::to_f32(a[aoff]);
            }
            load_b<E, VEC, B_MODE>(b, boff, p.b_inner, xb[u]);
        }
    };
    // Products and stores of the vectors fetched for v0 (CHECK: live ones;
    // nt: non-temporal stores, a run-time flag or a compile-time constant).
    auto finish = [&](auto check, auto nt, uint32_t v0, const float (&xa)[UNROLL][VEC],
                      const float (&xb)[UNROLL][VEC], const bool (&lv)[UNROLL]) {
        constexpr bool CHECK = decltype(check)::value;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if (CHECK && !lv[u]) continue;
            float r[VEC];
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                float prod = xa[u][i] * xb[u][i];
                r[i] = ADD_ZERO ? 0.0f + prod : prod;
            }
            if constexpr (std::is_same_v<decltype(nt), int>)
                store_out<VEC>(out + int64_t(v0 + u * stride) * VEC, r, nt);
            else
                store_out_fixed<VEC, decltype(nt)::value>(out + int64_t(v0 + u * stride) * VEC, r);
        }
    };
    using Checked = std::true_type;
    using Unchecked = std::false_type;
    float ra[UNROLL][VEC], rb[UNROLL][VEC];
    bool live[UNROLL];
    if (PE_PRODUCT_PIPE && HAS_OUTER) {
        // While every lane of the wave has all UNROLL vectors (a wave's
        // lanes hold 64 consecutive v), the next iteration's loads are
        // issued before this iteration's stores: the memory counter
        // completes in issue order, so waiting for loads issued after a
        // store would wait for the store as well.
        const uint32_t vmax = (uint32_t(__builtin_amdgcn_readfirstlane(int(v))) | 63u) + (UNROLL - 1) * stride;
        const uint32_t step = stride * UNROLL;
        // (The store flavour is fixed outside the loop: a branch around a
        // store inside it would make the compiler wait for every load.)
        // Two register sets in turn (copying one into the other would wait
        // for the loads just issued), in the order load X0, load Y1, store
        // X0, load X2, then per pair store Y(i), load Y(i + 2), store
        // X(i + 1), load X(i + 3): every store's data arrived before the
        // loads and the store issued after it, which stay in flight, and the
        // loop is entered in the state it repeats (the compiler takes the
        // smallest count over the loop's entry and its back edge).
        auto pipelined = [&](auto nt) {
            const uint32_t iters = (p.nvec - 1 - vmax) / step + 1;  // wave-uniform
            const uint32_t v0 = v;
            float xa[UNROLL][VEC], xb[UNROLL][VEC], ya[UNROLL][VEC], yb[UNROLL][VEC];
            bool xl[UNROLL], yl[UNROLL];
            fetch(Unchecked{}, v0, xa, xb, xl);
            if (iters > 1) {
                fetch(Unchecked{}, v0 + step, ya, yb, yl);
                __builtin_amdgcn_sched_barrier(0);
                finish(Unchecked{}, nt, v0, xa, xb, xl);
                fetch(Unchecked{}, v0 + 2 * step, xa, xb, xl);
                uint32_t i = 1;
                for (; i + 2 <= iters; i += 2) {
                    finish(Unchecked{}, nt, v0 + i * step, ya, yb, yl);
                    fetch(Unchecked{}, v0 + (i + 2) * step, ya, yb, yl);
                    __builtin_amdgcn_sched_barrier(0);
                    finish(Unchecked{}, nt, v0 + (i + 1) * step, xa, xb, xl);
                    fetch(Unchecked{}, v0 + (i + 3) * step, xa, xb, xl);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (i < iters) finish(Unchecked{}, nt, v0 + i * step, ya, yb, yl);
            } else {
                finish(Unchecked{}, nt, v0, xa, xb, xl);
            }
            v = v0 + iters * step;
        };
        if (vmax < p.nvec) {
            if (p.nt) pipelined(std::true_type{});
            else pipelined(std::false_type{});
        }
    }
    for (; v < p.nvec; v += stride * UNROLL) {
        fetch(Checked{}, v, ra, rb, live);
        finish(Checked{}, p.nt, v, ra, rb, live);
    }
}

// Fallback for outputs of 2^31 elements or more: 64-bit division per element.
template <typename E, bool ADD_ZERO>
__global__ __launch_bounds__(kThreads) void product_kernel_wide(
    const typename E::T* __restrict__ a, const typename E::T* __restrict__ b,
    float* __restrict__ out, int64_t n, int32_t ndims, pe_product_desc d) {
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    for (int64_t o = int64_t(blockIdx.x) * kThreads + threadIdx.x; o < n; o += stride) {
        int64_t rem = o, aoff = 0, boff = 0;
        for (int k = ndims - 1; k >= 0; --k) {
            int64_t x = rem % d.shape[k];
            rem /= d.shape[k];
            aoff += x * d.a_stride[k];
            boff += x * d.b_stride[k];
        }
        float prod = E::to_f32(a[aoff]) * E::to_f32(b[boff]);
        store_nt(out + o, ADD_ZERO ? 0.0f + prod : prod);
    }
}

// Merge adjacent output axes whose strides compose in both operands
// (stride[d] == extent[d+1] * stride[d+1]), dropping extent-1 axes.
void merge_axes(const pe_product_desc& d, std::vector<int64_t>& shape,
                std::vector<int64_t>& sa, std::vector<int64_t>& sb) {
    shape.clear(); sa.clear(); sb.clear();
    for (int k = 0; k < d.ndims; ++k) {
        if (d.shape[k] == 1) continue;
        if (!shape.empty() && sa.back() == d.shape[k] * d.a_stride[k] &&
            sb.back() == d.shape[k] * d.b_stride[k]) {
            shape.back() *= d.shape[k];
            sa.back() = d.a_stride[k];
            sb.back() = d.b_stride[k];
        } else {
            shape.push_back(d.shape[k]);
            sa.push_back(d.a_stride[k]);
            sb.push_back(d.b_stride[k]);
        }
    }
}

int grid_for(int64_t work_items, int per_block, int per_cu = PE_PRODUCT_GRID_PER_CU) {
    int64_t blocks = ceil_div(std::max<int64_t>(work_items, 1), per_block);
    int64_t cap = int64_t(cu_count()) * per_cu;
    return int(std::max<int64_t>(1, std::min(blocks, cap)));
}

template <typename E, int VEC, int B_MODE, bool ADD_ZERO, bool HAS_OUTER>
hipError_t launch_vec(const ProductArgs& args, hipStream_t s) {
    constexpr int U = (VEC >= 4) ? PE_PRODUCT_UNROLL : 4;
    int grid = grid_for(ceil_div(args.nvec, U), kThreads,
                        HAS_OUTER ? PE_PRODUCT_GRID_PER_CU : PE_PRODUCT_GRID_PER_CU_FLAT);
    hipLaunchKernelGGL((product_kernel<E, VEC, B_MODE, ADD_ZERO, HAS_OUTER, U>), dim3(grid),
                       dim3(kThreads), 0, s, args);
    return hipGetLastError();
}

template <typename E, int VEC, bool ADD_ZERO, bool HAS_OUTER>
hipError_t launch_bmode(const ProductArgs& args, int bmode, hipStream_t s) {
    if (bmode == 1) return launch_vec<E, VEC, 1, ADD_ZERO, HAS_OUTER>(args, s);
    if (bmode == 0) return launch_vec<E, VEC, 0, ADD_ZERO, HAS_OUTER>(args, s);
    return launch_vec<E, 1, 2, ADD_ZERO, HAS_OUTER>(args, s);
}

template <typename E>
int run(const pe_product_desc& d, const void* in0, const void* in1, float* out,
        hipStream_t s) {
    using T = typename E::T;
    std::vector<int64_t> shape, sa, sb;
    merge_axes(d, shape, sa, sb);
    int64_t n = 1;
    for (int64_t x : shape) n *= x;
    if (n == 0) return PE_OK;
    const bool add_zero = d.add_zero != 0;

    if (n >= (int64_t(1) << 31) || int(shape.size()) > kMaxOuter + 1) {
        pe_product_desc m = d;
        m.ndims = int32_t(shape.size());
        for (size_t k = 0; k < shape.size(); ++k) {
            m.shape[k] = shape[k]; m.a_stride[k] = sa[k]; m.b_stride[k] = sb[k];
        }
        int grid = grid_for(n, kThreads);
        if (add_zero)
            hipLaunchKernelGGL((product_kernel_wide<E, true>), dim3(grid), dim3(kThreads), 0, s,
                               (const T*)in0, (const T*)in1, out, n, m.ndims, m);
        else
            hipLaunchKernelGGL((product_kernel_wide<E, false>), dim3(grid), dim3(kThreads), 0, s,
                               (const T*)in0, (const T*)in1, out, n, m.ndims, m);
        PE_CHECK_HIP(hipGetLastError());
        return PE_OK;
    }

    ProductArgs args{};
    args.a = in0; args.b = in1; args.out = out;
    args.nt = nt_mode(n * 4);
    const int nd = int(shape.size());
    const int64_t inner = nd ? shape[nd - 1] : 1;
    args.inner = uint32_t(inner);
    args.a_inner = nd ? sa[nd - 1] : 0;
    args.b_inner = nd ? sb[nd - 1] : 0;
    args.nouter = std::max(0, nd - 1);
    for (int k = 0; k < args.nouter; ++k) {
        args.outer_div[k].init(uint32_t(shape[k]));
        args.a_outer[k] = sa[k];
        args.b_outer[k] = sb[k];
    }
    // A flat: unit inner stride and every outer stride the extent product of
    // the axes inside it, so A's element offset equals the output's.
    int64_t flat = inner;
    args.a_flat = nd > 0 && args.a_inner == 1;
    for (int k = args.nouter - 1; k >= 0; --k) {
        args.a_flat = args.a_flat && sa[k] == flat;
        flat *= shape[k];
    }
    args.b_first = 0;
    while (args.b_first < args.nouter && sb[args.b_first] == 0) ++args.b_first;

    // Vector path: VEC elements per lane along the innermost axis.  Four
    // elements give one 16-byte float32 store per lane, so each wave-wide
    // store covers 1 KB contiguously (float16 inputs load 8 bytes per lane).
    // Needs a unit inner stride, an inner extent and outer strides that are
    // whole vectors, and vector-aligned base pointers.
    constexpr int VEC = E::kBytes == 4 ? PE_PRODUCT_VEC_F32 : PE_PRODUCT_VEC_F16;
    constexpr size_t VB = size_t(VEC) * E::kBytes;
    bool vec_ok = nd > 0 && args.a_inner == 1 && (args.b_inner == 0 || args.b_inner == 1) &&
                  inner % VEC == 0 && aligned(in0, VB) && aligned(out, 16) &&
                  (args.b_inner == 0 || aligned(in1, VB));
    for (int k = 0; k < args.nouter && vec_ok; ++k)
        vec_ok = (sa[k] % VEC == 0) && (args.b_inner == 0 || sb[k] % VEC == 0);
    const bool has_outer = args.nouter > 0;

    hipError_t e;
    if (vec_ok) {
        args.nvec = uint32_t(n / VEC);
        args.inner_vecs.init(uint32_t(inner / VEC));
        int bmode = args.b_inner == 1 ? 1 : 0;
        if (add_zero)
            e = has_outer ? launch_bmode<E, VEC, true, true>(args, bmode, s)
                          : launch_bmode<E, VEC, true, false>(args, bmode, s);
        else
            e = has_outer ? launch_bmode<E, VEC, false, true>(args, bmode, s)
                          : launch_bmode<E, VEC, false, false>(args, bmode, s);
    } else {
        args.nvec = uint32_t(n);
        args.inner_vecs.init(uint32_t(inner));
        if (add_zero)
            e = has_outer ? launch_bmode<E, 1, true, true>(args, 2, s)
                          : launch_bmode<E, 1, true, false>(args, 2, s);
        else
            e = has_outer ? launch_bmode<E, 1, false, true>(args, 2, s)
                          : launch_bmode<E, 1, false, false>(args, 2, s);
    }
    PE_CHECK_HIP(e);
    return PE_OK;
}

}  // namespace

int validate_product(const pe_product_desc& d) {
    if (d.dtype != PE_F32 && d.dtype != PE_F16)
        return fail(PE_ERR_UNSUPPORTED, "product: dtype must be PE_F32 or PE_F16");
    if (d.ndims < 0 || d.ndims > PE_MAX_DIMS)
        return fail(PE_ERR_INVALID, "product: ndims out of range");
    int64_t amax = 0, bmax = 0, n = 1;
    for (int k = 0; k < d.ndims; ++k) {
        if (d.shape[k] < 0 || d.a_stride[k] < 0 || d.b_stride[k] < 0)
            return fail(PE_ERR_INVALID, "product: negative extent or stride");
        n *= d.shape[k];
        if (d.shape[k] > 0) {
            amax += (d.shape[k] - 1) * d.a_stride[k];
            bmax += (d.shape[k] - 1) * d.b_stride[k];
        }
    }
    if (n > 0 && (amax >= d.a_numel || bmax >= d.b_numel))
        return fail(PE_ERR_BOUNDS, "product: strides address past an operand's extent");
    return PE_OK;
}

}  // namespace pe

extern "C" int pe_product(const pe_product_desc* d, const void* in0, const void* in1,
                          float* out, void* stream) {
    if (!d) return pe::fail(PE_ERR_INVALID, "product: null descriptor");
    int st = pe::validate_product(*d);
    if (st != PE_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return d->dtype == PE_F32 ? pe::run<pe::F32>(*d, in0, in1, out, s)
                              : pe::run<pe::F16>(*d, in0, in1, out, s);
}
