// Attainable-peak probe for the measurement harness: MFMA throughput of this
// device with no memory traffic, the ceiling the GEMM kernels are held
// against next to the datasheet peak.
//
// Each wave keeps CHAINS independent accumulator chains and issues MFMAs round
// robin over them (a chain's next MFMA comes CHAINS MFMAs later, past the
// result latency), two waves per SIMD.  The operands rotate over eight
// register fragments per lane: with `random` they hold hashed values in
// [-1/8, 1/8) that differ per lane, fragment and block (the bit activity of a
// real GEMM's data), otherwise one constant.  The MFMA clock is set by power,
// and power by the operands' bit activity, so the two differ (the datasheet
// peak assumes the nominal clock).  Each lane stores the sum of its
// accumulators so that nothing is optimised away.
#include "pe_common.h"

#include <algorithm>

namespace pe {
namespace {

constexpr int kChains = 8;
constexpr int kFrags = 8;

__device__ __forceinline__ float hashed(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return (float(x & 0xffffu) / 65536.0f - 0.5f) * 0.25f;
}

__device__ __forceinline__ float operand(bool random, uint32_t key) { return random ? hashed(key) : 0.125f; }

template <bool F16>
__global__ __launch_bounds__(256, 2) void mfma_probe_kernel(int64_t iters, int32_t random, float* out) {
    const uint32_t tid = threadIdx.x, key = (blockIdx.x * 256u + tid) * 1024u;
    f32x16 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    if constexpr (F16) {
        f16x8 a[kFrags], b[kFrags];
#pragma unroll
        for (int j = 0; j < kFrags; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a[j][i] = _Float16(operand(random != 0, key + 16u * j + i));
                b[j][i] = _Float16(operand(random != 0, key + 16u * j + 8u + i + 512u));
            }
        for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int t = 0; t < 2 * kChains; ++t)
                acc[t % kChains] =
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(a[t % kFrags], b[(t / 2) % kFrags], acc[t % kChains], 0, 0, 0);
        }
    } else {
        float a[kFrags], b[kFrags];
#pragma unroll
        for (int j = 0; j < kFrags; ++j) {
            a[j] = operand(random != 0, key + j);
            b[j] = operand(random != 0, key + j + 512u);
        }
        for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int t = 0; t < 2 * kChains; ++t)
                acc[t % kChains] =
                    __builtin_amdgcn_mfma_f32_32x32x2f32(a[t % kFrags], b[(t / 2) % kFrags], acc[t % kChains], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s = s + acc[c][r];
    out[int64_t(blockIdx.x) * 256 + tid] = s;
}

// Launch-floor probe: one wave that stores one float.  Replayed in a graph
// beside the small GEMMs, its time per launch is the fixed cost any kernel
// pays on this device (dispatch, wave launch, completion signal), the floor
// a launch-bound case such as a 256^3 GEMM is read against.
__global__ __launch_bounds__(64) void launch_probe_kernel(float* out) {
    if (threadIdx.x == 0) out[0] = 0.0f;
}

}  // namespace
}  // namespace pe

extern "C" int pe_probe_launch(float* out, void* stream) {
    using namespace pe;
    if (!out) return fail(PE_ERR_INVALID, "probe_launch: null output");
    hipLaunchKernelGGL(launch_probe_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), out);
    PE_CHECK_HIP(hipGetLastError());
    return PE_OK;
}

extern "C" int64_t pe_probe_mfma_flops(int dtype, int64_t iters) {
    // blocks x 4 waves x iters x (2 * kChains) MFMAs x flops per MFMA
    const int64_t blocks = int64_t(pe::cu_count()) * 2;
    const int64_t per = dtype == PE_F16 ? 2LL * 32 * 32 * 16 : 2LL * 32 * 32 * 2;
    return blocks * 4 * iters * 2 * pe::kChains * per;
}

extern "C" int64_t pe_probe_out_len(void) { return int64_t(pe::cu_count()) * 2 * 256; }

extern "C" int pe_probe_mfma(int dtype, int random, int64_t iters, float* out, int64_t out_len, void* stream) {
    using namespace pe;
    if (dtype != PE_F16 && dtype != PE_F32) return fail(PE_ERR_UNSUPPORTED, "probe_mfma: dtype must be PE_F16 or PE_F32");
    if (iters < 1) return fail(PE_ERR_INVALID, "probe_mfma: iters must be >= 1");
    const int blocks = cu_count() * 2;
    if (!out || out_len < int64_t(blocks) * 256) return fail(PE_ERR_BOUNDS, "probe_mfma: out shorter than pe_probe_out_len()");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == PE_F16)
        hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(blocks), dim3(256), 0, s, iters, int32_t(random), out);
    else
        hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(blocks), dim3(256), 0, s, iters, int32_t(random), out);
    PE_CHECK_HIP(hipGetLastError());
    return PE_OK;
}
