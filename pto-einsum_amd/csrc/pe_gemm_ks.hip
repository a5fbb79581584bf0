// Host side of the k-split GEMM kernel (pe_gemm_ks.h): its float32
// instantiations (32 x 32 tiles, three LDS stages, one sub-slab per wave per
// stage, two accumulator sets), their residency and the launch.
#include "pe_gemm_ks.h"

namespace pe {

namespace {

template <int AL, int BL>
const void* ks_kernel_t() {
    return reinterpret_cast<const void*>(&gemm_ks_kernel<F32, kKsTile, kKsTile, AL, BL, 3, 1, 2>);
}

const void* ks_kernel(int al, int bl) {
    if (al == L_MN) return bl == L_MN ? ks_kernel_t<L_MN, L_MN>() : ks_kernel_t<L_MN, L_K>();
    return bl == L_MN ? ks_kernel_t<L_K, L_MN>() : ks_kernel_t<L_K, L_K>();
}

}  // namespace

int gemm_ks_resident(int al, int bl) {
    if ((al != L_MN && al != L_K) || (bl != L_MN && bl != L_K)) return 0;
    static int cache[4] = {-1, -1, -1, -1};
    int& c = cache[(al == L_K) * 2 + (bl == L_K)];
    if (c < 0) {
        const void* k = ks_kernel(al, bl);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > 0 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

hipError_t launch_gemm_ks(int al, int bl, const GemmArgs& g, hipStream_t s) {
    if (gemm_ks_resident(al, bl) < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    void* args[] = {&a};
    return hipLaunchKernel(ks_kernel(al, bl), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

}  // namespace pe
