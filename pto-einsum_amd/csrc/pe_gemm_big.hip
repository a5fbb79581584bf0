// Host side of the large float16 GEMM (pe_gemm_big.h): instantiations for
// the four operand layout pairings, their residency (with the spill check)
// and the persistent launch, one block per CU.
#include "pe_gemm_big.h"

#include <algorithm>

namespace pe {

// M16: the 16x16x32 schedule, for a k-contiguous A with an even number of
// 32-k slabs per tile.
template <bool TAIL>
static const void* big_kernel_t(int al, int bl, bool m16) {
    if (al == L_K)
        return bl == L_K ? (m16 ? reinterpret_cast<const void*>(&gemm_big_kernel<L_K, L_K, TAIL, true>)
                                : reinterpret_cast<const void*>(&gemm_big_kernel<L_K, L_K, TAIL, false>))
                         : (m16 ? reinterpret_cast<const void*>(&gemm_big_kernel<L_K, L_MN, TAIL, true>)
                                : reinterpret_cast<const void*>(&gemm_big_kernel<L_K, L_MN, TAIL, false>));
    return bl == L_K ? reinterpret_cast<const void*>(&gemm_big_kernel<L_MN, L_K, TAIL, false>)
                     : reinterpret_cast<const void*>(&gemm_big_kernel<L_MN, L_MN, TAIL, false>);
}
static const void* big_kernel(int al, int bl, bool tail, bool m16) {
    return tail ? big_kernel_t<true>(al, bl, m16) : big_kernel_t<false>(al, bl, m16);
}

// Resident blocks per CU of both variants (0 when either spilled).
int gemm_big_resident(int al, int bl) {
    static int cache[4] = {-1, -1, -1, -1};
    int& c = cache[(al == L_K) * 2 + (bl == L_K)];
    if (c < 0) {
        c = 1 << 30;
        for (bool tail : {false, true})
            for (bool m16 : {false, true}) {
                hipFuncAttributes at{};
                int n = 0;
                const void* k = big_kernel(al, bl, tail, m16);
                if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > 16 ||
                    hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
                    n = 0;
                c = std::min(c, n);
            }
    }
    return c;
}

hipError_t launch_gemm_big(int al, int bl, const GemmArgs& g, hipStream_t s) {
    const int resident = gemm_big_resident(al, bl);
    if (resident < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    const uint32_t cap = uint32_t(cu_count()) * uint32_t(resident);
    if (a.grid > cap) a.grid = cap;
    void* args[] = {&a};
    const bool m16 = al == L_K && ((a.K + 31) / 32) % 2 == 0;
    return hipLaunchKernel(big_kernel(al, bl, a.K % 32 != 0, m16), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

}  // namespace pe
