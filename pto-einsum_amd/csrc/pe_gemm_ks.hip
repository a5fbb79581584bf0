// Host side of the k-split GEMM kernel (pe_gemm_ks.h): its float32
// instantiations (32 x 32 and 64 x 64 tiles, three LDS stages, one sub-slab
// per wave per stage, two accumulator sets), their residency and the launch.
#include "pe_gemm_ks.h"

namespace pe {

namespace {

template <int TILE, int AL, int BL>
const void* ks_kernel_t() {
    return reinterpret_cast<const void*>(&gemm_ks_kernel<F32, TILE, TILE, AL, BL, 3, 1, 2>);
}

template <int TILE>
const void* ks_kernel_ab(int al, int bl) {
    if (al == L_MN) return bl == L_MN ? ks_kernel_t<TILE, L_MN, L_MN>() : ks_kernel_t<TILE, L_MN, L_K>();
    return bl == L_MN ? ks_kernel_t<TILE, L_K, L_MN>() : ks_kernel_t<TILE, L_K, L_K>();
}

const void* ks_kernel(int al, int bl, int tile) {
    return tile == 64 ? ks_kernel_ab<64>(al, bl) : ks_kernel_ab<32>(al, bl);
}

}  // namespace

int gemm_ks_resident(int al, int bl, int tile) {
    if ((al != L_MN && al != L_K) || (bl != L_MN && bl != L_K) || (tile != 32 && tile != 64)) return 0;
    static int cache[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
    int& c = cache[(tile == 64) * 4 + (al == L_K) * 2 + (bl == L_K)];
    if (c < 0) {
        const void* k = ks_kernel(al, bl, tile);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > 0 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

hipError_t launch_gemm_ks(int al, int bl, int tile, const GemmArgs& g, hipStream_t s) {
    if (gemm_ks_resident(al, bl, tile) < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    void* args[] = {&a};
    return hipLaunchKernel(ks_kernel(al, bl, tile), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

}  // namespace pe
