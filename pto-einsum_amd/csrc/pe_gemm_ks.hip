// Host side of the k-split GEMM kernel (pe_gemm_ks.h): its instantiations
// (float32 32 x 32 and 64 x 64 tiles with three LDS stages, float16 64 x 64
// tiles with four; one sub-slab per wave per stage, two accumulator sets),
// their residency and the launch.
#include "pe_gemm_ks.h"

namespace pe {

namespace {

template <typename E, int TILE, int NS, int AL, int BL>
const void* ks_kernel_t() {
    return reinterpret_cast<const void*>(&gemm_ks_kernel<E, TILE, TILE, AL, BL, NS, 1, 2>);
}

template <typename E, int TILE, int NS>
const void* ks_kernel_ab(int al, int bl) {
    if (al == L_MN) return bl == L_MN ? ks_kernel_t<E, TILE, NS, L_MN, L_MN>() : ks_kernel_t<E, TILE, NS, L_MN, L_K>();
    return bl == L_MN ? ks_kernel_t<E, TILE, NS, L_K, L_MN>() : ks_kernel_t<E, TILE, NS, L_K, L_K>();
}

const void* ks_kernel(int dtype, int al, int bl, int tile) {
    if (dtype == PE_F16) return ks_kernel_ab<F16, 64, 4>(al, bl);
    return tile == 64 ? ks_kernel_ab<F32, 64, 3>(al, bl) : ks_kernel_ab<F32, 32, 3>(al, bl);
}

}  // namespace

int gemm_ks_resident(int dtype, int al, int bl, int tile) {
    if ((al != L_MN && al != L_K) || (bl != L_MN && bl != L_K)) return 0;
    if (!((dtype == PE_F32 && (tile == 32 || tile == 64)) || (dtype == PE_F16 && tile == 64))) return 0;
    static int cache[12] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1};
    const int variant = dtype == PE_F16 ? 2 : (tile == 64 ? 1 : 0);
    int& c = cache[variant * 4 + (al == L_K) * 2 + (bl == L_K)];
    if (c < 0) {
        const void* k = ks_kernel(dtype, al, bl, tile);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > 0 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

hipError_t launch_gemm_ks(int dtype, int al, int bl, int tile, const GemmArgs& g, hipStream_t s) {
    if (gemm_ks_resident(dtype, al, bl, tile) < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    void* args[] = {&a};
    return hipLaunchKernel(ks_kernel(dtype, al, bl, tile), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

}  // namespace pe
