// Host side of the direct-load GEMM kernel (pe_gemm_dl.h): the
// instantiations for float32 and float16, their residency (with the
// register-spill check) and the launch.
#include "pe_gemm_dl.h"

namespace pe {

// Direct-load kernels: 64x64 and 128x128 tiles held to four resident blocks
// per CU, 256x128 / 128x256 tiles in two register budgets (two or three
// resident blocks per CU; which one fits a grid is decided in choose()).
template <typename E, int BM, int BN, int MINB>
static const void* dl_kernel_ab(int al, int bl) {
    if (al == L_MN)
        return bl == L_MN ? reinterpret_cast<const void*>(&gemm_dl_kernel<E, BM, BN, L_MN, L_MN, MINB>)
                          : reinterpret_cast<const void*>(&gemm_dl_kernel<E, BM, BN, L_MN, L_K, MINB>);
    return bl == L_MN ? reinterpret_cast<const void*>(&gemm_dl_kernel<E, BM, BN, L_K, L_MN, MINB>)
                      : reinterpret_cast<const void*>(&gemm_dl_kernel<E, BM, BN, L_K, L_K, MINB>);
}

template <typename E>
static const void* dl_kernel_t(int bm, int bn, int minb, int al, int bl) {
    if (bm == 256) return minb == 2 ? dl_kernel_ab<E, 256, 128, 2>(al, bl) : dl_kernel_ab<E, 256, 128, 3>(al, bl);
    if (bn == 256) return minb == 2 ? dl_kernel_ab<E, 128, 256, 2>(al, bl) : dl_kernel_ab<E, 128, 256, 3>(al, bl);
    return bm == 128 ? dl_kernel_ab<E, 128, 128, 4>(al, bl) : dl_kernel_ab<E, 64, 64, 4>(al, bl);
}

static const void* dl_kernel(int dtype, int bm, int bn, int minb, int al, int bl) {
    return dtype == PE_F32 ? dl_kernel_t<F32>(bm, bn, minb, al, bl) : dl_kernel_t<F16>(bm, bn, minb, al, bl);
}

static int dl_index(int dtype, int bm, int bn, int minb, int al, int bl) {
    const int t = bm == 256 ? (minb == 2 ? 2 : 3) : bn == 256 ? (minb == 2 ? 4 : 5) : bm == 128 ? 1 : 0;
    return ((((dtype == PE_F32) ? 0 : 6) + t) * 2 + (al == L_K)) * 2 + (bl == L_K);
}

// Instantiations whose register allocation spilled more than this many bytes
// per lane are never launched (larger spills sit inside the MFMA loop).  Of
// the 256-wide tiles at three blocks per CU, those with one or both operands
// k-contiguous spill 8-12 bytes (a lane offset reloaded once per slab) and
// run as fast as spill-free ones; the float16 ones spill hundreds.
#ifndef PE_GEMM_DL_MAX_SPILL
#define PE_GEMM_DL_MAX_SPILL 16
#endif

int gemm_dl_resident(int dtype, int bm, int bn, int minb, int al, int bl) {
    static int cache[2 * 6 * 4];
    static bool init = false;
    if (!init) {
        for (int& c : cache) c = -1;
        init = true;
    }
    int& c = cache[dl_index(dtype, bm, bn, minb, al, bl)];
    if (c < 0) {
        const void* k = dl_kernel(dtype, bm, bn, minb, al, bl);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > PE_GEMM_DL_MAX_SPILL ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

bool gemm_dl_eligible(int dtype, int al, int bl, int64_t M, int64_t N, int64_t K, int64_t c_ms, int64_t c_ns) {
    if (!PE_GEMM_DL) return false;
    if (dtype == PE_F16 && !PE_GEMM_DL_F16) return false;
    const int vec = dtype == PE_F32 ? 4 : 8;  // elements per 16-byte vector
    if (al != L_MN && al != L_K) return false;
    if (bl != L_MN && bl != L_K) return false;
    if (al == L_MN && M % vec != 0) return false;
    if (bl == L_MN && N % vec != 0) return false;
    if ((al == L_K || bl == L_K) && K % vec != 0) return false;
    // 32-bit store offsets: every element of a tile (at most 256 x 256)
    // within 2^31 bytes of its corner, for the output and for the row-major
    // split-K partials (strides N and 1).
    const int64_t lim = int64_t(1) << 29;
    if (c_ms < 0 || c_ns < 0 || 255 * (c_ms + c_ns) >= lim || 255 * (N + 1) >= lim) return false;
    return true;
}

hipError_t launch_gemm_dl(int dtype, int bm, int bn, int minb, int al, int bl, bool persist, const GemmArgs& g,
                          hipStream_t s) {
    const int resident = gemm_dl_resident(dtype, bm, bn, minb, al, bl);
    if (resident < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    const uint32_t cap = persist ? uint32_t(cu_count()) * uint32_t(resident) : 0x7fffffffu;
    if (a.grid > cap) a.grid = cap;
    void* args[] = {&a};
    return hipLaunchKernel(dl_kernel(dtype, bm, bn, minb, al, bl), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

// Short-K all-resident kernel (gemm_res_kernel), every k slab of K resident
// in LDS.  float16: 64x128 tiles (A rows x B rows), four 32-k slabs (K in
// (96, 128]), 48 KB of LDS, three blocks per CU; float32: 128x128 tiles,
// eight 16-k slabs (K in (112, 128]), one block per CU.  A block holds its
// registers and LDS until its output stores have completed, so the number
// of resident blocks sets how much of one block's store drain overlaps the
// loads and MFMAs of others.  float16 on one MI355X (float32 output, cold
// operands and outputs), 64x128 against 128x128 tiles at two blocks per CU:
// 4096^2 x 128 (config 5.1) 15.8-16.0 -> 14.4-14.5 us, 2048^2 x 128 8.2 ->
// 7.8, 4096 x 8192 x 128 27.2-27.4 -> 25.9, 8192^2 x 128 50.0-50.3 -> 50.5,
// 8192 x 16384 x 128 100.1-101.6 -> 96.4, K = 112 at 4096^2 16.7 -> 16.2;
// 64x64 tiles at five blocks per CU: 15.4, 7.9, 27.6, 54.7, 102.2 and
// 15.1 us.
#ifndef PE_GEMM_RES_F16_BM
#define PE_GEMM_RES_F16_BM 64
#endif
#ifndef PE_GEMM_RES_F16_BN
#define PE_GEMM_RES_F16_BN 128
#endif
#ifndef PE_GEMM_RES_F16_MINB
#define PE_GEMM_RES_F16_MINB 3
#endif
template <typename E, int BM, int BN, int NS, int MINB>
static const void* res_kernel_t(int al, int bl) {
    if (al == L_MN)
        return bl == L_MN ? reinterpret_cast<const void*>(&gemm_res_kernel<E, BM, BN, L_MN, L_MN, NS, MINB>)
                          : reinterpret_cast<const void*>(&gemm_res_kernel<E, BM, BN, L_MN, L_K, NS, MINB>);
    return bl == L_MN ? reinterpret_cast<const void*>(&gemm_res_kernel<E, BM, BN, L_K, L_MN, NS, MINB>)
                      : reinterpret_cast<const void*>(&gemm_res_kernel<E, BM, BN, L_K, L_K, NS, MINB>);
}
static const void* res_kernel(int dtype, int al, int bl) {
    return dtype == PE_F32 ? res_kernel_t<F32, 128, 128, 8, 1>(al, bl)
                           : res_kernel_t<F16, PE_GEMM_RES_F16_BM, PE_GEMM_RES_F16_BN, 4, PE_GEMM_RES_F16_MINB>(al, bl);
}

// Tile rows and columns of the short-K kernel for dtype.
int gemm_res_tile_m(int dtype) { return dtype == PE_F32 ? 128 : PE_GEMM_RES_F16_BM; }
int gemm_res_tile_n(int dtype) { return dtype == PE_F32 ? 128 : PE_GEMM_RES_F16_BN; }

int gemm_res_resident(int dtype, int al, int bl) {
    static int cache[2][4] = {{-1, -1, -1, -1}, {-1, -1, -1, -1}};
    int& c = cache[dtype == PE_F32][(al == L_K) * 2 + (bl == L_K)];
    if (c < 0) {
        const void* k = res_kernel(dtype, al, bl);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > PE_GEMM_DL_MAX_SPILL ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

hipError_t launch_gemm_res(int dtype, int al, int bl, const GemmArgs& g, hipStream_t s) {
    if (gemm_res_resident(dtype, al, bl) < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    void* args[] = {&a};
    return hipLaunchKernel(res_kernel(dtype, al, bl), dim3(a.total_blocks), dim3(kGemmThreads), args, 0, s);
}

}  // namespace pe
