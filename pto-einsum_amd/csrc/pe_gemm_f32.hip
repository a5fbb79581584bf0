// float32 instantiations of the batched MFMA GEMM (v_mfma_f32_32x32x2_f32).
#include "pe_gemm_dl.h"

// Slab depth and LDS layout for float32 (see GemmGeom).
#ifndef PE_GEMM_F32_BK
#define PE_GEMM_F32_BK 16
#endif
#ifndef PE_GEMM_F32_KC
#define PE_GEMM_F32_KC 0
#endif
#ifndef PE_GEMM_F32_NBUF
#define PE_GEMM_F32_NBUF 1
#endif

namespace pe {

// persist: 0 launches one block per tile; > 0 caps the grid at that many
// blocks per CU; < 0 caps it at this kernel's own occupancy (every block
// resident, each walking several tiles).
template <int BM, int BN, int AL, int BL>
static hipError_t go(const GemmArgs& g, int persist, hipStream_t s) {
    const auto kernel = gemm_kernel<F32, BM, BN, PE_GEMM_F32_BK, bool(PE_GEMM_F32_KC), PE_GEMM_F32_NBUF, AL, BL>;
    GemmArgs a = g;
    if (persist != 0) {
        static const int resident = [&] {
            int n = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kernel),
                                                             kGemmThreads, 0) != hipSuccess || n < 1)
                n = 1;
            return n;
        }();
        const uint32_t cap = uint32_t(cu_count()) * uint32_t(persist < 0 ? resident : persist);
        if (a.grid > cap) a.grid = cap;
    }
    if (a.grid > 0x7fffffffu) a.grid = 0x7fffffffu;  // grid limit; the tile walk strides over the rest
    hipLaunchKernelGGL(kernel, dim3(a.grid), dim3(kGemmThreads), 0, s, a);
    return hipGetLastError();
}

template <int BM, int BN, int AL>
static hipError_t go_b(int bl, const GemmArgs& g, int persist, hipStream_t s) {
    switch (bl) {
        case L_MN: return go<BM, BN, AL, L_MN>(g, persist, s);
        case L_K: return go<BM, BN, AL, L_K>(g, persist, s);
        default: return go<BM, BN, AL, L_GENERIC>(g, persist, s);
    }
}

template <int BM, int BN>
static hipError_t go_a(int al, int bl, const GemmArgs& g, int persist, hipStream_t s) {
    switch (al) {
        case L_MN: return go_b<BM, BN, L_MN>(bl, g, persist, s);
        case L_K: return go_b<BM, BN, L_K>(bl, g, persist, s);
        default: return go_b<BM, BN, L_GENERIC>(bl, g, persist, s);
    }
}

int gemm_bk_f16();
int gemm_bk(int dtype) { return dtype == PE_F32 ? PE_GEMM_F32_BK : gemm_bk_f16(); }

template <int BM, int BN>
static int occ() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&gemm_kernel<F32, BM, BN, PE_GEMM_F32_BK, bool(PE_GEMM_F32_KC), PE_GEMM_F32_NBUF, L_MN, L_MN>),
            kGemmThreads, 0) != hipSuccess || n < 1)
        n = 1;
    return n;
}

int gemm_occupancy_f32(int bm, int bn) {
    static const int o[6] = {occ<64, 64>(),   occ<128, 128>(), occ<256, 128>(),
                             occ<128, 256>(), occ<192, 128>(), occ<128, 192>()};
    if (bm == 256) return o[2];
    if (bn == 256) return o[3];
    if (bm == 192) return o[4];
    if (bn == 192) return o[5];
    return bm == 128 ? o[1] : o[0];
}

// Direct-load kernels: 64x64 and 128x128 tiles held to four resident blocks
// per CU, 256x128 / 128x256 tiles in two register budgets (two or three
// resident blocks per CU; which one fits a grid is decided in choose()).
template <int BM, int BN, int MINB>
static const void* dl_kernel_ab(int al, int bl) {
    if (al == L_MN)
        return bl == L_MN ? reinterpret_cast<const void*>(&gemm_dl_kernel<BM, BN, L_MN, L_MN, MINB>)
                          : reinterpret_cast<const void*>(&gemm_dl_kernel<BM, BN, L_MN, L_K, MINB>);
    return bl == L_MN ? reinterpret_cast<const void*>(&gemm_dl_kernel<BM, BN, L_K, L_MN, MINB>)
                      : reinterpret_cast<const void*>(&gemm_dl_kernel<BM, BN, L_K, L_K, MINB>);
}

static const void* dl_kernel(int bm, int bn, int minb, int al, int bl) {
    if (bm == 256) return minb == 2 ? dl_kernel_ab<256, 128, 2>(al, bl) : dl_kernel_ab<256, 128, 3>(al, bl);
    if (bn == 256) return minb == 2 ? dl_kernel_ab<128, 256, 2>(al, bl) : dl_kernel_ab<128, 256, 3>(al, bl);
    return bm == 128 ? dl_kernel_ab<128, 128, 4>(al, bl) : dl_kernel_ab<64, 64, 4>(al, bl);
}

static int dl_index(int bm, int bn, int minb, int al, int bl) {
    const int t = bm == 256 ? (minb == 2 ? 2 : 3) : bn == 256 ? (minb == 2 ? 4 : 5) : bm == 128 ? 1 : 0;
    return (t * 2 + (al == L_K)) * 2 + (bl == L_K);
}

// Instantiations whose register allocation spilled more than this many bytes
// per lane are never launched.  The 128x256 tile at three blocks per CU
// spills one lane offset (8 bytes, reloaded once per slab) and runs config 2
// as fast as the spill-free variants; larger spills sit inside the MFMA loop.
#ifndef PE_GEMM_DL_MAX_SPILL
#define PE_GEMM_DL_MAX_SPILL 16
#endif

int gemm_dl_resident(int bm, int bn, int minb, int al, int bl) {
    static int cache[6 * 4];
    static bool init = false;
    if (!init) {
        for (int& c : cache) c = -1;
        init = true;
    }
    int& c = cache[dl_index(bm, bn, minb, al, bl)];
    if (c < 0) {
        const void* k = dl_kernel(bm, bn, minb, al, bl);
        hipFuncAttributes at{};
        int n = 0;
        if (hipFuncGetAttributes(&at, k) != hipSuccess || at.localSizeBytes > PE_GEMM_DL_MAX_SPILL ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGemmThreads, 0) != hipSuccess || n < 1)
            n = 0;
        c = n;
    }
    return c;
}

bool gemm_dl_eligible(int al, int bl, int64_t M, int64_t N, int64_t K) {
    if (!PE_GEMM_DL) return false;
    if (al != L_MN && al != L_K) return false;
    if (bl != L_MN && bl != L_K) return false;
    if (al == L_MN && M % 4 != 0) return false;
    if (bl == L_MN && N % 4 != 0) return false;
    if ((al == L_K || bl == L_K) && K % 4 != 0) return false;
    return true;
}

hipError_t launch_gemm_f32_dl(int bm, int bn, int minb, int al, int bl, const GemmArgs& g, hipStream_t s) {
    const int resident = gemm_dl_resident(bm, bn, minb, al, bl);
    if (resident < 1) return hipErrorInvalidConfiguration;
    GemmArgs a = g;
    const uint32_t cap = uint32_t(cu_count()) * uint32_t(resident);
    if (a.grid > cap) a.grid = cap;
    void* args[] = {&a};
    return hipLaunchKernel(dl_kernel(bm, bn, minb, al, bl), dim3(a.grid), dim3(kGemmThreads), args, 0, s);
}

hipError_t launch_gemm_f32(int bm, int bn, int al, int bl, int persist, const GemmArgs& g,
                           hipStream_t s) {
    if (bm == 256) return go_a<256, 128>(al, bl, g, persist, s);
    if (bn == 256) return go_a<128, 256>(al, bl, g, persist, s);
    if (bm == 192) return go_a<192, 128>(al, bl, g, persist, s);
    if (bn == 192) return go_a<128, 192>(al, bl, g, persist, s);
    return bm == 128 ? go_a<128, 128>(al, bl, g, persist, s) : go_a<64, 64>(al, bl, g, persist, s);
}

}  // namespace pe
