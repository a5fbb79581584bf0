// float32 instantiations of the batched MFMA GEMM (v_mfma_f32_32x32x2_f32).
#include "pe_gemm_kernel.h"

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

hipError_t launch_gemm_f32(int bm, int bn, int al, int bl, int persist, const GemmArgs& g,
                           hipStream_t s) {
    if (bm == 256) return go_a<256, 128>(al, bl, g, persist, s);
    if (bn == 256) return go_a<128, 256>(al, bl, g, persist, s);
    if (bm == 192) return go_a<192, 128>(al, bl, g, persist, s);
    if (bn == 192) return go_a<128, 192>(al, bl, g, persist, s);
    return bm == 128 ? go_a<128, 128>(al, bl, g, persist, s) : go_a<64, 64>(al, bl, g, persist, s);
}

}  // namespace pe
