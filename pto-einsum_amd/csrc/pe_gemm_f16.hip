// float16 instantiations of the batched MFMA GEMM (v_mfma_f32_32x32x16_f16,
// float32 accumulation; every fp16 x fp16 product is exact in float32).
#include "pe_gemm_kernel.h"

namespace pe {

template <int BM, int AL, int BL>
static hipError_t go(const GemmArgs& g, hipStream_t s) {
    hipLaunchKernelGGL((gemm_kernel<F16, BM, BM, AL, BL>), dim3(g.total_blocks),
                       dim3(kGemmThreads), 0, s, g);
    return hipGetLastError();
}

template <int BM, int AL>
static hipError_t go_b(int bl, const GemmArgs& g, hipStream_t s) {
    switch (bl) {
        case L_MN: return go<BM, AL, L_MN>(g, s);
        case L_K: return go<BM, AL, L_K>(g, s);
        default: return go<BM, AL, L_GENERIC>(g, s);
    }
}

template <int BM>
static hipError_t go_a(int al, int bl, const GemmArgs& g, hipStream_t s) {
    switch (al) {
        case L_MN: return go_b<BM, L_MN>(bl, g, s);
        case L_K: return go_b<BM, L_K>(bl, g, s);
        default: return go_b<BM, L_GENERIC>(bl, g, s);
    }
}

hipError_t launch_gemm_f16(int bm, int al, int bl, const GemmArgs& g, hipStream_t s) {
    return bm == 128 ? go_a<128>(al, bl, g, s) : go_a<64>(al, bl, g, s);
}

}  // namespace pe
