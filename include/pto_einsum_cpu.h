/*
 * pto_einsum_cpu.h -- the CPU route of the einsum API (device="cpu").
 *
 * Reference counterpart: include/cpu_einsum.h (the reference's CPU path,
 * selected with device="cpu", README.md:129-134).  Same contract: a
 * per-shape JIT library includes this header with compile-time configuration
 * structs (the config_tpose_* / config_einsum layout of templates.py:1-62)
 * and computes, single-threaded,
 *
 *   A = permute(input0, tpose_inp0)          -> [I, L0, C]
 *   B = permute(input1, tpose_inp1)          -> [I, C, L1]
 *   R[i,l0,l1] = sum_{c ascending} A*B       (float32, starting from +0)
 *   output = permute(R, tpose_out)
 *
 * or, for the Hadamard route, output[i] = input0[i] * input1[i].  Built with
 * g++ -O3 -std=c++17 and no FMA, so every product and partial sum rounds to
 * float32 exactly as the reference CPU route does.
 */
#ifndef PTO_EINSUM_CPU_H
#define PTO_EINSUM_CPU_H

#include <cstddef>
#include <cstdint>
#include <vector>

namespace pto_einsum_cpu {

// Copy `src` into the row-major destination described by CFG: destination
// axis d walks the source with stride CFG::perm_strides[d].  An odometer
// carries the source offset so no division is done per element.
template <typename T, typename CFG>
void permute(const T* src, T* dst) {
    constexpr unsigned D = CFG::dims;
    if (D == 0) {
        dst[0] = src[0];
        return;
    }
    unsigned long long idx[D > 0 ? D : 1] = {};
    unsigned long long off = 0;
    for (unsigned long long o = 0; o < CFG::N; ++o) {
        dst[o] = src[off];
        for (int d = int(D) - 1; d >= 0; --d) {
            off += CFG::perm_strides[d];
            if (++idx[d] < CFG::to_shape[d]) break;
            off -= CFG::perm_strides[d] * CFG::to_shape[d];
            idx[d] = 0;
        }
    }
}

template <typename T, typename CFG>
void einsum(const T* in0, const T* in1, float* out) {
    using C0 = typename CFG::tpose_inp0_config;
    using C1 = typename CFG::tpose_inp1_config;
    using CO = typename CFG::tpose_out_conf;
    std::vector<T> a(C0::N), b(C1::N);
    std::vector<float> r(CO::N);
    permute<T, C0>(in0, a.data());
    permute<T, C1>(in1, b.data());
    const unsigned long long I = CFG::n_inplace, L0 = CFG::n_free0, L1 = CFG::n_free1,
                             C = CFG::n_contract;
    for (unsigned long long i = 0; i < I; ++i) {
        const T* ab = a.data() + i * L0 * C;
        const T* bb = b.data() + i * C * L1;
        float* rb = r.data() + i * L0 * L1;
        for (unsigned long long m = 0; m < L0; ++m) {
            for (unsigned long long n = 0; n < L1; ++n) {
                float s = 0.0f;
                for (unsigned long long k = 0; k < C; ++k)
                    s += static_cast<float>(ab[m * C + k]) * static_cast<float>(bb[k * L1 + n]);
                rb[m * L1 + n] = s;
            }
        }
    }
    permute<float, CO>(r.data(), out);
}

template <typename T, typename CFG>
void hadamard(const T* in0, const T* in1, float* out) {
    for (unsigned long long i = 0; i < CFG::N; ++i)
        out[i] = static_cast<float>(in0[i]) * static_cast<float>(in1[i]);
}

}  // namespace pto_einsum_cpu

#endif /* PTO_EINSUM_CPU_H */
