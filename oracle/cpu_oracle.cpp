// CPU ORACLE -- test infrastructure only.
//
// A clean-room C++ restatement of the reference's CPU einsum path
// (`src/pto_einsum/include/cpu_einsum.h`), used as the parity checker for the
// MI355X kernels.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load it; the product never does.
//
// Parity pins (see oracle/README.md for the full list): every function is
// checked bit-for-bit against the reference header compiled from its own
// source (oracle/_ref, when /root/reference is present), against committed
// golden vectors made from that build, against torch.permute / torch.mul
// closed forms, against a brute-force float32 loop on tiny shapes and, within
// a tolerance, against a float64 einsum.
//
// Build: g++ -O3 -std=c++17 -ffp-contract=off -shared -fPIC (no -march, so no
// FMA contraction, matching the reference's `g++ -O3 -shared -fPIC -std=c++17`
// at builder.py:705-709 on x86-64).  Never build with -ffast-math: the
// summation order and subnormals must stay exactly IEEE.
#include <cstddef>
#include <cstdint>
#include <vector>

namespace {

// Destination flat index -> source flat index for a permutation copy:
//   src = sum_k ((i / prod_{j>k} to_shape[j]) mod to_shape[k]) * perm_strides[k]
// cpu_einsum.h:35-43 (transfer_idx), widened to 64-bit indices.
inline int64_t source_index(int64_t i, int dims, const int64_t* to_shape,
                            const int64_t* perm_strides) {
    int64_t src = 0;
    for (int k = dims - 1; k >= 0; --k) {
        src += (i % to_shape[k]) * perm_strides[k];
        i /= to_shape[k];
    }
    return src;
}

template <typename T>
void gather(const T* data, T* res, int64_t n, int dims, const int64_t* to_shape,
            const int64_t* perm_strides) {
    // cpu_einsum.h:45-51 (transpose): res[i] = data[source_index(i)].
    for (int64_t i = 0; i < n; ++i) res[i] = data[source_index(i, dims, to_shape, perm_strides)];
}

}  // namespace

extern "C" {

// Permutation gather of 4-byte and 2-byte elements (bit copies).
void oracle_gather_b32(const uint32_t* data, uint32_t* res, int64_t n, int dims,
                       const int64_t* to_shape, const int64_t* perm_strides) {
    gather(data, res, n, dims, to_shape, perm_strides);
}
void oracle_gather_b16(const uint16_t* data, uint16_t* res, int64_t n, int dims,
                       const int64_t* to_shape, const int64_t* perm_strides) {
    gather(data, res, n, dims, to_shape, perm_strides);
}

// The batched triple loop of cpu_einsum.h:53-83 on already-permuted operands:
//   A is [I, L0, C], B is [I, C, L1], R is [I, L0, L1];
//   R[i,l0,l1] = (((0 + A[.,0]*B[0,.]) + A[.,1]*B[1,.]) + ...) in float32,
// one rounding per product and one per addition, c ascending.
void oracle_bmm_f32(const float* A, const float* B, float* R, int64_t I, int64_t L0,
                    int64_t L1, int64_t C) {
    for (int64_t i = 0; i < I; ++i) {
        for (int64_t l0 = 0; l0 < L0; ++l0) {
            const float* arow = A + (i * L0 + l0) * C;
            for (int64_t l1 = 0; l1 < L1; ++l1) {
                const float* bcol = B + i * L1 * C + l1;
                float acc = 0.0f;
                for (int64_t c = 0; c < C; ++c) {
                    float prod = arow[c] * bcol[c * L1];
                    acc = acc + prod;
                }
                R[(i * L0 + l0) * L1 + l1] = acc;
            }
        }
    }
}

// Selected outputs of the same triple loop, addressed straight in the raw
// (unpermuted) operands: for output q, A element c sits at a_base[q] +
// sum over contract axes of index*stride, enumerated in recipe contract order
// (row-major over k_shape); likewise B.  Used for full-size spot checks whose
// values are bit-identical to the full oracle at those positions.
void oracle_sampled_f32(const float* in0, const float* in1, int64_t nq,
                        const int64_t* a_base, const int64_t* b_base, int kdims,
                        const int64_t* k_shape, const int64_t* k_sa, const int64_t* k_sb,
                        float* res) {
    int64_t C = 1;
    for (int d = 0; d < kdims; ++d) C *= k_shape[d];
    std::vector<int64_t> offa(C), offb(C);
    for (int64_t c = 0; c < C; ++c) {
        int64_t rem = c, oa = 0, ob = 0;
        for (int d = kdims - 1; d >= 0; --d) {
            int64_t x = rem % k_shape[d];
            rem /= k_shape[d];
            oa += x * k_sa[d];
            ob += x * k_sb[d];
        }
        offa[c] = oa;
        offb[c] = ob;
    }
    for (int64_t q = 0; q < nq; ++q) {
        float acc = 0.0f;
        for (int64_t c = 0; c < C; ++c) {
            float prod = in0[a_base[q] + offa[c]] * in1[b_base[q] + offb[c]];
            acc = acc + prod;
        }
        res[q] = acc;
    }
}

// cpu_einsum.h:87-92 (elementwise_mul): one float32 multiply per element.
void oracle_hadamard_f32(const float* a, const float* b, float* r, int64_t n) {
    for (int64_t i = 0; i < n; ++i) r[i] = a[i] * b[i];
}

}  // extern "C"
