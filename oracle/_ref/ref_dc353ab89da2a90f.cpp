#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 28;
    static constexpr unsigned from_shape[2] = {4, 7};
    static constexpr unsigned to_shape[2] = {4, 7};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {7, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 36;
    static constexpr unsigned from_shape[2] = {4, 9};
    static constexpr unsigned to_shape[2] = {4, 9};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {9, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 252;
    static constexpr unsigned from_shape[3] = {4, 7, 9};
    static constexpr unsigned to_shape[3] = {4, 7, 9};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {63, 9, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 7;
    static const unsigned n_free1 = 9;
    static const unsigned n_contract = 1;
    static const unsigned n_inplace = 4;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
