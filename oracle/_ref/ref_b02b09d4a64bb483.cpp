#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 210;
    static constexpr unsigned from_shape[3] = {5, 6, 7};
    static constexpr unsigned to_shape[3] = {5, 6, 7};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {42, 7, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 56;
    static constexpr unsigned from_shape[2] = {7, 8};
    static constexpr unsigned to_shape[2] = {7, 8};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {8, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 240;
    static constexpr unsigned from_shape[3] = {5, 6, 8};
    static constexpr unsigned to_shape[3] = {5, 8, 6};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {48, 1, 8};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 30;
    static const unsigned n_free1 = 8;
    static const unsigned n_contract = 7;
    static const unsigned n_inplace = 1;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
