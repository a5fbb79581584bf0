#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 1024;
    static constexpr unsigned from_shape[4] = {2, 8, 4, 16};
    static constexpr unsigned to_shape[4] = {8, 16, 2, 4};
    static constexpr unsigned perm[4] = {1, 3, 0, 2};
    static constexpr unsigned perm_strides[4] = {64, 1, 512, 16};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 128;
    static constexpr unsigned from_shape[2] = {8, 16};
    static constexpr unsigned to_shape[2] = {8, 16};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {16, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 1024;
    static constexpr unsigned from_shape[4] = {8, 16, 2, 4};
    static constexpr unsigned to_shape[4] = {2, 8, 4, 16};
    static constexpr unsigned perm[4] = {2, 0, 3, 1};
    static constexpr unsigned perm_strides[4] = {4, 128, 1, 8};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 8;
    static const unsigned n_free1 = 1;
    static const unsigned n_contract = 1;
    static const unsigned n_inplace = 128;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
