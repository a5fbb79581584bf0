#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 135;
    static constexpr unsigned from_shape[3] = {3, 5, 9};
    static constexpr unsigned to_shape[3] = {3, 5, 9};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {45, 9, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 459;
    static constexpr unsigned from_shape[3] = {3, 17, 9};
    static constexpr unsigned to_shape[3] = {3, 9, 17};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {153, 1, 9};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 255;
    static constexpr unsigned from_shape[3] = {3, 5, 17};
    static constexpr unsigned to_shape[3] = {3, 5, 17};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {85, 17, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 5;
    static const unsigned n_free1 = 17;
    static const unsigned n_contract = 9;
    static const unsigned n_inplace = 3;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
