#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 12288;
    static constexpr unsigned from_shape[4] = {2, 48, 4, 32};
    static constexpr unsigned to_shape[4] = {2, 4, 48, 32};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {6144, 32, 128, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 10240;
    static constexpr unsigned from_shape[4] = {2, 40, 4, 32};
    static constexpr unsigned to_shape[4] = {2, 4, 32, 40};
    static constexpr unsigned perm[4] = {0, 2, 3, 1};
    static constexpr unsigned perm_strides[4] = {5120, 32, 1, 128};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 15360;
    static constexpr unsigned from_shape[4] = {2, 4, 48, 40};
    static constexpr unsigned to_shape[4] = {2, 48, 4, 40};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {7680, 40, 1920, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 48;
    static const unsigned n_free1 = 40;
    static const unsigned n_contract = 32;
    static const unsigned n_inplace = 8;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
