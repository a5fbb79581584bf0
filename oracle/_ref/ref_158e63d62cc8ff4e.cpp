#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 32768;
    static constexpr unsigned from_shape[4] = {4, 16, 8, 64};
    static constexpr unsigned to_shape[4] = {4, 8, 16, 64};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {8192, 64, 512, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 32768;
    static constexpr unsigned from_shape[4] = {4, 16, 8, 64};
    static constexpr unsigned to_shape[4] = {4, 8, 64, 16};
    static constexpr unsigned perm[4] = {0, 2, 3, 1};
    static constexpr unsigned perm_strides[4] = {8192, 64, 1, 512};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 8192;
    static constexpr unsigned from_shape[4] = {4, 8, 16, 16};
    static constexpr unsigned to_shape[4] = {4, 16, 8, 16};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {2048, 16, 256, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 16;
    static const unsigned n_free1 = 16;
    static const unsigned n_contract = 64;
    static const unsigned n_inplace = 32;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
