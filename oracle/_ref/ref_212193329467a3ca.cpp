#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 4096;
    static constexpr unsigned from_shape[3] = {8, 16, 32};
    static constexpr unsigned to_shape[3] = {8, 16, 32};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {512, 32, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 32768;
    static constexpr unsigned from_shape[3] = {16, 32, 64};
    static constexpr unsigned to_shape[3] = {16, 32, 64};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {2048, 64, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 512;
    static constexpr unsigned from_shape[2] = {8, 64};
    static constexpr unsigned to_shape[2] = {8, 64};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {64, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 8;
    static const unsigned n_free1 = 64;
    static const unsigned n_contract = 512;
    static const unsigned n_inplace = 1;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
