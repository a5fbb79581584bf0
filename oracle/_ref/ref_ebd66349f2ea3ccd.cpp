#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 12288;
    static constexpr unsigned from_shape[3] = {24, 32, 16};
    static constexpr unsigned to_shape[3] = {24, 16, 32};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {512, 1, 16};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 49152;
    static constexpr unsigned from_shape[3] = {24, 32, 64};
    static constexpr unsigned to_shape[3] = {24, 32, 64};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {2048, 64, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 24576;
    static constexpr unsigned from_shape[3] = {24, 16, 64};
    static constexpr unsigned to_shape[3] = {24, 16, 64};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {1024, 64, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 16;
    static const unsigned n_free1 = 64;
    static const unsigned n_contract = 32;
    static const unsigned n_inplace = 24;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
