#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 16384;
    static constexpr unsigned from_shape[4] = {2, 64, 4, 32};
    static constexpr unsigned to_shape[4] = {2, 4, 64, 32};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {8192, 32, 128, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 24576;
    static constexpr unsigned from_shape[4] = {2, 96, 4, 32};
    static constexpr unsigned to_shape[4] = {2, 4, 32, 96};
    static constexpr unsigned perm[4] = {0, 2, 3, 1};
    static constexpr unsigned perm_strides[4] = {12288, 32, 1, 128};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 49152;
    static constexpr unsigned from_shape[4] = {2, 4, 64, 96};
    static constexpr unsigned to_shape[4] = {2, 64, 4, 96};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {24576, 96, 6144, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 64;
    static const unsigned n_free1 = 96;
    static const unsigned n_contract = 32;
    static const unsigned n_inplace = 8;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
