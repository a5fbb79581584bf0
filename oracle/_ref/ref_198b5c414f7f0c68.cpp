#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 5120;
    static constexpr unsigned from_shape[4] = {2, 8, 16, 20};
    static constexpr unsigned to_shape[4] = {2, 8, 16, 20};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {2560, 320, 20, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 7680;
    static constexpr unsigned from_shape[4] = {2, 8, 24, 20};
    static constexpr unsigned to_shape[4] = {2, 8, 20, 24};
    static constexpr unsigned perm[4] = {0, 1, 3, 2};
    static constexpr unsigned perm_strides[4] = {3840, 480, 1, 20};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 6144;
    static constexpr unsigned from_shape[4] = {2, 8, 16, 24};
    static constexpr unsigned to_shape[4] = {2, 8, 16, 24};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {3072, 384, 24, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 16;
    static const unsigned n_free1 = 24;
    static const unsigned n_contract = 20;
    static const unsigned n_inplace = 16;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
