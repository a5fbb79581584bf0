#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 15400;
    static constexpr unsigned from_shape[3] = {2, 77, 100};
    static constexpr unsigned to_shape[3] = {2, 100, 77};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {7700, 1, 100};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 23562;
    static constexpr unsigned from_shape[3] = {2, 77, 153};
    static constexpr unsigned to_shape[3] = {2, 77, 153};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {11781, 153, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 30600;
    static constexpr unsigned from_shape[3] = {2, 100, 153};
    static constexpr unsigned to_shape[3] = {2, 100, 153};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {15300, 153, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 100;
    static const unsigned n_free1 = 153;
    static const unsigned n_contract = 77;
    static const unsigned n_inplace = 2;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
