#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 15;
    static constexpr unsigned from_shape[2] = {3, 5};
    static constexpr unsigned to_shape[2] = {3, 5};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {5, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 24;
    static constexpr unsigned from_shape[2] = {4, 6};
    static constexpr unsigned to_shape[2] = {4, 6};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {6, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 360;
    static constexpr unsigned from_shape[4] = {3, 5, 4, 6};
    static constexpr unsigned to_shape[4] = {3, 4, 5, 6};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {120, 6, 24, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 15;
    static const unsigned n_free1 = 24;
    static const unsigned n_contract = 1;
    static const unsigned n_inplace = 1;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
