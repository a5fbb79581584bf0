#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 120;
    static constexpr unsigned from_shape[3] = {5, 4, 6};
    static constexpr unsigned to_shape[3] = {6, 4, 5};
    static constexpr unsigned perm[3] = {2, 1, 0};
    static constexpr unsigned perm_strides[3] = {1, 6, 24};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 60;
    static constexpr unsigned from_shape[3] = {3, 4, 5};
    static constexpr unsigned to_shape[3] = {4, 5, 3};
    static constexpr unsigned perm[3] = {1, 2, 0};
    static constexpr unsigned perm_strides[3] = {5, 1, 20};
};

struct config_tpose_out {
    static constexpr unsigned dims = 2;
    static constexpr unsigned N = 18;
    static constexpr unsigned from_shape[2] = {6, 3};
    static constexpr unsigned to_shape[2] = {6, 3};
    static constexpr unsigned perm[2] = {0, 1};
    static constexpr unsigned perm_strides[2] = {3, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 6;
    static const unsigned n_free1 = 3;
    static const unsigned n_contract = 20;
    static const unsigned n_inplace = 1;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
