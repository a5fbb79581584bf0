#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 51200;
    static constexpr unsigned from_shape[3] = {4, 200, 64};
    static constexpr unsigned to_shape[3] = {4, 200, 64};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {12800, 64, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 32768;
    static constexpr unsigned from_shape[3] = {4, 64, 128};
    static constexpr unsigned to_shape[3] = {4, 64, 128};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {8192, 128, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 102400;
    static constexpr unsigned from_shape[3] = {4, 200, 128};
    static constexpr unsigned to_shape[3] = {4, 200, 128};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {25600, 128, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 200;
    static const unsigned n_free1 = 128;
    static const unsigned n_contract = 64;
    static const unsigned n_inplace = 4;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
