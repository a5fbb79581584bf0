#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 65536;
    static constexpr unsigned from_shape[3] = {8, 128, 64};
    static constexpr unsigned to_shape[3] = {8, 128, 64};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {8192, 64, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 65536;
    static constexpr unsigned from_shape[3] = {8, 128, 64};
    static constexpr unsigned to_shape[3] = {8, 64, 128};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {8192, 1, 64};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 131072;
    static constexpr unsigned from_shape[3] = {8, 128, 128};
    static constexpr unsigned to_shape[3] = {8, 128, 128};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {16384, 128, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 128;
    static const unsigned n_free1 = 128;
    static const unsigned n_contract = 64;
    static const unsigned n_inplace = 8;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
