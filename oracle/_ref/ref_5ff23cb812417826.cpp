#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 131072;
    static constexpr unsigned from_shape[4] = {4, 128, 4, 64};
    static constexpr unsigned to_shape[4] = {4, 4, 64, 128};
    static constexpr unsigned perm[4] = {0, 2, 3, 1};
    static constexpr unsigned perm_strides[4] = {32768, 64, 1, 256};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 131072;
    static constexpr unsigned from_shape[4] = {4, 128, 4, 64};
    static constexpr unsigned to_shape[4] = {4, 4, 128, 64};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {32768, 64, 256, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 65536;
    static constexpr unsigned from_shape[4] = {4, 4, 64, 64};
    static constexpr unsigned to_shape[4] = {4, 4, 64, 64};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {16384, 4096, 64, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 64;
    static const unsigned n_free1 = 64;
    static const unsigned n_contract = 128;
    static const unsigned n_inplace = 16;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
