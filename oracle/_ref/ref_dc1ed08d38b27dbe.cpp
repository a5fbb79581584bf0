#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 262144;
    static constexpr unsigned from_shape[4] = {4, 128, 8, 64};
    static constexpr unsigned to_shape[4] = {4, 8, 128, 64};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {65536, 64, 512, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 131072;
    static constexpr unsigned from_shape[4] = {4, 8, 64, 64};
    static constexpr unsigned to_shape[4] = {4, 8, 64, 64};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {32768, 4096, 64, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 262144;
    static constexpr unsigned from_shape[4] = {4, 8, 128, 64};
    static constexpr unsigned to_shape[4] = {4, 128, 8, 64};
    static constexpr unsigned perm[4] = {0, 2, 1, 3};
    static constexpr unsigned perm_strides[4] = {65536, 64, 8192, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 128;
    static const unsigned n_free1 = 64;
    static const unsigned n_contract = 64;
    static const unsigned n_inplace = 32;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
