#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 16640;
    static constexpr unsigned from_shape[4] = {2, 4, 16, 130};
    static constexpr unsigned to_shape[4] = {2, 4, 16, 130};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {8320, 2080, 130, 1};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 266240;
    static constexpr unsigned from_shape[4] = {2, 4, 256, 130};
    static constexpr unsigned to_shape[4] = {2, 4, 130, 256};
    static constexpr unsigned perm[4] = {0, 1, 3, 2};
    static constexpr unsigned perm_strides[4] = {133120, 33280, 1, 130};
};

struct config_tpose_out {
    static constexpr unsigned dims = 4;
    static constexpr unsigned N = 32768;
    static constexpr unsigned from_shape[4] = {2, 4, 16, 256};
    static constexpr unsigned to_shape[4] = {2, 4, 16, 256};
    static constexpr unsigned perm[4] = {0, 1, 2, 3};
    static constexpr unsigned perm_strides[4] = {16384, 4096, 256, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 16;
    static const unsigned n_free1 = 256;
    static const unsigned n_contract = 130;
    static const unsigned n_inplace = 8;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
