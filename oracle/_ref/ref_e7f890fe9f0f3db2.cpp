#include "cpu_einsum.h"

struct config_tpose_inp0 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 777000;
    static constexpr unsigned from_shape[3] = {1, 777, 1000};
    static constexpr unsigned to_shape[3] = {1, 1000, 777};
    static constexpr unsigned perm[3] = {0, 2, 1};
    static constexpr unsigned perm_strides[3] = {777000, 1, 1000};
};

struct config_tpose_inp1 {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 1193472;
    static constexpr unsigned from_shape[3] = {1, 777, 1536};
    static constexpr unsigned to_shape[3] = {1, 777, 1536};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {1193472, 1536, 1};
};

struct config_tpose_out {
    static constexpr unsigned dims = 3;
    static constexpr unsigned N = 1536000;
    static constexpr unsigned from_shape[3] = {1, 1000, 1536};
    static constexpr unsigned to_shape[3] = {1, 1000, 1536};
    static constexpr unsigned perm[3] = {0, 1, 2};
    static constexpr unsigned perm_strides[3] = {1536000, 1536, 1};
};

struct config_einsum {
    typedef config_tpose_inp0 tpose_inp0_config;
    typedef config_tpose_inp1 tpose_inp1_config;
    typedef config_tpose_out tpose_out_conf;
    static const unsigned n_free0 = 1000;
    static const unsigned n_free1 = 1536;
    static const unsigned n_contract = 777;
    static const unsigned n_inplace = 1;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::einsum<float, config_einsum>(input0, input1, output);
}
