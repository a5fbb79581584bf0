#include "cpu_einsum.h"

struct config_elementwise {
    static const unsigned N = 1000;
};

extern "C" void run_einsum(const float* input0, const float* input1, float* output, void* stream) {
    cpu::elementwise_mul<float, config_elementwise>(input0, input1, output);
}
