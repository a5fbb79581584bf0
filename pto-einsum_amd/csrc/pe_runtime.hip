// Plan executor and runtime plumbing of the einsum core library.
//
// Reference counterparts: einsum_setup / einsum_exec / einsum_teardown /
// einsum (pto_einsum.h:193-290).  The reference allocates a workspace for
// Phase A/C staging and launches one fused kernel whose phases are separated
// by cross-core barriers.  Here a plan is a short sequence of launches on one
// stream -- stream order replaces the barriers -- and the workspace is only
// allocated when an operand cannot be read in place (a free or contracted
// axis group that does not collapse to one stride), when the output needs a
// separate permutation, or for split-K partial tiles.
#include "pe_common.h"

#include <mutex>

namespace pe {

int validate_product(const pe_product_desc& d);
int validate_permute(const pe_permute_desc& d);
int validate_gemm(const pe_gemm_desc& d);

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return int(e);
}

int cu_count() {
    static int cache[64] = {0};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

namespace {

constexpr int64_t kMinWorkspace = 256;

int64_t gemm_ws_offset(const pe_einsum_plan& p) {
    return (p.ws_bytes + 255) / 256 * 256;
}

int64_t plan_workspace_bytes(const pe_einsum_plan& p) {
    if (p.route != PE_ROUTE_GEMM) return kMinWorkspace;
    int64_t total = gemm_ws_offset(p) + pe_gemm_workspace_bytes(&p.gemm);
    return total < kMinWorkspace ? kMinWorkspace : total;
}

}  // namespace
}  // namespace pe

extern "C" const char* pe_last_error(void) { return pe::g_last_error.c_str(); }

extern "C" int pe_device_cu_count(void) { return pe::cu_count(); }

extern "C" const char* pe_version(void) { return "pto-einsum-amd 0.2.0 (gfx950)"; }

extern "C" int64_t pe_einsum_workspace_bytes(const pe_einsum_plan* p) {
    return p ? pe::plan_workspace_bytes(*p) : 0;
}

extern "C" void* pe_einsum_setup(const pe_einsum_plan* p, void* stream) {
    (void)stream;
    if (!p) {
        pe::fail(PE_ERR_INVALID, "setup: null plan");
        return nullptr;
    }
    void* ws = nullptr;
    hipError_t e = hipMalloc(&ws, size_t(pe::plan_workspace_bytes(*p)));
    if (e != hipSuccess) {
        pe::hip_status(e, "hipMalloc(workspace)");
        return nullptr;
    }
    return ws;
}

extern "C" int pe_einsum_teardown(void* ws) {
    if (!ws) return PE_OK;
    // Launches that use the workspace may still be queued on any stream.
    PE_CHECK_HIP(hipDeviceSynchronize());
    PE_CHECK_HIP(hipFree(ws));
    return PE_OK;
}

extern "C" int pe_einsum_exec(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                              void* ws, void* stream) {
    using namespace pe;
    if (!p) return fail(PE_ERR_INVALID, "exec: null plan");
    if (p->skip_phases < 0 || p->skip_phases > 7 || p->reserved != 0)
        return fail(PE_ERR_INVALID, "exec: skip_phases must be in [0, 7] and reserved 0");
    const bool run_a = !(p->skip_phases & 1), run_b = !(p->skip_phases & 2), run_c = !(p->skip_phases & 4);
    if (p->route == PE_ROUTE_PRODUCT) return run_b ? pe_product(&p->product, in0, in1, out, stream) : PE_OK;
    if (p->route != PE_ROUTE_GEMM) return fail(PE_ERR_INVALID, "exec: unknown route");
    char* w = static_cast<char*>(ws);
    const bool staged = p->gather0 || p->gather1 || p->scatter_out;
    const int64_t gws = pe_gemm_workspace_bytes(&p->gemm);
    if ((staged || gws > 0) && !w) return fail(PE_ERR_WORKSPACE, "exec: plan needs a workspace");
    const void* a = in0;
    const void* b = in1;
    int st;
    if (p->gather0) {
        st = run_a ? pe_permute(&p->perm0, in0, w + p->ws0_off, stream) : PE_OK;
        if (st != PE_OK) return st;
        a = w + p->ws0_off;
    }
    if (p->gather1) {
        st = run_a ? pe_permute(&p->perm1, in1, w + p->ws1_off, stream) : PE_OK;
        if (st != PE_OK) return st;
        b = w + p->ws1_off;
    }
    float* c = p->scatter_out ? reinterpret_cast<float*>(w + p->wsout_off) : out;
    st = run_b ? pe_gemm(&p->gemm, a, b, c, w ? w + gemm_ws_offset(*p) : nullptr, gws, stream) : PE_OK;
    if (st != PE_OK) return st;
    if (p->scatter_out && run_c) {
        st = pe_permute(&p->perm_out, c, out, stream);
        if (st != PE_OK) return st;
    }
    return PE_OK;
}

// ------------------------------------------------ allocation-free executor --
//
// Device scratch of pe_einsum_exec_noalloc: a file-scope device array that
// every GPU this library runs on holds (PE_NOALLOC_SCRATCH_BYTES of it) until
// the process ends.  In host code `scratch` names a host-side stand-in, not a
// device address: the device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that pointer is
// ever handed to a launch.
static __device__ __align__(256) char scratch[PE_NOALLOC_SCRATCH_BYTES];

namespace pe {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// Device address of the current device's copy of `scratch`.
int device_scratch(void** out) {
    int dev = 0;
    PE_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(PE_ERR_UNSUPPORTED, "exec_noalloc: device ordinal above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        PE_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return fail(PE_ERR_WORKSPACE, "exec_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return PE_OK;
}

}  // namespace
}  // namespace pe

extern "C" int pe_einsum_exec_noalloc(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                                      void* stream) {
    using namespace pe;
    if (!p) return fail(PE_ERR_INVALID, "exec_noalloc: null plan");
    const int64_t need = plan_workspace_bytes(*p);
    if (need > int64_t(PE_NOALLOC_SCRATCH_BYTES))
        return fail(PE_ERR_WORKSPACE, "exec_noalloc: the plan needs " + std::to_string(need) +
                                          " bytes of workspace, above the " +
                                          std::to_string(int64_t(PE_NOALLOC_SCRATCH_BYTES)) +
                                          "-byte scratch limit; use run_einsum_setup / pe_einsum_exec");
    void* ws = nullptr;
    const int st = device_scratch(&ws);
    if (st != PE_OK) return st;
    // Every workspace region the plan uses (operand gathers, the staged
    // result, split-K partials) is written in full before it is read, so no
    // clearing is needed and the previous call's contents are harmless.
    return pe_einsum_exec(p, in0, in1, out, ws, stream);
}

extern "C" int pe_einsum_run(const pe_einsum_plan* p, const void* in0, const void* in1, float* out,
                             void* stream) {
    void* ws = pe_einsum_setup(p, stream);
    if (!ws) return PE_ERR_WORKSPACE;
    int st = pe_einsum_exec(p, in0, in1, out, ws, stream);
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    int st2 = pe_einsum_teardown(ws);
    if (st != PE_OK) return st;
    if (e != hipSuccess) return pe::hip_status(e, "hipStreamSynchronize");
    return st2;
}
