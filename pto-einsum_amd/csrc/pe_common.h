// Shared helpers for the gfx950 einsum kernels: error reporting, integer
// division by run-time constants, vector types and launch utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "pto_einsum_hip.h"

namespace pe {

// ---------------------------------------------------------------- errors --

// Records a message for pe_last_error() and returns `code`.
int fail(int code, const std::string& msg);
int hip_status(hipError_t e, const char* what);

#define PE_CHECK_HIP(expr)                                       \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return ::pe::hip_status(_e, #expr); \
    } while (0)

// ------------------------------------------------- division by constants --

// Unsigned 32-bit division by a run-time constant d >= 1 via one multiply-high
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant): with l = ceil(log2 d) and
// m = floor(2^32 * (2^l - d) / d) + 1, q = (mulhi(n, m) + n) >> l for all
// n < 2^32.  The 33-bit sum is formed as t + ((n - t) >> 1) to stay in 32 bits.
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t s;  // l
    FastDiv() : d(1), m(0), s(0) {}
    explicit FastDiv(uint32_t div) { init(div); }
    void init(uint32_t div) {
        d = div ? div : 1;
        uint32_t l = 0;
        while (l < 32 && (uint64_t(1) << l) < d) ++l;
        s = l;
        m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        uint32_t t = __umulhi(n, m);
#else
        uint32_t t = uint32_t((uint64_t(n) * m) >> 32);
#endif
        if (s == 0) return n;  // d == 1
        return (t + ((n - t) >> 1)) >> (s - 1);
    }
    __host__ __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
        q = div(n);
        r = n - q * d;
    }
};

// ------------------------------------------------------------ vectors --

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Element type tags: storage type and exact conversion to float.
struct F32 {
    using T = float;
    static constexpr int kBytes = 4;
    __device__ __forceinline__ static float to_f32(float x) { return x; }
};
struct F16 {
    using T = _Float16;
    static constexpr int kBytes = 2;
    __device__ __forceinline__ static float to_f32(_Float16 x) { return (float)x; }
};

// Outputs at least this large are written with non-temporal stores, smaller
// ones with ordinary stores.  Measured with a fresh output buffer per call
// (the outputs rotating over 1 GiB, as a caller's successive results do):
// 32 MB against the earlier 128 MB took config 5.1's 67 MB GEMM output from
// 19.5 to 17.7 us and the GDN 64x16 / 16x48 products (67 / 50 MB) 4 % lower;
// 8 MB changed nothing further.  Split-K partials, which the reduction
// kernel reads back at once, keep ordinary stores up to
// PE_NT_PARTIAL_MIN_BYTES.
#ifndef PE_NT_MIN_BYTES
#define PE_NT_MIN_BYTES (32ll << 20)
#endif
#ifndef PE_NT_PARTIAL_MIN_BYTES
#define PE_NT_PARTIAL_MIN_BYTES (128ll << 20)
#endif
// Outputs of at least this many bytes (beyond the 256 MB Infinity Cache)
// take non-temporal stores at system scope (nt sc0 sc1).  One MI355X,
// alternating runs on one box (two boxes): config 3 (2.15 GB) 408-425 ->
// 394-408 us, its output transpose (2.15 GB) 686-692 -> 659-663 us, 8192^3
// float16 NT 899-906 -> 881-890 us (NN unchanged), 4a (268 MB) 133-134 ->
// 132-133 us; config 5.1's 67 MB output ran slower that way (14.3-15.4 ->
// 15.8-15.9 us).  The float32 GEMM epilogues keep the plain non-temporal
// flavour (pe_gemm_dl.h).
#ifndef PE_NT_SYS_MIN_BYTES
#define PE_NT_SYS_MIN_BYTES (256ll << 20)
#endif

// Store flavour of an output of `bytes`: 0 ordinary, 1 non-temporal (from
// nt_min bytes), 2 non-temporal at system scope.
inline int nt_mode(int64_t bytes, int64_t nt_min = PE_NT_MIN_BYTES) {
    return bytes >= PE_NT_SYS_MIN_BYTES ? 2 : bytes >= nt_min ? 1 : 0;
}

// Non-temporal vector stores (global_store_* ... nt), written as inline
// assembly: a __builtin_nontemporal_store on one side of a runtime branch
// whose other side stores to the same address is merged with it into an
// ordinary store (the hint is dropped), which measured up to 19 % slower on
// store-bound kernels.
__device__ __forceinline__ void store_nt(float* p, float v) {
    asm volatile("global_store_dword %0, %1, off nt" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt(f32x4* p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off nt" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt(u32x4* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off nt" : : "v"(p), "v"(v) : "memory");
}

// The same at system scope (store flavour 2).
__device__ __forceinline__ void store_nt_sys(float* p, float v) {
    asm volatile("global_store_dword %0, %1, off nt sc0 sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt_sys(f32x4* p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off nt sc0 sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt_sys(u32x4* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off nt sc0 sc1" : : "v"(p), "v"(v) : "memory");
}

// A store of flavour `mode` (nt_mode).
template <typename P, typename V>
__device__ __forceinline__ void store_f(P* p, V v, int mode) {
    if (mode == 2) store_nt_sys(p, v);
    else if (mode == 1) store_nt(p, v);
    else *p = v;
}

// --------------------------------------------------------------- device --

// Number of compute units of the current device (memoised per device).
int cu_count();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

}  // namespace pe
