// Shared device and host helpers for the kernelforge_amd HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kernelforge_amd.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local message, see kf_last_error()).
// ---------------------------------------------------------------------------
namespace kf {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Record a failed HIP call and return KF_E_HIP.
int hip_failure(hipError_t err, const char* what);

// Check for a launch error right after a kernel launch.
inline int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_failure(err, what);
    return KF_OK;
}

// Number of compute units on the current device (cached per device).
int device_cu_count();

}  // namespace kf

#define KF_REQUIRE(cond, code, ...)        \
    do {                                   \
        if (!(cond)) {                     \
            ::kf::set_error(__VA_ARGS__);  \
            return (code);                 \
        }                                  \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
namespace kf {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Storage-type conversions.  bf16/f16 rounding is round-to-nearest-even
// (v_cvt_pk_bf16_f32 / v_cvt_f16_f32 on gfx950).
template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

// 16-byte vector of storage elements.
template <typename T> struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    T v[N];
};

__device__ __forceinline__ float wave_sum(float x) {
    // Butterfly over the 64 lanes of a wavefront.
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
    return x;
}

}  // namespace kf
