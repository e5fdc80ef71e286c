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

// Short vectors of a 16-bit storage type, as the MFMA builtins take them.
template <typename T> struct V {
    typedef T x8 __attribute__((ext_vector_type(8)));
    typedef T x4 __attribute__((ext_vector_type(4)));
};
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// MFMA wrappers (gfx950).  Operand layouts, with lane l of the wavefront:
//   16x16x32: A[m][k]: m = l%16, k = 8*(l/16)+j   B[k][n]: n = l%16, k = 8*(l/16)+j
//             D[m][n]: n = l%16, m = 4*(l/16)+i                    (i = 0..3)
//   32x32x16: A[m][k]: m = l%32, k = 8*(l/32)+j   B[k][n]: n = l%32, k = 8*(l/32)+j
//             D[m][n]: n = l%32, m = 8*(i/4) + 4*(l/32) + i%4      (i = 0..15)
__device__ __forceinline__ f32x4 mfma16x16x32(V<bf16>::x8 a, V<bf16>::x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(V<f16>::x8 a, V<f16>::x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(V<bf16>::x8 a, V<bf16>::x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(V<f16>::x8 a, V<f16>::x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// the 4 lanes 4q..4q+3 each address 4 consecutive 16-bit elements, together
// a 16-element row q (q = 0..3); lane j of the group then receives element j
// of rows 0..3.  Used to read a [row][col] tile column-wise for MFMA operands
// whose K index runs along the rows.
__device__ __forceinline__ V<bf16>::x4 lds_read_tr(const bf16* p) {
    typedef __attribute__((address_space(3))) V<bf16>::x4 lds_t;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_t*)(p));
}
__device__ __forceinline__ V<f16>::x4 lds_read_tr(const f16* p) {
    typedef __fp16 fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
    typedef __attribute__((address_space(3))) fp16x4 lds_t;
    return __builtin_bit_cast(V<f16>::x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_t*)(p)));
}

// ReLU on 8 packed 16-bit floats (bf16 or f16): clear every element whose
// sign bit is set (so -0 -> +0).
__device__ __forceinline__ u32x4 relu_packed16(u32x4 x) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned s = (x[i] >> 15) & 0x00010001u;
        r[i] = x[i] & ~(s * 0xffffu);
    }
    return r;
}

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
