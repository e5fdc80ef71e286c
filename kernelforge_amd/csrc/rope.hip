// Rotary position embedding of LiteLA (SANA), in place on the packed qkv.
//
// Semantics: apply_rotary_emb(x, (cos, sin), use_real=True,
// use_real_unbind_dim=-2) as LiteLA.forward applies it to q and k
// (SANA_LinearAttention/original.py:14-58, 136-138): within each head the
// channels pair up as (2i, 2i+1) = (real, imaginary), and
//   out[2i]   = x[2i]   * cos[n][2i]   + (-x[2i+1]) * sin[n][2i]
//   out[2i+1] = x[2i+1] * cos[n][2i+1] + ( x[2i])   * sin[n][2i+1]
// with the products and the sum each rounded in fp32 (no fused multiply-add)
// and the result rounded to the storage type, as the reference's
// x.float() * cos + x_rotated.float() * sin, .to(x.dtype) does.
//
// Layout: qkv[b][n][part][h*D + d] (part 0 = q, 1 = k are rotated, 2 = v is
// not); cos, sin fp32 [N][D].  One thread per 16-byte vector of a q or k row;
// a vector never straddles a head (D % 8 == 0) and holds whole pairs.
#include "kf_common.h"

namespace kf {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void rope_packed_kernel(T* qkv, const float* __restrict__ cs,
                                                          const float* __restrict__ sn, int64_t B,
                                                          int64_t N, int64_t C, int D) {
    // hipcc contracts a*b + c*d into a fused multiply-add by default; the
    // reference rounds both products and the sum.
#pragma clang fp contract(off)
    constexpr int VEC = 16 / sizeof(T);
    const int64_t vec_per_part = C / VEC;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= B * N * 2 * vec_per_part) return;
    const int64_t row = i / (2 * vec_per_part);  // b * N + n
    const int64_t rem = i - row * 2 * vec_per_part;
    const int64_t part = rem / vec_per_part;     // 0 = q, 1 = k
    const int64_t c0 = (rem - part * vec_per_part) * VEC;
    const int64_t n = row % N;
    const int d0 = (int)(c0 % D);

    u32x4* p = reinterpret_cast<u32x4*>(qkv + (row * 3 + part) * C + c0);
    const u32x4 raw = *p;
    const T* x = reinterpret_cast<const T*>(&raw);
    const float* c = cs + n * D + d0;
    const float* s = sn + n * D + d0;
    u32x4 res;
    T* o = reinterpret_cast<T*>(&res);
#pragma unroll
    for (int j = 0; j < VEC; j += 2) {
        const float re = to_f32(x[j]), im = to_f32(x[j + 1]);
        const float a0 = re * c[j], b0 = -im * s[j];
        const float a1 = im * c[j + 1], b1 = re * s[j + 1];
        o[j] = from_f32<T>(a0 + b0);
        o[j + 1] = from_f32<T>(a1 + b1);
    }
    *p = res;
}

template <typename T>
int launch_rope(void* qkv, const float* cs, const float* sn, int64_t B, int64_t N, int64_t C, int D,
                hipStream_t stream) {
    const int64_t work = B * N * 2 * (C / (16 / (int64_t)sizeof(T)));
    const int64_t blocks = (work + 255) / 256;
    if (blocks > 0x7fffffff) {
        set_error("rope: grid too large");
        return KF_E_UNSUPPORTED;
    }
    hipLaunchKernelGGL((rope_packed_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<T*>(qkv), cs, sn, B, N, C, D);
    return check_launch("rope_packed_kernel launch");
}

}  // namespace
}  // namespace kf

extern "C" int kf_rope_packed(void* qkv, const float* cos, const float* sin, int64_t batch,
                              int64_t seq_len, int64_t heads, int64_t dim, int dtype,
                              kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(batch >= 0 && seq_len >= 0 && heads > 0 && dim > 0, KF_E_INVALID, "rope: bad shape");
    KF_REQUIRE(dim % 8 == 0, KF_E_INVALID, "rope: head dim must be a multiple of 8, got %lld", (long long)dim);
    KF_REQUIRE(heads <= (1 << 20) && dim <= 4096 && seq_len <= ((int64_t)1 << 40), KF_E_INVALID,
               "rope: shape out of range");
    KF_REQUIRE(dtype == KF_F32 || dtype == KF_F16 || dtype == KF_BF16, KF_E_INVALID, "rope: bad dtype");
    if (batch == 0 || seq_len == 0) return KF_OK;
    KF_REQUIRE(qkv && cos && sin, KF_E_INVALID, "rope: null pointer");
    KF_REQUIRE(((uintptr_t)qkv & 15) == 0, KF_E_INVALID, "rope: qkv must be 16-byte aligned");
    const int64_t C = heads * dim;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case KF_F32: return launch_rope<float>(qkv, cos, sin, batch, seq_len, C, (int)dim, s);
        case KF_F16: return launch_rope<f16>(qkv, cos, sin, batch, seq_len, C, (int)dim, s);
        default: return launch_rope<bf16>(qkv, cos, sin, batch, seq_len, C, (int)dim, s);
    }
}
