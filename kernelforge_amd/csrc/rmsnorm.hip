// RMSNorm forward for gfx950: one HBM read of x, one write of y.
//
// Semantics follow RMSNorm.forward (rmsnorm/original.py:38, 51-52) and the
// compiled rms_norm kernel (rmsnorm/custom.py:25-73):
//   inv = 1 / sqrt(sum(x^2) / dim + eps)          (fp32 accumulation)
//   y   = dt( float(dt(x * inv)) * float(w) )     (two rounding points)
// `inv` is a correctly rounded 1/sqrt (not v_rsq_f32) so that the first
// rounding point lands where the host oracle puts it.
//
// Layout: the row is split into 16-byte vectors; vector j of a row lives in
// lane (j % 64) of wave-slice (j / 64) % WPR at register slot j / (64*WPR),
// so every load/store instruction of a wave covers a contiguous 1 KiB span.
// A row is owned by WPR waves (WPR = 1 needs no LDS and no barrier).  Rows of
// 4-16 KiB are spread over 2-8 waves with 2 vectors per lane: short-lived
// waves with few loads each kept the HBM queues fuller than long-lived ones
// in sweeps of (VPT, WPR, block size) on MI355X.  Blocks holding two rows
// stage the weight in LDS once per block: re-reading it from L2 for every row
// cost 2-3% of the HBM rate at 2048-4096 channels; with one row per block
// (8192) the staging costs more than it saves.
#include "kf_common.h"

namespace kf {
namespace {

constexpr int kBlock = 256;  // 4 waves (generic kernel)

// x and y rows start every ld_x / ld_y elements (ld >= dim); the 16-byte
// vector path needs those strides, like the base pointers, 16-byte aligned.
// y may alias x (in place, same stride): every row is read whole into
// registers before any of it is written.
template <typename T, int VPT, int WPR, int WAVES, bool HAS_W>
__global__ __launch_bounds__(64 * WAVES) void rmsnorm_vec_kernel(const T* x, const T* __restrict__ w,
                                                                 T* y, int64_t rows, int dim,
                                                                 int64_t ld_x, int64_t ld_y, float eps) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int ROWS_PER_BLOCK = WAVES / WPR;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row_in_block = wave / WPR;
    const int slice = wave % WPR;
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + row_in_block;
    const bool row_ok = row < rows;
    const int nvec = dim / VEC;

    // Blocks of two or more rows read the weight once per block into LDS
    // instead of once per row (an 8 KiB L2 read per row at dim 4096).
    constexpr bool kStageW = HAS_W && WPR > 1 && ROWS_PER_BLOCK > 1;
    __shared__ u32x4 wl[kStageW ? VPT * WPR * 64 : 1];
    const u32x4* wr = reinterpret_cast<const u32x4*>(w);

    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * ld_x);
    u32x4 xv[VPT];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int j = (i * WPR + slice) * 64 + lane;
        if (row_ok && j < nvec) {
            xv[i] = __builtin_nontemporal_load(xr + j);
        } else {
            xv[i] = u32x4{0u, 0u, 0u, 0u};
        }
    }
    if constexpr (kStageW) {
        for (int j = threadIdx.x; j < nvec; j += 64 * WAVES) wl[j] = wr[j];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const T* e = reinterpret_cast<const T*>(&xv[i]);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const float f = to_f32(e[k]);
            ss = fmaf(f, f, ss);
        }
    }
    ss = wave_sum(ss);
    if constexpr (WPR > 1) {
        __shared__ float part[WAVES];
        if (lane == 0) part[wave] = ss;
        __syncthreads();  // also publishes the staged weight
        float t = 0.f;
#pragma unroll
        for (int s = 0; s < WPR; ++s) t += part[row_in_block * WPR + s];
        ss = t;
    }
    if (!row_ok) return;
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);

    u32x4* yr = reinterpret_cast<u32x4*>(y + row * ld_y);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int j = (i * WPR + slice) * 64 + lane;
        if (j < nvec) {
            const T* e = reinterpret_cast<const T*>(&xv[i]);
            u32x4 wv;
            if constexpr (kStageW)
                wv = wl[j];
            else if constexpr (HAS_W)
                wv = wr[j];
            const T* we = reinterpret_cast<const T*>(&wv);
            u32x4 ov;
            T* o = reinterpret_cast<T*>(&ov);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const T n = from_f32<T>(to_f32(e[k]) * inv);
                if constexpr (HAS_W)
                    o[k] = from_f32<T>(to_f32(n) * to_f32(we[k]));
                else
                    o[k] = n;
            }
            __builtin_nontemporal_store(ov, yr + j);
        }
    }
}

// Any dim / alignment: one block per row, two passes over the row.
template <typename T, bool HAS_W>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(const T* x, const T* __restrict__ w,
                                                                 T* y, int64_t rows, int64_t dim,
                                                                 int64_t ld_x, int64_t ld_y, float eps) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const T* xr = x + row * ld_x;
    float ss = 0.f;
    for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
        const float f = to_f32(xr[c]);
        ss = fmaf(f, f, ss);
    }
    ss = wave_sum(ss);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = part[0] + part[1] + part[2] + part[3];
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    T* yr = y + row * ld_y;
    for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
        const T n = from_f32<T>(to_f32(xr[c]) * inv);
        if constexpr (HAS_W)
            yr[c] = from_f32<T>(to_f32(n) * to_f32(w[c]));
        else
            yr[c] = n;
    }
}

template <typename T, int VPT, int WPR, int WAVES, bool HAS_W>
int launch_vec(const void* x, const void* w, void* y, int64_t rows, int64_t dim, int64_t ld_x,
               int64_t ld_y, float eps, hipStream_t stream) {
    static_assert(WAVES % WPR == 0, "a block holds whole rows");
    constexpr int ROWS_PER_BLOCK = WAVES / WPR;
    const int64_t blocks = (rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK;
    KF_REQUIRE(blocks <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: %lld rows exceed the grid limit",
               (long long)rows);
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, VPT, WPR, WAVES, HAS_W>), dim3((unsigned)blocks),
                       dim3(64 * WAVES), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<T*>(y), rows, (int)dim, ld_x, ld_y, eps);
    return check_launch("rmsnorm_vec_kernel launch");
}

template <typename T, bool HAS_W>
int dispatch(const void* x, const void* w, void* y, int64_t rows, int64_t dim, int64_t ld_x,
             int64_t ld_y, float eps, hipStream_t stream) {
    if (rows == 0) return KF_OK;
    constexpr int VEC = 16 / sizeof(T);
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) &&
                         (!HAS_W || (uintptr_t)w % 16 == 0) && (dim % VEC == 0) &&
                         (ld_x % VEC == 0) && (ld_y % VEC == 0);
    const int64_t nvec = dim / VEC;
    if (aligned) {
        // (vectors per lane, waves per row, waves per block).
        if (nvec <= 64) return launch_vec<T, 1, 1, 4, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 128) return launch_vec<T, 2, 1, 4, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 256) return launch_vec<T, 2, 2, 4, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 512) return launch_vec<T, 2, 4, 8, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 1024) return launch_vec<T, 2, 8, 8, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 2048) return launch_vec<T, 4, 8, 8, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
        if (nvec <= 4096) return launch_vec<T, 8, 8, 8, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream);
    }
    KF_REQUIRE(rows <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: %lld rows exceed the grid limit",
               (long long)rows);
    hipLaunchKernelGGL((rmsnorm_generic_kernel<T, HAS_W>), dim3((unsigned)rows), dim3(kBlock), 0,
                       stream, static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<T*>(y), rows, dim, ld_x, ld_y, eps);
    return check_launch("rmsnorm_generic_kernel launch");
}

}  // namespace
}  // namespace kf

extern "C" int kf_rmsnorm_fwd_strided(const void* x, const void* weight, void* y, int64_t rows,
                                      int64_t dim, int64_t ld_x, int64_t ld_y, float eps, int dtype,
                                      kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(rows >= 0 && dim >= 1, KF_E_INVALID, "rmsnorm: bad shape rows=%lld dim=%lld",
               (long long)rows, (long long)dim);
    KF_REQUIRE(ld_x >= dim && ld_y >= dim, KF_E_INVALID,
               "rmsnorm: row strides ld_x=%lld ld_y=%lld must be >= dim=%lld", (long long)ld_x,
               (long long)ld_y, (long long)dim);
    KF_REQUIRE(rows == 0 || (x && y && weight), KF_E_INVALID, "rmsnorm: null pointer");
    KF_REQUIRE(dim <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: dim %lld too large", (long long)dim);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case KF_F32: return dispatch<float, true>(x, weight, y, rows, dim, ld_x, ld_y, eps, s);
        case KF_F16: return dispatch<f16, true>(x, weight, y, rows, dim, ld_x, ld_y, eps, s);
        case KF_BF16: return dispatch<bf16, true>(x, weight, y, rows, dim, ld_x, ld_y, eps, s);
        default: set_error("rmsnorm: unknown dtype %d", dtype); return KF_E_INVALID;
    }
}

extern "C" int kf_rmsnorm_fwd(const void* x, const void* weight, void* y, int64_t rows,
                              int64_t dim, float eps, int dtype, kf_stream_t stream) {
    return kf_rmsnorm_fwd_strided(x, weight, y, rows, dim, dim, dim, eps, dtype, stream);
}

extern "C" int kf_rmsnorm_noweight_f32(const float* a, float* b, int64_t rows, int64_t n,
                                       float eps, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(rows >= 0 && n >= 1, KF_E_INVALID, "rmsnorm: bad shape rows=%lld n=%lld",
               (long long)rows, (long long)n);
    KF_REQUIRE(rows == 0 || (a && b), KF_E_INVALID, "rmsnorm: null pointer");
    KF_REQUIRE(n <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: n %lld too large", (long long)n);
    return dispatch<float, false>(a, nullptr, b, rows, n, n, n, eps, static_cast<hipStream_t>(stream));
}
