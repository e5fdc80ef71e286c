// RMSNorm forward and backward for gfx950: one HBM read of x, one write of y.
//
// Semantics follow RMSNorm.forward (rmsnorm/original.py:38, 51-52) and the
// compiled rms_norm kernel (rmsnorm/custom.py:25-73):
//   inv = 1 / sqrt(sum(x^2) / dim + eps)          (fp32 accumulation)
//   y   = ty( float(tx(x * inv)) * float(w) )     (two rounding points)
// where tx is x's storage type and ty = promote(tx, tw) is the output type:
// bf16 x with the module's default fp32 weight gives an fp32 y, as torch's
// type promotion does in `output * self.weight` (original.py:52).
// `inv` is a correctly rounded 1/sqrt (not v_rsq_f32) so that the first
// rounding point lands where the host oracle puts it.
//
// Layout: the row is split into 16-byte vectors of x; vector j of a row lives
// in lane (j % 64) of wave-slice (j / 64) % WPR at register slot j / (64*WPR),
// so every load/store instruction of a wave covers a contiguous 1 KiB span of
// x.  A row is owned by WPR waves (WPR = 1 needs no LDS and no barrier).  Rows
// of 4-16 KiB are spread over 2-8 waves with 2 vectors per lane: short-lived
// waves with few loads each kept the HBM queues fuller than long-lived ones
// in sweeps of (VPT, WPR, block size) on MI355X.  Blocks holding two rows
// stage the weight in LDS once per block: re-reading it from L2 for every row
// cost 2-3% of the HBM rate at 2048-4096 channels; with one row per block
// (8192) the staging costs more than it saves.
#include "kf_common.h"

namespace kf {
namespace {

constexpr int kBlock = 256;  // 4 waves (generic kernels)

// N elements of T as one aligned register value: the slice of a row that
// matches one 16-byte vector of x.
template <typename T, int N>
struct alignas(sizeof(T) * N < 16 ? sizeof(T) * N : 16) Pack {
    T v[N];
};

// Non-temporal store of a Pack of 8, 16 or 32 bytes.
template <typename T, int N>
__device__ __forceinline__ void store_nt(Pack<T, N>* dst, const Pack<T, N>& p) {
    constexpr int BYTES = sizeof(T) * N;
    if constexpr (BYTES % 16 == 0) {
        const u32x4* s = reinterpret_cast<const u32x4*>(&p);
        u32x4* d = reinterpret_cast<u32x4*>(dst);
#pragma unroll
        for (int i = 0; i < BYTES / 16; ++i) __builtin_nontemporal_store(s[i], d + i);
    } else {
        static_assert(BYTES == 8, "packs are 8, 16 or 32 bytes");
        __builtin_nontemporal_store(*reinterpret_cast<const u32x2*>(&p), reinterpret_cast<u32x2*>(dst));
    }
}

// x and y rows start every ld_x / ld_y elements (ld >= dim); the vector path
// needs those strides, like the base pointers, aligned to the vector slices.
// y may alias x (in place, same stride and type): every row is read whole
// into registers before any of it is written.
template <typename TX, typename TW, typename TY, int VPT, int WPR, int WAVES, bool HAS_W>
__global__ __launch_bounds__(64 * WAVES) void rmsnorm_vec_kernel(const TX* x, const TW* __restrict__ w,
                                                                 TY* y, int64_t rows, int dim,
                                                                 int64_t ld_x, int64_t ld_y, float eps) {
    constexpr int VEC = 16 / sizeof(TX);
    typedef Pack<TW, VEC> WPack;
    typedef Pack<TY, VEC> YPack;
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
    __shared__ WPack wl[kStageW ? VPT * WPR * 64 : 1];
    const WPack* wr = reinterpret_cast<const WPack*>(w);

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
        const TX* e = reinterpret_cast<const TX*>(&xv[i]);
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

    YPack* yr = reinterpret_cast<YPack*>(y + row * ld_y);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int j = (i * WPR + slice) * 64 + lane;
        if (j < nvec) {
            const TX* e = reinterpret_cast<const TX*>(&xv[i]);
            WPack wv;
            if constexpr (kStageW)
                wv = wl[j];
            else if constexpr (HAS_W)
                wv = wr[j];
            YPack ov;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const TX n = from_f32<TX>(to_f32(e[k]) * inv);
                if constexpr (HAS_W)
                    ov.v[k] = from_f32<TY>(to_f32(n) * to_f32(wv.v[k]));
                else
                    ov.v[k] = from_f32<TY>(to_f32(n));
            }
            store_nt(yr + j, ov);
        }
    }
}

// Any dim / alignment: one block per row, two passes over the row.
template <typename TX, typename TW, typename TY, bool HAS_W>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(const TX* x, const TW* __restrict__ w,
                                                                 TY* y, int64_t rows, int64_t dim,
                                                                 int64_t ld_x, int64_t ld_y, float eps) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const TX* xr = x + row * ld_x;
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
    TY* yr = y + row * ld_y;
    for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
        const TX n = from_f32<TX>(to_f32(xr[c]) * inv);
        if constexpr (HAS_W)
            yr[c] = from_f32<TY>(to_f32(n) * to_f32(w[c]));
        else
            yr[c] = from_f32<TY>(to_f32(n));
    }
}

template <typename TX, typename TW, typename TY, int VPT, int WPR, int WAVES, bool HAS_W>
int launch_vec(const void* x, const void* w, void* y, int64_t rows, int64_t dim, int64_t ld_x,
               int64_t ld_y, float eps, hipStream_t stream) {
    static_assert(WAVES % WPR == 0, "a block holds whole rows");
    constexpr int ROWS_PER_BLOCK = WAVES / WPR;
    const int64_t blocks = (rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK;
    KF_REQUIRE(blocks <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: %lld rows exceed the grid limit",
               (long long)rows);
    hipLaunchKernelGGL((rmsnorm_vec_kernel<TX, TW, TY, VPT, WPR, WAVES, HAS_W>), dim3((unsigned)blocks),
                       dim3(64 * WAVES), 0, stream, static_cast<const TX*>(x),
                       static_cast<const TW*>(w), static_cast<TY*>(y), rows, (int)dim, ld_x, ld_y, eps);
    return check_launch("rmsnorm_vec_kernel launch");
}

bool aligned_to(const void* p, size_t a) { return (uintptr_t)p % a == 0; }

template <typename TX, typename TW, typename TY, bool HAS_W>
int dispatch(const void* x, const void* w, void* y, int64_t rows, int64_t dim, int64_t ld_x,
             int64_t ld_y, float eps, hipStream_t stream) {
    if (rows == 0) return KF_OK;
    constexpr int VEC = 16 / sizeof(TX);
    // Byte alignment of the weight and output slices of one x vector.
    constexpr size_t WA = sizeof(Pack<TW, VEC>) < 16 ? sizeof(Pack<TW, VEC>) : 16;
    constexpr size_t YA = sizeof(Pack<TY, VEC>) < 16 ? sizeof(Pack<TY, VEC>) : 16;
    const bool aligned = aligned_to(x, 16) && aligned_to(y, YA) && (!HAS_W || aligned_to(w, WA)) &&
                         (dim % VEC == 0) && (ld_x % VEC == 0) && (ld_y * sizeof(TY)) % YA == 0;
    const int64_t nvec = dim / VEC;
    if (aligned) {
#define KF_RMS_VEC(VPT, WPR, WAVES) \
    return launch_vec<TX, TW, TY, VPT, WPR, WAVES, HAS_W>(x, w, y, rows, dim, ld_x, ld_y, eps, stream)
        // (vectors per lane, waves per row, waves per block).
        if (nvec <= 64) KF_RMS_VEC(1, 1, 4);
        if (nvec <= 128) KF_RMS_VEC(2, 1, 4);
        if (nvec <= 256) KF_RMS_VEC(2, 2, 4);
        if (nvec <= 512) KF_RMS_VEC(2, 4, 8);
        if (nvec <= 1024) KF_RMS_VEC(2, 8, 8);
        if (nvec <= 2048) KF_RMS_VEC(4, 8, 8);
        if (nvec <= 4096) KF_RMS_VEC(8, 8, 8);
#undef KF_RMS_VEC
    }
    KF_REQUIRE(rows <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: %lld rows exceed the grid limit",
               (long long)rows);
    hipLaunchKernelGGL((rmsnorm_generic_kernel<TX, TW, TY, HAS_W>), dim3((unsigned)rows), dim3(kBlock), 0,
                       stream, static_cast<const TX*>(x), static_cast<const TW*>(w),
                       static_cast<TY*>(y), rows, dim, ld_x, ld_y, eps);
    return check_launch("rmsnorm_generic_kernel launch");
}

// --------------------------------------------------------------------------
// Backward.
// --------------------------------------------------------------------------
// Gradient of y = ty(float(tx(x * inv)) * float(w)) with the rounding points
// taken as identities (as torch's autograd treats the casts of
// original.py:51-52):
//   n   = tx(x * inv)                          (the saved normalised value)
//   g   = float(tx(float(dy) * float(w)))      (gradient at n: torch forms
//                                               `grad * weight` and casts it to
//                                               n's type tx)
//   dx  = inv * g - x * inv^3 * sum(g * x) / dim
//   dw  = tw(sum over rows of float(dy) * float(n))   (fp32 sum of unrounded
//                                               products)
// Each block owns a contiguous run of rows and keeps its dw partial sums in
// fp32 in `partial[block][dim]` (its own row of the workspace, so no two
// blocks touch the same partial); rmsnorm_dw_reduce_kernel then adds the
// block partials in block order (fixed order: deterministic, no atomics).
template <typename TX, typename TW, typename TY>
__global__ __launch_bounds__(kBlock) void rmsnorm_bwd_kernel(const TX* __restrict__ x,
                                                             const TW* __restrict__ w,
                                                             const TY* __restrict__ dy,
                                                             TX* __restrict__ dx,
                                                             float* __restrict__ partial, int64_t rows,
                                                             int64_t dim, int64_t rows_per_block,
                                                             float eps) {
    __shared__ float part[2][4];
    float* pw = partial + (int64_t)blockIdx.x * dim;
    for (int64_t c = threadIdx.x; c < dim; c += kBlock) pw[c] = 0.f;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    for (int64_t row = r0; row < r1; ++row) {
        const TX* xr = x + row * dim;
        const TY* gr = dy + row * dim;
        float ss = 0.f, dot = 0.f;
        for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
            const float f = to_f32(xr[c]);
            const float g = to_f32(from_f32<TX>(to_f32(gr[c]) * to_f32(w[c])));
            ss = fmaf(f, f, ss);
            dot = fmaf(g, f, dot);
        }
        ss = wave_sum(ss);
        dot = wave_sum(dot);
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) {
            part[0][wave] = ss;
            part[1][wave] = dot;
        }
        __syncthreads();
        ss = part[0][0] + part[0][1] + part[0][2] + part[0][3];
        dot = part[1][0] + part[1][1] + part[1][2] + part[1][3];
        __syncthreads();  // part is rewritten by the next row
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
        const float k = inv * inv * inv * dot / (float)dim;
        TX* dr = dx + row * dim;
        for (int64_t c = threadIdx.x; c < dim; c += kBlock) {
            const float f = to_f32(xr[c]);
            const float gy = to_f32(gr[c]);
            const float g = to_f32(from_f32<TX>(gy * to_f32(w[c])));
            dr[c] = from_f32<TX>(inv * g - f * k);
            const float n = to_f32(from_f32<TX>(f * inv));
            pw[c] += gy * n;  // the same thread owns column c for every row
        }
    }
}

template <typename TW>
__global__ __launch_bounds__(kBlock) void rmsnorm_dw_reduce_kernel(const float* __restrict__ partial,
                                                                   TW* __restrict__ dw, int64_t dim,
                                                                   int nblocks) {
    const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (c >= dim) return;
    float acc = 0.f;
    for (int b = 0; b < nblocks; ++b) acc += partial[(int64_t)b * dim + c];
    dw[c] = from_f32<TW>(acc);
}

constexpr int64_t kBwdMaxBlocks = 1024;

int64_t bwd_blocks(int64_t rows) { return rows < kBwdMaxBlocks ? rows : kBwdMaxBlocks; }

template <typename TX, typename TW, typename TY>
int run_bwd(const void* x, const void* w, const void* dy, void* dx, void* dw, float* partial,
            int64_t rows, int64_t dim, float eps, hipStream_t stream) {
    const int64_t nb = bwd_blocks(rows);
    const int64_t per = nb > 0 ? (rows + nb - 1) / nb : 1;
    const int64_t used = (rows + per - 1) / per;  // blocks that own at least one row
    if (used > 0) {
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<TX, TW, TY>), dim3((unsigned)used), dim3(kBlock), 0, stream,
                           static_cast<const TX*>(x), static_cast<const TW*>(w), static_cast<const TY*>(dy),
                           static_cast<TX*>(dx), partial, rows, dim, per, eps);
        if (int rc = check_launch("rmsnorm_bwd_kernel launch")) return rc;
    }
    // With no rows the reduction adds nothing and writes a zero weight gradient.
    hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<TW>), dim3((unsigned)((dim + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, stream, partial, static_cast<TW*>(dw), dim, (int)used);
    return check_launch("rmsnorm_dw_reduce_kernel launch");
}

bool valid_dt(int d) { return d == KF_F32 || d == KF_F16 || d == KF_BF16; }

// torch.promote_types over {fp32, fp16, bf16}: equal types stay, any mix
// gives fp32.
int promote(int a, int b) { return a == b ? a : KF_F32; }

// Calls F<TX, TW, TY>::run(args...) for the (x, weight) dtype pair; TY is
// their promotion.
template <template <typename, typename, typename> class F, typename... A>
int by_types(int xd, int wd, A... args) {
    switch (xd * 3 + wd) {
        case KF_F32 * 3 + KF_F32: return F<float, float, float>::run(args...);
        case KF_F32 * 3 + KF_F16: return F<float, f16, float>::run(args...);
        case KF_F32 * 3 + KF_BF16: return F<float, bf16, float>::run(args...);
        case KF_F16 * 3 + KF_F32: return F<f16, float, float>::run(args...);
        case KF_F16 * 3 + KF_F16: return F<f16, f16, f16>::run(args...);
        case KF_F16 * 3 + KF_BF16: return F<f16, bf16, float>::run(args...);
        case KF_BF16 * 3 + KF_F32: return F<bf16, float, float>::run(args...);
        case KF_BF16 * 3 + KF_F16: return F<bf16, f16, float>::run(args...);
        case KF_BF16 * 3 + KF_BF16: return F<bf16, bf16, bf16>::run(args...);
    }
    set_error("rmsnorm: unknown dtype pair (%d, %d)", xd, wd);
    return KF_E_INVALID;
}

template <typename TX, typename TW, typename TY> struct FwdOp {
    static int run(const void* x, const void* w, void* y, int64_t rows, int64_t dim, int64_t ld_x,
                   int64_t ld_y, float eps, hipStream_t s) {
        return dispatch<TX, TW, TY, true>(x, w, y, rows, dim, ld_x, ld_y, eps, s);
    }
};

template <typename TX, typename TW, typename TY> struct BwdOp {
    static int run(const void* x, const void* w, const void* dy, void* dx, void* dw, float* partial,
                   int64_t rows, int64_t dim, float eps, hipStream_t s) {
        return run_bwd<TX, TW, TY>(x, w, dy, dx, dw, partial, rows, dim, eps, s);
    }
};

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
    KF_REQUIRE(valid_dt(dtype), KF_E_INVALID, "rmsnorm: unknown dtype %d", dtype);
    return by_types<FwdOp>(dtype, dtype, x, weight, y, rows, dim, ld_x, ld_y, eps,
                           static_cast<hipStream_t>(stream));
}

extern "C" int kf_rmsnorm_fwd(const void* x, const void* weight, void* y, int64_t rows,
                              int64_t dim, float eps, int dtype, kf_stream_t stream) {
    return kf_rmsnorm_fwd_strided(x, weight, y, rows, dim, dim, dim, eps, dtype, stream);
}

extern "C" int kf_rmsnorm_fwd_mixed(const void* x, const void* weight, void* y, int64_t rows,
                                    int64_t dim, float eps, int x_dtype, int w_dtype, int y_dtype,
                                    kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(rows >= 0 && dim >= 1, KF_E_INVALID, "rmsnorm: bad shape rows=%lld dim=%lld",
               (long long)rows, (long long)dim);
    KF_REQUIRE(valid_dt(x_dtype) && valid_dt(w_dtype), KF_E_INVALID, "rmsnorm: unknown dtype (%d, %d)",
               x_dtype, w_dtype);
    KF_REQUIRE(y_dtype == promote(x_dtype, w_dtype), KF_E_INVALID,
               "rmsnorm: output dtype %d is not the promotion of x dtype %d and weight dtype %d", y_dtype,
               x_dtype, w_dtype);
    KF_REQUIRE(rows == 0 || (x && y && weight), KF_E_INVALID, "rmsnorm: null pointer");
    KF_REQUIRE(dim <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: dim %lld too large", (long long)dim);
    return by_types<FwdOp>(x_dtype, w_dtype, x, weight, y, rows, dim, dim, dim, eps,
                           static_cast<hipStream_t>(stream));
}

extern "C" int64_t kf_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t dim) {
    if (rows < 0 || dim < 1) return -1;
    return (int64_t)sizeof(float) * kf::bwd_blocks(rows) * dim;
}

extern "C" int kf_rmsnorm_bwd(const void* x, const void* weight, const void* dy, void* dx, void* dweight,
                              void* workspace, int64_t workspace_bytes, int64_t rows, int64_t dim,
                              float eps, int x_dtype, int w_dtype, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(rows >= 0 && dim >= 1, KF_E_INVALID, "rmsnorm: bad shape rows=%lld dim=%lld",
               (long long)rows, (long long)dim);
    KF_REQUIRE(valid_dt(x_dtype) && valid_dt(w_dtype), KF_E_INVALID, "rmsnorm: unknown dtype (%d, %d)",
               x_dtype, w_dtype);
    KF_REQUIRE(dim <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: dim %lld too large", (long long)dim);
    KF_REQUIRE(x || rows == 0, KF_E_INVALID, "rmsnorm: null pointer");
    KF_REQUIRE(weight && dweight, KF_E_INVALID, "rmsnorm: null weight or weight gradient");
    const int64_t need = kf_rmsnorm_bwd_workspace_bytes(rows, dim);
    KF_REQUIRE(rows == 0 || (workspace && workspace_bytes >= need), KF_E_WORKSPACE,
               "rmsnorm: workspace of %lld bytes needed, %lld given", (long long)need,
               (long long)workspace_bytes);
    KF_REQUIRE(rows == 0 || (dy && dx), KF_E_INVALID, "rmsnorm: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    return by_types<BwdOp>(x_dtype, w_dtype, x, weight, dy, dx, dweight, static_cast<float*>(workspace),
                           rows, dim, eps, s);
}

extern "C" int kf_rmsnorm_noweight_f32(const float* a, float* b, int64_t rows, int64_t n,
                                       float eps, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(rows >= 0 && n >= 1, KF_E_INVALID, "rmsnorm: bad shape rows=%lld n=%lld",
               (long long)rows, (long long)n);
    KF_REQUIRE(rows == 0 || (a && b), KF_E_INVALID, "rmsnorm: null pointer");
    KF_REQUIRE(n <= 0x7fffffff, KF_E_UNSUPPORTED, "rmsnorm: n %lld too large", (long long)n);
    return dispatch<float, float, float, false>(a, nullptr, b, rows, n, n, n, eps,
                                                static_cast<hipStream_t>(stream));
}
