// SANA ReLU linear attention for gfx950.
//
// Semantics (LiteLA.attn_matmul, SANA_LinearAttention/original.py:99-117, with
// fp32_attention): per (batch b, head h)
//   S[r][c] = sum_t v[t][r] relu(k[t][c])        (r, c < D: the value/key state)
//   z[c]    = sum_t relu(k[t][c])                 (the padded ones row, PAD_VAL = 1)
//   out[t][r] = sum_c S[r][c] relu(q[t][c]) / (sum_c z[c] relu(q[t][c]) + eps)
// on the packed layout qkv[b][t][part][h*D + r], part 0/1/2 = q/k/v
// (LiteLA.forward, :124-134), out[b][t][h*D + r].
//
// Pipeline (D = 32, bf16/f16 input):
//   1. linattn_state_kernel   grid (splits, ceil(H/2), B): each workgroup streams
//      one sequence split of two adjacent heads (128 contiguous bytes of K and of
//      V per token) through LDS and accumulates S with v_mfma_f32_32x32x16; the
//      token-major operands are read with ds_read_b64_tr_b16.  z accumulates on
//      the VALU from the same registers.  Partials [B][H][splits][D+1][D] fp32.
//   2. linattn_reduce_kernel  grid (H, B): sums the partials in split order
//      (fixed order: deterministic, no atomics).
//   3. linattn_out_kernel     grid (ceil(N/128), ceil(H/4), B): one wavefront per
//      head keeps S and z in registers as hi+lo 16-bit pairs (so the products
//      carry ~16 mantissa bits of the fp32 state) and streams relu(q) straight
//      from HBM as the B operand of v_mfma_f32_16x16x32; z is a third A operand
//      whose rows all equal z, so the denominator lands in the same lanes as the
//      numerator.  No LDS, no barriers.
// Other head dims (128 % D == 0) and fp32 input take a VALU path with the same
// three stages and the same fixed-order split reduction.
#include "kf_common.h"

namespace kf {
namespace {

constexpr int kD = 32;              // head dim of the MFMA path
constexpr int kState = (kD + 1) * kD;
constexpr int kTT = 64;             // tokens per state tile
constexpr int kRS = 72;             // LDS row stride (elements) of a 64-channel row
constexpr int kOutTokens = 128;     // tokens per output workgroup

// --------------------------------------------------------------------------
// 1. Split-state producer (MFMA).
// --------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void linattn_state_kernel(const T* __restrict__ qkv,
                                                            float* __restrict__ partial, int N,
                                                            int H, int split_len, int splits) {
    const int s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t C = (int64_t)H * kD;
    const int h0 = 2 * g;
    const int nh = min(2, H - h0);
    const int t_begin = s * split_len;
    const int t_end = min(N, t_begin + split_len);

    __shared__ __attribute__((aligned(16))) T tile[2][2][kTT * kRS];  // [buf][K,V][tok*kRS+ch]
    __shared__ float comb[2][64][17];

    // Global -> register staging: 4 x 16 B per thread per tile.  Chunk c:
    // token c/16, part (c/8)%2 (0 = K, 1 = V), 16-byte segment c%8 of the
    // 128-byte two-head span.
    u32x4 reg[4];
    auto gload = [&](int t0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * 256 + tid;
            const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
            const int t = t0 + tok;
            if (t < t_end && seg < nh * 4) {
                const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (1 + part) * C +
                               (int64_t)h0 * kD + seg * 8;
                u32x4 v = *reinterpret_cast<const u32x4*>(src);
                reg[i] = part == 0 ? relu_packed16(v) : v;
            } else {
                reg[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * 256 + tid;
            const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
            *reinterpret_cast<u32x4*>(&tile[buf][part][tok * kRS + seg * 8]) = reg[i];
        }
    };

    // Wave (hw, th): head slot hw, token half th of each 64-token tile.
    const int hw = wave & 1, th = wave >> 1;
    const int G = lane >> 4, j16 = lane & 15;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    float zsum = 0.f;

    const int ntile = t_end > t_begin ? (t_end - t_begin + kTT - 1) / kTT : 0;
    if (ntile > 0) {
        gload(t_begin);
        lstore(0);
    }
    __syncthreads();
    for (int it = 0; it < ntile; ++it) {
        const int buf = it & 1;
        if (it + 1 < ntile) gload(t_begin + (it + 1) * kTT);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int row = 32 * th + 16 * ks + 8 * (G >> 1) + (j16 >> 2);
            const int col = hw * 32 + 16 * (G & 1) + 4 * (j16 & 3);
            const T* vb = &tile[buf][1][row * kRS + col];
            const T* kb = &tile[buf][0][row * kRS + col];
            typename V<T>::x4 a0 = lds_read_tr(vb), a1 = lds_read_tr(vb + 4 * kRS);
            typename V<T>::x4 b0 = lds_read_tr(kb), b1 = lds_read_tr(kb + 4 * kRS);
            typename V<T>::x8 a, bk;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = a0[j];
                a[j + 4] = a1[j];
                bk[j] = b0[j];
                bk[j + 4] = b1[j];
            }
            acc = mfma32x32x16(a, bk, acc);
#pragma unroll
            for (int j = 0; j < 8; ++j) zsum += (float)bk[j];
        }
        if (it + 1 < ntile) lstore(buf ^ 1);
        __syncthreads();
    }

    // Combine the two token halves of each head, then write the partial.
    if (th == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) comb[hw][lane][i] = acc[i];
        comb[hw][lane][16] = zsum;
    }
    __syncthreads();
    if (th == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] += comb[hw][lane][i];
        zsum += comb[hw][lane][16];
        zsum += __shfl_xor(zsum, 32, 64);  // lanes l and l+32 hold the same channel
        if (hw < nh) {
            float* P = partial + ((int64_t)(b * H + h0 + hw) * splits + s) * kState;
            const int c = lane & 31;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                P[r * kD + c] = acc[i];
            }
            if (lane < 32) P[kD * kD + c] = zsum;
        }
    }
}

// --------------------------------------------------------------------------
// 2. Fixed-order reduction of the split partials.
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void linattn_reduce_kernel(const float* __restrict__ partial,
                                                             float* __restrict__ state, int H,
                                                             int splits, int state_size) {
    const int h = blockIdx.x, b = blockIdx.y;
    const float* P = partial + (int64_t)(b * H + h) * splits * state_size;
    float* S = state + (int64_t)(b * H + h) * state_size;
    for (int e = threadIdx.x; e < state_size; e += 256) {
        float acc = 0.f;
        for (int s = 0; s < splits; ++s) acc += P[(int64_t)s * state_size + e];
        S[e] = acc;
    }
}

// --------------------------------------------------------------------------
// 3. Output contraction (MFMA, state in registers).
// --------------------------------------------------------------------------
template <typename TO> struct Store4;
template <> struct Store4<float> {
    __device__ static void run(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <typename TO> struct Store4 {
    __device__ static void run(TO* p, f32x4 v) {
        typename V<TO>::x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (TO)v[i];
        *reinterpret_cast<typename V<TO>::x4*>(p) = o;
    }
};

template <typename T, typename TO>
__global__ __launch_bounds__(256) void linattn_out_kernel(const T* __restrict__ qkv,
                                                          const float* __restrict__ state,
                                                          TO* __restrict__ out, int N, int H,
                                                          float eps) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.z;
    const int h = blockIdx.y * 4 + wave;
    if (h >= H) return;
    const int64_t C = (int64_t)H * kD;
    const float* S = state + (int64_t)(b * H + h) * kState;
    const int m16 = lane & 15, kg = lane >> 4;

    // A operands: rows r = 16*mb + m16, k = c = 8*kg + j; the third operand
    // repeats z on every row.
    float sv[2][8], zv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sv[0][j] = S[(m16)*kD + 8 * kg + j];
        sv[1][j] = S[(16 + m16) * kD + 8 * kg + j];
        zv[j] = S[kD * kD + 8 * kg + j];
    }
    // fp16 has a narrow exponent range: rescale the whole state by a power of
    // two (out = num/den is invariant to a common factor; only eps sees it).
    float scale = 1.f;
    if constexpr (sizeof(T) == 2 && !__is_same(T, bf16)) {
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            mx = fmaxf(mx, fmaxf(fabsf(zv[j]), fmaxf(fabsf(sv[0][j]), fabsf(sv[1][j]))));
        mx = wave_max(mx);
        if (mx > 0.f) {
            int e;
            frexpf(mx, &e);
            scale = ldexpf(1.f, -e);
        }
    }
    typename V<T>::x8 shi[2], slo[2], zhi, zlo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const float x = sv[mb][j] * scale;
            const T hi = (T)x;
            shi[mb][j] = hi;
            slo[mb][j] = (T)(x - (float)hi);
        }
        const float x = zv[j] * scale;
        const T hi = (T)x;
        zhi[j] = hi;
        zlo[j] = (T)(x - (float)hi);
    }

    const int t_block = blockIdx.x * kOutTokens;
    const int t_stop = min(N, t_block + kOutTokens);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = t_block; t0 < t_stop; t0 += 64) {
        u32x4 qv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int t = t0 + 16 * u + m16;
            if (t < t_stop) {
                const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (int64_t)h * kD + 8 * kg;
                qv[u] = relu_packed16(*reinterpret_cast<const u32x4*>(src));
            } else {
                qv[u] = u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const typename V<T>::x8 bq = __builtin_bit_cast(typename V<T>::x8, qv[u]);
            f32x4 n0 = mfma16x16x32(shi[0], bq, zero);
            n0 = mfma16x16x32(slo[0], bq, n0);
            f32x4 n1 = mfma16x16x32(shi[1], bq, zero);
            n1 = mfma16x16x32(slo[1], bq, n1);
            f32x4 dn = mfma16x16x32(zhi, bq, zero);
            dn = mfma16x16x32(zlo, bq, dn);
            const int t = t0 + 16 * u + m16;
            if (t < t_stop) {
                const float den = dn[0] + eps;
                f32x4 o0, o1;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o0[i] = n0[i] / den;
                    o1[i] = n1[i] / den;
                }
                TO* dst = out + ((int64_t)b * N + t) * C + (int64_t)h * kD + 4 * kg;
                Store4<TO>::run(dst, o0);
                Store4<TO>::run(dst + 16, o1);
            }
        }
    }
}

// --------------------------------------------------------------------------
// Generic VALU path: any D with 128 % D == 0, any input dtype.
// --------------------------------------------------------------------------
constexpr int kGT = 32;  // tokens per generic tile

template <typename T, int DG>
__global__ __launch_bounds__(256) void linattn_state_generic(const T* __restrict__ qkv,
                                                             float* __restrict__ partial, int N,
                                                             int H, int split_len, int splits) {
    constexpr int SS = (DG + 1) * DG;
    constexpr int EPT = (SS + 255) / 256;
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int64_t C = (int64_t)H * DG;
    const int t_begin = s * split_len, t_end = min(N, t_begin + split_len);
    __shared__ float kt[kGT][DG], vt[kGT][DG + 1];
    float acc[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) acc[e] = 0.f;
    for (int t0 = t_begin; t0 < t_end; t0 += kGT) {
        for (int i = threadIdx.x; i < kGT * DG; i += 256) {
            const int tok = i / DG, c = i % DG, t = t0 + tok;
            float kv = 0.f, vv = 0.f;
            if (t < t_end) {
                const T* row = qkv + ((int64_t)b * N + t) * 3 * C + (int64_t)h * DG + c;
                kv = fmaxf(to_f32(row[C]), 0.f);
                vv = to_f32(row[2 * C]);
            }
            kt[tok][c] = kv;
            vt[tok][c] = vv;
            if (c == 0) vt[tok][DG] = t < t_end ? 1.f : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const int idx = threadIdx.x + 256 * e;
            if (idx < SS) {
                const int r = idx / DG, c = idx % DG;
                float a = acc[e];
                for (int tok = 0; tok < kGT; ++tok) a = fmaf(vt[tok][r], kt[tok][c], a);
                acc[e] = a;
            }
        }
        __syncthreads();
    }
    float* P = partial + ((int64_t)(b * H + h) * splits + s) * SS;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int idx = threadIdx.x + 256 * e;
        if (idx < SS) P[idx] = acc[e];
    }
}

template <typename T, typename TO, int DG>
__global__ __launch_bounds__(256) void linattn_out_generic(const T* __restrict__ qkv,
                                                           const float* __restrict__ state,
                                                           TO* __restrict__ out, int N, int H,
                                                           float eps) {
    constexpr int SS = (DG + 1) * DG;
    constexpr int TPI = 256 / DG > 0 ? 256 / DG : 1;  // tokens per pass (one thread per (t, r))
    const int h = blockIdx.y, b = blockIdx.z;
    const int64_t C = (int64_t)H * DG;
    __shared__ float st[SS];
    __shared__ float qt[TPI][DG];
    const float* S = state + (int64_t)(b * H + h) * SS;
    for (int i = threadIdx.x; i < SS; i += 256) st[i] = S[i];
    const int t_block = blockIdx.x * kOutTokens;
    const int t_stop = min(N, t_block + kOutTokens);
    for (int t0 = t_block; t0 < t_stop; t0 += TPI) {
        __syncthreads();
        for (int i = threadIdx.x; i < TPI * DG; i += 256) {
            const int tok = i / DG, c = i % DG, t = t0 + tok;
            qt[tok][c] = t < t_stop
                             ? fmaxf(to_f32(qkv[((int64_t)b * N + t) * 3 * C + (int64_t)h * DG + c]), 0.f)
                             : 0.f;
        }
        __syncthreads();
        if (threadIdx.x < TPI * DG) {
            const int tok = threadIdx.x / DG, r = threadIdx.x % DG, t = t0 + tok;
            if (t < t_stop) {
                float num = 0.f, den = 0.f;
                for (int c = 0; c < DG; ++c) {
                    num = fmaf(st[r * DG + c], qt[tok][c], num);
                    den = fmaf(st[DG * DG + c], qt[tok][c], den);
                }
                out[((int64_t)b * N + t) * C + (int64_t)h * DG + r] = from_f32<TO>(num / (den + eps));
            }
        }
    }
}

// --------------------------------------------------------------------------
// Host side.
// --------------------------------------------------------------------------
int64_t split_len_for(int64_t N, int64_t splits, int64_t align) {
    int64_t len = (N + splits - 1) / splits;
    return (len + align - 1) / align * align;
}

template <typename T, typename TO>
int run_mfma(const void* qkv, void* out, float* partial, float* state, int B, int N, int H,
             int splits, int split_len, float eps, hipStream_t stream) {
    hipLaunchKernelGGL((linattn_state_kernel<T>), dim3(splits, (H + 1) / 2, B), dim3(256), 0,
                       stream, static_cast<const T*>(qkv), partial, N, H, split_len, splits);
    if (int rc = check_launch("linattn_state_kernel launch")) return rc;
    hipLaunchKernelGGL(linattn_reduce_kernel, dim3(H, B), dim3(256), 0, stream, partial, state, H,
                       splits, kState);
    if (int rc = check_launch("linattn_reduce_kernel launch")) return rc;
    hipLaunchKernelGGL((linattn_out_kernel<T, TO>),
                       dim3((N + kOutTokens - 1) / kOutTokens, (H + 3) / 4, B), dim3(256), 0,
                       stream, static_cast<const T*>(qkv), state, static_cast<TO*>(out), N, H, eps);
    return check_launch("linattn_out_kernel launch");
}

template <typename T, typename TO, int DG>
int run_generic(const void* qkv, void* out, float* partial, float* state, int B, int N, int H,
                int splits, int split_len, float eps, hipStream_t stream) {
    hipLaunchKernelGGL((linattn_state_generic<T, DG>), dim3(splits, H, B), dim3(256), 0, stream,
                       static_cast<const T*>(qkv), partial, N, H, split_len, splits);
    if (int rc = check_launch("linattn_state_generic launch")) return rc;
    hipLaunchKernelGGL(linattn_reduce_kernel, dim3(H, B), dim3(256), 0, stream, partial, state, H,
                       splits, (DG + 1) * DG);
    if (int rc = check_launch("linattn_reduce_kernel launch")) return rc;
    hipLaunchKernelGGL((linattn_out_generic<T, TO, DG>),
                       dim3((N + kOutTokens - 1) / kOutTokens, H, B), dim3(256), 0, stream,
                       static_cast<const T*>(qkv), state, static_cast<TO*>(out), N, H, eps);
    return check_launch("linattn_out_generic launch");
}

template <typename T, typename TO>
int run_generic_d(int D, const void* qkv, void* out, float* partial, float* state, int B, int N,
                  int H, int splits, int split_len, float eps, hipStream_t stream) {
#define KF_GENERIC_CASE(DD) \
    case DD: return run_generic<T, TO, DD>(qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
    switch (D) {
        KF_GENERIC_CASE(1) KF_GENERIC_CASE(2) KF_GENERIC_CASE(4) KF_GENERIC_CASE(8)
        KF_GENERIC_CASE(16) KF_GENERIC_CASE(32) KF_GENERIC_CASE(64) KF_GENERIC_CASE(128)
        default: set_error("linattn: unsupported head dim %d", D); return KF_E_UNSUPPORTED;
    }
#undef KF_GENERIC_CASE
}

template <typename T>
int run_in(int out_dt, bool mfma, int D, const void* qkv, void* out, float* partial, float* state,
           int B, int N, int H, int splits, int split_len, float eps, hipStream_t stream) {
    if (mfma) {
        if constexpr (sizeof(T) == 2) {
            switch (out_dt) {
                case KF_F32: return run_mfma<T, float>(qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
                case KF_F16: return run_mfma<T, f16>(qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
                case KF_BF16: return run_mfma<T, bf16>(qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
            }
        }
    }
    switch (out_dt) {
        case KF_F32: return run_generic_d<T, float>(D, qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
        case KF_F16: return run_generic_d<T, f16>(D, qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
        case KF_BF16: return run_generic_d<T, bf16>(D, qkv, out, partial, state, B, N, H, splits, split_len, eps, stream);
    }
    set_error("linattn: unknown output dtype %d", out_dt);
    return KF_E_INVALID;
}

bool valid_dim(int64_t D) { return D > 0 && D <= 128 && 128 % D == 0; }

}  // namespace
}  // namespace kf

extern "C" int64_t kf_linattn_default_splits(int64_t batch, int64_t heads, int64_t dim,
                                             int64_t seq_len) {
    // Aim for about four state workgroups per CU, each streaming at least 64
    // tokens (one tile) of a head pair.
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 1;
    const int64_t groups = dim == kf::kD ? batch * ((heads + 1) / 2) : batch * heads;
    const int64_t target = 4 * (int64_t)kf::device_cu_count();
    int64_t splits = (target + groups - 1) / groups;
    const int64_t max_splits = (seq_len + kf::kTT - 1) / kf::kTT;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    return splits;
}

extern "C" int64_t kf_linattn_workspace_bytes(int64_t batch, int64_t heads, int64_t dim,
                                              int64_t splits) {
    if (batch <= 0 || heads <= 0 || !kf::valid_dim(dim)) return 0;
    if (splits < 1) splits = 1;
    const int64_t state = (dim + 1) * dim;
    return (int64_t)sizeof(float) * batch * heads * state * (splits + 1);
}

extern "C" int kf_linattn_fwd(const void* qkv, void* out, void* workspace, int64_t workspace_bytes,
                              int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                              int64_t splits, float eps, int in_dtype, int out_dtype,
                              kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(batch >= 0 && seq_len >= 0 && heads >= 0, KF_E_INVALID,
               "linattn: negative shape B=%lld N=%lld H=%lld", (long long)batch,
               (long long)seq_len, (long long)heads);
    KF_REQUIRE(valid_dim(dim), KF_E_INVALID, "linattn: dim must divide 128 and be at most 128, got %lld",
               (long long)dim);
    KF_REQUIRE(in_dtype == KF_F32 || in_dtype == KF_F16 || in_dtype == KF_BF16, KF_E_INVALID,
               "linattn: unknown input dtype %d", in_dtype);
    KF_REQUIRE(out_dtype == KF_F32 || out_dtype == KF_F16 || out_dtype == KF_BF16, KF_E_INVALID,
               "linattn: unknown output dtype %d", out_dtype);
    if (batch == 0 || seq_len == 0 || heads == 0) return KF_OK;
    KF_REQUIRE(qkv && out, KF_E_INVALID, "linattn: null pointer");
    KF_REQUIRE(batch <= 65535 && heads <= 65535 && seq_len <= 0x3fffffff, KF_E_UNSUPPORTED,
               "linattn: shape exceeds grid limits");
    if (splits <= 0) splits = kf_linattn_default_splits(batch, heads, dim, seq_len);
    if (splits > seq_len) splits = seq_len;
    const int64_t need = kf_linattn_workspace_bytes(batch, heads, dim, splits);
    KF_REQUIRE(workspace && workspace_bytes >= need, KF_E_WORKSPACE,
               "linattn: workspace of %lld bytes needed, %lld given", (long long)need,
               (long long)workspace_bytes);
    const bool mfma = dim == kD && in_dtype != KF_F32 && (uintptr_t)qkv % 16 == 0 &&
                      (uintptr_t)out % 16 == 0;
    const int64_t split_len = split_len_for(seq_len, splits, mfma ? kTT : kGT);
    const int64_t eff_splits = (seq_len + split_len - 1) / split_len;
    KF_REQUIRE(eff_splits <= 0x7fffffff, KF_E_UNSUPPORTED, "linattn: too many splits");
    const int64_t state_size = (dim + 1) * dim;
    float* partial = static_cast<float*>(workspace);
    float* state = partial + batch * heads * state_size * splits;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int B = (int)batch, N = (int)seq_len, H = (int)heads, D = (int)dim;
    const int S = (int)eff_splits, L = (int)split_len;
    switch (in_dtype) {
        case KF_BF16: return run_in<bf16>(out_dtype, mfma, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
        case KF_F16: return run_in<f16>(out_dtype, mfma, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
        default: return run_in<float>(out_dtype, false, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
    }
}
