// Fused LiteLA projection + ReLU linear attention for gfx950 (head dim 32,
// bf16/f16): the idea of SANA_LinearAttention/custom.py:606-809 (K/V
// projection fused with ReLU and the state partials; Q projection fused with
// the partial reduction and the output), for any batch, sequence length and
// head count.
//
// For x[b][t][:] (C = 32 H channels) and the packed weight W[3C][C] (rows
// 0..C-1 = q, C..2C-1 = k, 2C..3C-1 = v, plus an optional bias[3C]):
//   q, k, v = dt(x W^T + bias)            (fp32 accumulation, one rounding)
//   S_h[r][c] = sum_t v[t][32h + r] relu(k[t][32h + c]),  z_h[c] = sum_t relu(k[t][32h + c])
//   out[t][32h + r] = dt( sum_c S_h[r][c] relu(q[t][32h + c]) / (sum_c z_h[c] relu(q[t][32h + c]) + eps) )
// i.e. LiteLA.forward up to the output projection (original.py:119-142, the
// fp32 attention of :99-117) with the q, k and v values the unfused path
// stores in its packed qkv buffer.
//
// Three launches; the first and last are 256-token x HG-head (HG = 3 or 4)
// tile GEMMs on the gemm_tile.h mainloop:
//   1. litela_kv_state_kernel: the tile's k and v channels (256 weight rows),
//      rounded, ReLU on k, staged in LDS, then S and z of the tile's 256
//      tokens on v_mfma_f32_32x32x16 -> one partial per (batch, head, token
//      tile) in the workspace.  k and v never reach HBM.
//   2. litela_state_reduce_kernel: the partials of each (batch, head) summed
//      in token-tile order (deterministic).
//   3. litela_q_out_kernel: the tile's q channels, rounded, ReLU, staged in
//      LDS, contracted with the state held as hi+lo 16-bit MFMA operands (the
//      denominator rides as a third operand), normalised and stored.  q never
//      reaches HBM.
#include <cmath>

#include "gemm_tile.h"

namespace kf {
namespace {

constexpr int kHD = 32;                        // head dim
constexpr int kHState = (kHD + 1) * kHD;       // S (32 x 32) then z (32), floats
constexpr int kTok = 256;                      // tokens per workgroup

// kv tile of HG heads (3 or 4): 2 * 32 HG weight rows (HG heads of k, then HG
// of v); 4 x 2 wavefronts of 64 tokens x 32 HG channels: wavefront column 0
// holds k, column 1 holds v.
template <typename T, int HG> using KvCfg = GemmCfg<T, kTok, 2 * HG * kHD, 4, 2, false>;
// q tile: 32 HG weight rows (HG heads of q), three stages.
template <typename T, int HG> using QCfg = GemmCfg<T, kTok, HG * kHD, 4, 3, false>;

struct FusedLaParams {
    const void* x;       // [B][N][C]
    const void* w;       // [3C][C]
    const void* bias;    // [3C] or null
    void* out;           // [B][N][C]
    float* partial;      // [B][H][TT][33][32]
    float* state;        // [B][H][33][32]
    int B, N, H, C, TT, HG;
    float eps;
};

// kv tile in LDS: [256 tokens][256 channels] of 16-bit values, 512-byte rows,
// k of head j at channels 32j.., v of head j at 128 + 32j.. (rows padded when
// HG = 3).  The 16-byte chunk index is xor'ed with kvswz(t) < 16 (so k and v
// stay in their 256-byte halves): the 16 tokens of an 8-byte accumulator store
// hit 16 distinct chunk slots, and the 4 consecutive tokens of a transposing
// operand read land in 4 distinct 64-byte quarters of a bank line.
__device__ __forceinline__ int kvswz(int t) { return 4 * (t & 3) + ((t >> 2) & 3); }
__device__ __forceinline__ int kv_elem(int t, int ch) { return t * 256 + ((((ch >> 3) ^ kvswz(t))) << 3) + (ch & 7); }
// q tile: [256 tokens][128 channels] (padded when HG = 3), 256-byte rows,
// chunk ^ (t & 15): the 16 tokens of an operand read (one chunk each) hit 16
// distinct slots.
__device__ __forceinline__ int q_elem(int t, int ch) { return t * 128 + ((((ch >> 3) ^ (t & 15))) << 3) + (ch & 7); }

// Logical block -> (token tile row tm over all batches of the launch, head
// group hg), 8 token tiles per head-group step (the gemm_tile.h XCD ranges
// then share x panels and weight panels).
__device__ __forceinline__ void fused_tile(int blk, int tiles_m, int hg_count, int& tm, int& hg) {
    const int per_group = 8 * hg_count;
    const int g = blk / per_group, r = blk - g * per_group;
    const int first = g * 8;
    const int gm = min(8, tiles_m - first);
    tm = first + r % gm;
    hg = r / gm;
}

// Four accumulators (+ bias) rounded to T.
template <typename T> __device__ __forceinline__ void round4(const f32x4& v, const float (&bv)[4], T (&o)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (T)(v[i] + bv[i]);
}

template <typename T> __device__ __forceinline__ void load_bias4(const T* bias, int64_t idx, float (&bv)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) bv[i] = bias ? to_f32(bias[idx + i]) : 0.f;
}

template <typename T, int HG>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void litela_kv_state_kernel(FusedLaParams p) {
    typedef KvCfg<T, HG> Cf;
    constexpr int KW = HG * kHD;  // k (or v) channels of the tile
    constexpr int STAGE_ELEMS = Cf::STAGES * (Cf::XS + Cf::WS);
    constexpr int KV_ELEMS = kTok * 256;
    constexpr int COMB_BYTES = HG * 64 * 17 * 4;
    constexpr int LDS_BYTES = (STAGE_ELEMS > KV_ELEMS ? STAGE_ELEMS : KV_ELEMS) * 2 + COMB_BYTES;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(16))) unsigned char lds_raw[LDS_BYTES];
    T* lds = reinterpret_cast<T*>(lds_raw);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int tm, hg;
    fused_tile(gemm_logical_block(), gridDim.x / p.HG, p.HG, tm, hg);
    const int bl = tm / p.TT, tt = tm - bl * p.TT;  // batch within the launch, token tile
    const int b = bl;
    const int t0 = tt * kTok, h0 = hg * HG;
    const int64_t C = p.C;
    const T* x = static_cast<const T*>(p.x);
    const T* w = static_cast<const T*>(p.w);
    const T* bias = static_cast<const T*>(p.bias);

    f32x4 acc[Cf::NB][Cf::MB];
    {
        const int64_t row0 = (int64_t)b * p.N + t0;
        GemmSrc<T> src{x, C, row0, (int64_t)b * p.N + p.N, w, p.C, 0, 0};
        src.w_rows_linear = true;  // 8-row blocks stay inside one head's 32 rows of k or v
        const int hlast = p.H - 1;
        auto wrow = [C, h0, hlast](int r) {
            const int part = r >= KW ? 1 : 0, rr = r - part * KW;
            const int hh = min(h0 + (rr >> 5), hlast);
            return (int64_t)(1 + part) * C + (int64_t)hh * kHD + (rr & 31);
        };
        gemm_mainloop<T, Cf>(src, wrow, lds, wave, lane, acc);
    }

    // ---- k and v tile -> LDS (rounded, ReLU on k, zero past the sequence) ----
    __syncthreads();  // every wavefront is done with the stage buffers
    const int wm = wave / Cf::WAVES_N, wn = wave % Cf::WAVES_N;  // wn 0: k, 1: v
#pragma unroll
    for (int nb = 0; nb < Cf::NB; ++nb) {
        const int cw = 16 * nb + 4 * (lane >> 4);  // channel within the k (or v) part
        const int ch = wn * 128 + cw;              // LDS channel
        const int hh = min(h0 + (cw >> 5), p.H - 1);
        float bv[4];
        load_bias4(bias, (int64_t)(1 + wn) * C + (int64_t)hh * kHD + (cw & 31), bv);
#pragma unroll
        for (int mb = 0; mb < Cf::MB; ++mb) {
            const int t = wm * Cf::WM + 16 * mb + (lane & 15);
            T o[4];
            round4(acc[nb][mb], bv, o);
            const bool live = t0 + t < p.N;
            u32x2 pk;
            unsigned short* e = reinterpret_cast<unsigned short*>(&pk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                unsigned short bits = __builtin_bit_cast(unsigned short, o[i]);
                if (wn == 0 && (bits & 0x8000u)) bits = 0;  // ReLU (-0 -> +0)
                e[i] = live ? bits : (unsigned short)0;
            }
            *reinterpret_cast<u32x2*>(lds + kv_elem(t, ch)) = pk;
        }
    }
    __syncthreads();

    // ---- S = v^T relu(k), z = sum relu(k): wavefront (head hl, token half th) ----
    const int hl = wave >> 1, th = wave & 1;
    const int g16 = lane >> 4, j16 = lane & 15;
    f32x16 s32;
#pragma unroll
    for (int i = 0; i < 16; ++i) s32[i] = 0.f;
    float zsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        const int row = th * 128 + ks * 16 + 8 * (g16 >> 1) + (j16 >> 2);
        const int c4 = 16 * (g16 & 1) + 4 * (j16 & 3);
        const typename V<T>::x4 a0 = lds_read_tr(lds + kv_elem(row, 128 + 32 * hl + c4));
        const typename V<T>::x4 a1 = lds_read_tr(lds + kv_elem(row + 4, 128 + 32 * hl + c4));
        const typename V<T>::x4 b0 = lds_read_tr(lds + kv_elem(row, 32 * hl + c4));
        const typename V<T>::x4 b1 = lds_read_tr(lds + kv_elem(row + 4, 32 * hl + c4));
        typename V<T>::x8 av, bk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            av[j] = a0[j];
            av[j + 4] = a1[j];
            bk[j] = b0[j];
            bk[j + 4] = b1[j];
        }
        s32 = mfma32x32x16(av, bk, s32);
#pragma unroll
        for (int j = 0; j < 8; ++j) zsum += (float)bk[j];
    }
    zsum += __shfl_xor(zsum, 32, 64);  // lanes l and l+32 hold the same key channel

    // Combine the two token halves (half 0 + half 1), write the partial.
    float (*comb)[64][17] = reinterpret_cast<float (*)[64][17]>(lds_raw + LDS_BYTES - COMB_BYTES);
    if (th == 1 && hl < HG) {
#pragma unroll
        for (int i = 0; i < 16; ++i) comb[hl][lane][i] = s32[i];
        comb[hl][lane][16] = zsum;
    }
    __syncthreads();
    const int h = h0 + hl;
    if (th == 0 && hl < HG && h < p.H) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s32[i] += comb[hl][lane][i];
        zsum += comb[hl][lane][16];
        float* P = p.partial + (((int64_t)b * p.H + h) * p.TT + tt) * kHState;
        const int c = lane & 31;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            P[r * kHD + c] = s32[i];
        }
        if (lane < 32) P[kHD * kHD + c] = zsum;
    }
}

// state[b][h][:] = sum over token tiles j (in order) of partial[b][h][j][:];
// one thread per 16-byte vector, eight tiles' loads in flight at a time.
__global__ __launch_bounds__(256) void litela_state_reduce_kernel(const float* __restrict__ partial,
                                                                  float* __restrict__ state, int64_t nbh, int TT) {
    constexpr int V4 = kHState / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= nbh * V4) return;
    const int64_t bh = idx / V4;
    const int v = (int)(idx - bh * V4);
    const f32x4* P = reinterpret_cast<const f32x4*>(partial + bh * TT * kHState) + v;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < TT; j0 += 8) {
        f32x4 t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = j0 + j < TT ? P[(int64_t)(j0 + j) * V4] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += t[j];  // tile order; padding adds zero
    }
    reinterpret_cast<f32x4*>(state + bh * kHState)[v] = acc;
}

template <typename T, int HG>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void litela_q_out_kernel(FusedLaParams p) {
    typedef QCfg<T, HG> Cf;
    constexpr int STAGE_ELEMS = Cf::STAGES * (Cf::XS + Cf::WS);
    constexpr int Q_ELEMS = kTok * 128;
    static_assert(STAGE_ELEMS >= Q_ELEMS, "q tile fits in the stage buffers");
    __shared__ __attribute__((aligned(16))) T lds[STAGE_ELEMS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int tm, hg;
    fused_tile(gemm_logical_block(), gridDim.x / p.HG, p.HG, tm, hg);
    const int bl = tm / p.TT, tt = tm - bl * p.TT;
    const int b = bl;
    const int t0 = tt * kTok, h0 = hg * HG;
    const int64_t C = p.C;
    const T* x = static_cast<const T*>(p.x);
    const T* w = static_cast<const T*>(p.w);
    const T* bias = static_cast<const T*>(p.bias);

    f32x4 acc[Cf::NB][Cf::MB];
    {
        const int64_t row0 = (int64_t)b * p.N + t0;
        GemmSrc<T> src{x, C, row0, (int64_t)b * p.N + p.N, w, p.C, 0, 0};
        src.w_rows_linear = true;  // 8-row blocks stay inside one head's 32 rows of q
        const int hlast = p.H - 1;
        auto wrow = [h0, hlast](int r) { return (int64_t)min(h0 + (r >> 5), hlast) * kHD + (r & 31); };
        gemm_mainloop<T, Cf>(src, wrow, lds, wave, lane, acc);
    }

    // ---- relu(q) tile -> LDS ----
    __syncthreads();
    const int wm = wave / Cf::WAVES_N, wn = wave % Cf::WAVES_N;
#pragma unroll
    for (int nb = 0; nb < Cf::NB; ++nb) {
        const int ch = wn * Cf::WN + 16 * nb + 4 * (lane >> 4);
        const int hh = min(h0 + (ch >> 5), p.H - 1);
        float bv[4];
        load_bias4(bias, (int64_t)hh * kHD + (ch & 31), bv);
#pragma unroll
        for (int mb = 0; mb < Cf::MB; ++mb) {
            const int t = wm * Cf::WM + 16 * mb + (lane & 15);
            T o[4];
            round4(acc[nb][mb], bv, o);
            u32x2 pk;
            unsigned short* e = reinterpret_cast<unsigned short*>(&pk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned short bits = __builtin_bit_cast(unsigned short, o[i]);
                e[i] = (bits & 0x8000u) ? (unsigned short)0 : bits;  // ReLU (-0 -> +0)
            }
            *reinterpret_cast<u32x2*>(lds + q_elem(t, ch)) = pk;
        }
    }

    // ---- the state of head hl as hi+lo 16-bit A operands ----
    const int hl = wave >> 1, th = wave & 1;
    const int h = min(h0 + hl, p.H - 1);
    const int m16 = lane & 15, kg = lane >> 4;
    const float* S0 = p.state + ((int64_t)b * p.H + h) * kHState;
    float sv[2][8], zv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sv[0][j] = S0[m16 * kHD + 8 * kg + j];
        sv[1][j] = S0[(16 + m16) * kHD + 8 * kg + j];
        zv[j] = S0[kHD * kHD + 8 * kg + j];
    }
    // fp16 has a narrow exponent range: rescale the state by a power of two
    // (out = num/den is invariant to a common factor; only eps sees it).
    float scale = 1.f;
    if constexpr (!__is_same(T, bf16)) {
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
            const float v = sv[mb][j] * scale;
            const T hi = (T)v;
            shi[mb][j] = hi;
            slo[mb][j] = (T)(v - (float)hi);
        }
        const float v = zv[j] * scale;
        const T hi = (T)v;
        zhi[j] = hi;
        zlo[j] = (T)(v - (float)hi);
    }
    const float eps = p.eps * scale;
    __syncthreads();  // the q tile is complete

    // ---- out = S relu(q) / (z . relu(q) + eps), 16 tokens per step ----
    T* out = static_cast<T*>(p.out);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const int ch0 = (kg & 1) ? 16 + 4 * (kg - 1) : 4 * kg;
    const bool head_live = hl < HG && h0 + hl < p.H;
#pragma unroll 2
    for (int u = 0; u < 8; ++u) {
        const int t = th * 128 + 16 * u + m16;
        const typename V<T>::x8 bq =
            *reinterpret_cast<const typename V<T>::x8*>(lds + q_elem(t, 32 * hl + 8 * kg));
        f32x4 n0 = mfma16x16x32(shi[0], bq, zero);
        n0 = mfma16x16x32(slo[0], bq, n0);
        f32x4 n1 = mfma16x16x32(shi[1], bq, zero);
        n1 = mfma16x16x32(slo[1], bq, n1);
        f32x4 dn = mfma16x16x32(zhi, bq, zero);
        dn = mfma16x16x32(zlo, bq, dn);
        const float inv = 1.0f / (dn[0] + eps);
        typename V<T>::x8 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(n0[k] * inv), __float_as_uint(n1[k] * inv),
                                                            false, false);
            o[k] = (T)__uint_as_float(r[0]);
            o[k + 4] = (T)__uint_as_float(r[1]);
        }
        if (head_live && t0 + t < p.N) {
            T* dst = out + ((int64_t)b * p.N + t0 + t) * C + (int64_t)(h0 + hl) * kHD + ch0;
            __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), reinterpret_cast<u32x4*>(dst));
        }
    }
}

bool aligned_to(const void* p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

template <typename T, int HG> int run_fused(FusedLaParams p, hipStream_t st) {
    p.HG = (p.H + HG - 1) / HG;
    const int grid = p.B * p.TT * p.HG;
    hipLaunchKernelGGL((litela_kv_state_kernel<T, HG>), dim3(grid), dim3(512), 0, st, p);
    if (int rc = check_launch("litela_kv_state_kernel")) return rc;
    const int64_t nbh = (int64_t)p.B * p.H;
    const int64_t threads = nbh * (kHState / 4);
    hipLaunchKernelGGL(litela_state_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       p.partial, p.state, nbh, p.TT);
    if (int rc = check_launch("litela_state_reduce_kernel")) return rc;
    hipLaunchKernelGGL((litela_q_out_kernel<T, HG>), dim3(grid), dim3(512), 0, st, p);
    return check_launch("litela_q_out_kernel");
}

// Heads per workgroup (3 or 4): one workgroup per CU, so each launch takes
// ceil(tiles / CUs) rounds of a cost about proportional to the tile width
// plus a fixed part (the projection GEMM's model), summed over both launches.
int pick_heads_per_group(int B, int TT, int H) {
    const int cus = device_cu_count();
    auto cost = [&](int hg) {
        const long long tiles = (long long)B * TT * ((H + hg - 1) / hg);
        const long long rounds = (tiles + cus - 1) / cus;
        return rounds * (64 * hg + 32) + rounds * (32 * hg + 32);
    };
    return cost(3) < cost(4) ? 3 : 4;
}

}  // namespace
}  // namespace kf

extern "C" int64_t kf_litela_fused_workspace_bytes(int64_t batch, int64_t seq_len, int64_t heads) {
    using namespace kf;
    if (batch < 0 || seq_len < 0 || heads < 1) return -1;
    const int64_t tt = (seq_len + kTok - 1) / kTok;
    return 4 * batch * heads * kHState * (tt + 1);
}

namespace kf {
namespace {

// heads_per_group: 3 or 4 heads per workgroup, 0 = chosen per shape.
int litela_fused_run(const void* x, const void* qkv_weight, const void* qkv_bias, void* out, void* workspace,
                     int64_t workspace_bytes, int64_t batch, int64_t seq_len, int64_t heads, int64_t dim, float eps,
                     int dtype, int heads_per_group, kf_stream_t stream) {
    clear_error();
    KF_REQUIRE(dtype == KF_BF16 || dtype == KF_F16, KF_E_INVALID, "kf_litela_fused_attn: dtype must be bf16 or f16");
    KF_REQUIRE(dim == kHD, KF_E_UNSUPPORTED, "kf_litela_fused_attn: head dim must be 32, got %lld", (long long)dim);
    KF_REQUIRE(batch >= 0 && seq_len >= 0 && heads >= 1, KF_E_INVALID, "kf_litela_fused_attn: bad shape");
    KF_REQUIRE(std::isfinite(eps) && eps >= 0.f, KF_E_INVALID, "kf_litela_fused_attn: eps must be finite and >= 0");
    const int64_t C = heads * kHD;
    KF_REQUIRE(batch * seq_len < (1LL << 31) && 3 * C < (1LL << 31) &&
                   batch * ((seq_len + kTok - 1) / kTok) * ((heads + 2) / 3) < (1LL << 31),
               KF_E_INVALID,
               "kf_litela_fused_attn: sizes must fit in 31 bits");
    if (batch == 0 || seq_len == 0) return KF_OK;
    KF_REQUIRE(x && qkv_weight && out, KF_E_INVALID, "kf_litela_fused_attn: null pointer");
    KF_REQUIRE(aligned_to(x, 16) && aligned_to(qkv_weight, 16) && aligned_to(out, 16) &&
                   (!qkv_bias || aligned_to(qkv_bias, 2)),
               KF_E_INVALID, "kf_litela_fused_attn: x, qkv_weight and out must be 16-byte aligned");
    const int64_t need = kf_litela_fused_workspace_bytes(batch, seq_len, heads);
    KF_REQUIRE(workspace && workspace_bytes >= need && aligned_to(workspace, 256), KF_E_WORKSPACE,
               "kf_litela_fused_attn: need a 256-byte aligned workspace of %lld bytes, got %lld", (long long)need,
               (long long)workspace_bytes);
    FusedLaParams p{};
    p.x = x;
    p.w = qkv_weight;
    p.bias = qkv_bias;
    p.out = out;
    const int64_t tt = (seq_len + kTok - 1) / kTok;
    p.partial = static_cast<float*>(workspace);
    p.state = p.partial + batch * heads * tt * kHState;
    p.B = (int)batch;
    p.N = (int)seq_len;
    p.H = (int)heads;
    p.C = (int)C;
    p.TT = (int)tt;
    p.eps = eps;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int hg = heads_per_group > 0 ? heads_per_group : pick_heads_per_group(p.B, p.TT, p.H);
    if (hg == 3) return dtype == KF_BF16 ? run_fused<bf16, 3>(p, st) : run_fused<f16, 3>(p, st);
    return dtype == KF_BF16 ? run_fused<bf16, 4>(p, st) : run_fused<f16, 4>(p, st);
}

}  // namespace
}  // namespace kf

extern "C" int kf_litela_fused_attn(const void* x, const void* qkv_weight, const void* qkv_bias, void* out,
                                    void* workspace, int64_t workspace_bytes, int64_t batch, int64_t seq_len,
                                    int64_t heads, int64_t dim, float eps, int dtype, kf_stream_t stream) {
    return kf::litela_fused_run(x, qkv_weight, qkv_bias, out, workspace, workspace_bytes, batch, seq_len, heads,
                                dim, eps, dtype, 0, stream);
}

// Test entry point (not in the public header): kf_litela_fused_attn with 3 or
// 4 heads per workgroup forced (0 keeps the per-shape choice), so tests reach
// both tile shapes.
extern "C" int kfm_litela_fused_attn_heads(const void* x, const void* qkv_weight, const void* qkv_bias, void* out,
                                           void* workspace, int64_t workspace_bytes, int64_t batch, int64_t seq_len,
                                           int64_t heads, int64_t dim, float eps, int dtype, int heads_per_group,
                                           kf_stream_t stream) {
    KF_REQUIRE(heads_per_group == 0 || heads_per_group == 3 || heads_per_group == 4, KF_E_INVALID,
               "kf_litela_fused_attn: heads per workgroup must be 0, 3 or 4");
    return kf::litela_fused_run(x, qkv_weight, qkv_bias, out, workspace, workspace_bytes, batch, seq_len, heads,
                                dim, eps, dtype, heads_per_group, stream);
}
