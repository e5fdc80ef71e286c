// Projection GEMM of the SANA LiteLA block on gfx950:
//   y[m][n] = dt( sum_k x[m][k] * W[n][k]  (+ bias[n]) )
// the QKV projection (no bias) and the bias-fused output projection of
// SANA_LinearAttention/custom.py:23-85 and :457-523, for either weight layout
// (the tile machinery and its design notes are in gemm_tile.h).
#include "gemm_tile.h"

namespace kf {
namespace {

constexpr int kGroupM = 8;  // tile rows walked before the next tile column

struct GemmParams {
    const void* x;     // [M][ldx]
    const void* w;     // [N][K] (NK) or [K][N] (KN), dense
    const void* bias;  // [N] or null
    void* y;           // [M][ldy]
    int M, N, K;
    int64_t ldx, ldy;
    int tiles_m, tiles_n;
    int staged_out;  // y and its row stride are 16-byte aligned: whole-chunk stores
};

// Logical block -> (tile row, tile column), kGroupM tile rows per column step:
// consecutive logical blocks (one XCD's range) share activation and weight
// panels in that XCD's L2.
__device__ __forceinline__ void gemm_tile(int blk, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int per_group = kGroupM * tiles_n;
    const int g = blk / per_group, r = blk - g * per_group;
    const int first = g * kGroupM;
    const int gm = min(kGroupM, tiles_m - first);
    tm = first + r % gm;
    tn = r / gm;
}

// Output tile staged in the (then free) stage buffers: rows of BN elements
// plus 16 bytes, so the 16 rows one 8- or 16-byte staging write touches fall
// on different banks.  A tile that does not fit goes through in PASSES bands
// of whole wavefront rows (WM rows each).
template <typename T, typename C> struct StagedOut {
    static constexpr int ROWE = C::BN + 16 / (int)sizeof(T);     // elements per staged row
    static constexpr int CHUNKS = C::BN * (int)sizeof(T) / 16;    // 16-byte chunks per output row
    static constexpr int SPACE = C::STAGES * (C::XS + C::WS);     // elements of the stage buffers
    static constexpr int PASSES = C::BM * ROWE <= SPACE ? 1 : (C::BM / 2) * ROWE <= SPACE ? 2 : 4;
    static constexpr int ROWS = C::BM / PASSES;                   // rows per pass
    static constexpr bool FITS = ROWS * ROWE <= SPACE && ROWS % C::WM == 0;
};

template <typename T, typename C, bool BIAS>
__global__ __launch_bounds__(C::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void proj_gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) T lds[C::STAGES * (C::XS + C::WS)];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int tm, tn;
    gemm_tile(gemm_logical_block(), p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;

    f32x4 acc[C::NB][C::MB];
    GemmSrc<T> src{static_cast<const T*>(p.x), p.ldx, m0, p.M, static_cast<const T*>(p.w), p.K, n0, p.N};
    src.w_rows_linear = n0 + C::BN <= p.N;  // no clamped weight rows in this tile
    const int nlast = p.N - 1;
    gemm_mainloop<T, C>(src, [n0, nlast](int r) { return (int64_t)min(n0 + r, nlast); }, lds, wave, lane, acc);

    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    T* y = static_cast<T*>(p.y);
    typedef StagedOut<T, C> SO;
    if constexpr (SO::FITS) {
        if (p.staged_out) {
            // Round (+ bias) into the staged tile, then store whole rows in
            // 16-byte chunks: full cache lines instead of the 32-byte row
            // pieces one MFMA block holds (which wrote 1.5x the output's
            // bytes at N = 2240).
#pragma unroll
            for (int pass = 0; pass < SO::PASSES; ++pass) {
                __syncthreads();  // the stage buffers (or the previous band) are free
                if (wm * C::WM / SO::ROWS == pass) {
#pragma unroll
                    for (int nb = 0; nb < C::NB; ++nb) {
                        const int nl = wn * C::WN + 16 * nb + 4 * (lane >> 4);
                        float bv[4] = {0.f, 0.f, 0.f, 0.f};
                        if constexpr (BIAS) {
                            if (n0 + nl < p.N) {
                                const T* bias = static_cast<const T*>(p.bias) + n0 + nl;
#pragma unroll
                                for (int i = 0; i < 4; ++i) bv[i] = to_f32(bias[i]);
                            }
                        }
#pragma unroll
                        for (int mb = 0; mb < C::MB; ++mb) {
                            const int ml = wm * C::WM - pass * SO::ROWS + 16 * mb + (lane & 15);
                            store4<BIAS>(lds + ml * SO::ROWE + nl, acc[nb][mb], bv);
                        }
                    }
                }
                __syncthreads();
                constexpr int TOTAL = SO::ROWS * SO::CHUNKS;
#pragma unroll
                for (int k = 0; k < (TOTAL + C::THREADS - 1) / C::THREADS; ++k) {
                    const int c = k * C::THREADS + threadIdx.x;
                    if (TOTAL % C::THREADS != 0 && c >= TOTAL) break;
                    const int r = c / SO::CHUNKS, ch = c - r * SO::CHUNKS;
                    const int m = m0 + pass * SO::ROWS + r, n = n0 + ch * (16 / (int)sizeof(T));
                    // Nontemporal: 2.5-3.5% faster than plain stores at the
                    // config A shapes on MI355X (the output is not re-read here).
                    if (m < p.M && n < p.N)
                        __builtin_nontemporal_store(
                            *reinterpret_cast<const u32x4*>(lds + r * SO::ROWE + ch * (16 / (int)sizeof(T))),
                            reinterpret_cast<u32x4*>(y + (int64_t)m * p.ldy + n));
                }
            }
            return;
        }
    }
#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb) {
        const int n = n0 + wn * C::WN + 16 * nb + 4 * (lane >> 4);
        if (n >= p.N) continue;  // N % 4 == 0: all four channels are in or out
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (BIAS) {
            const T* bias = static_cast<const T*>(p.bias) + n;
#pragma unroll
            for (int i = 0; i < 4; ++i) bv[i] = to_f32(bias[i]);
        }
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) {
            const int m = m0 + wm * C::WM + 16 * mb + (lane & 15);
            if (m < p.M) store4<BIAS>(y + (int64_t)m * p.ldy + n, acc[nb][mb], bv);
        }
    }
}

// Tile shapes: 256 activation rows times BN output channels, 8 wavefronts of
// 64 x BN/2 (4 x 2; 4 x 2 measured faster than 2 x 4 at BN = 256), two
// 128-byte-row LDS stages (three for BN = 128).  The WeightT layout's swizzle
// needs BN = 128 or 256.
template <typename T, int BN, bool KN> struct ProjTile {
    typedef GemmCfg<T, 256, BN, 4, BN == 128 ? 3 : 2, KN> C;
};

template <typename C>
int launch_cfg(GemmParams p, bool bias, hipStream_t stream) {
    p.tiles_m = (p.M + C::BM - 1) / C::BM;
    p.tiles_n = (p.N + C::BN - 1) / C::BN;
    const int grid = p.tiles_m * p.tiles_n;
    if (bias) hipLaunchKernelGGL((proj_gemm_kernel<typename C::Elem, C, true>), dim3(grid), dim3(C::THREADS), 0, stream, p);
    else hipLaunchKernelGGL((proj_gemm_kernel<typename C::Elem, C, false>), dim3(grid), dim3(C::THREADS), 0, stream, p);
    return check_launch("proj_gemm_kernel");
}

// Output-tile width for an M x N problem.  One workgroup runs per CU, so the
// launch takes ceil(tiles / CUs) rounds, and a round of BN-wide tiles costs
// about BN + 92 (a fixed per-tile part plus work proportional to the width).
// Fitted to a sweep of every width over nine shapes on MI355X (M = 4096-16384,
// N = 1152-6720, K = 1152-2240): per round at K = 2240 about 36 us at BN = 128,
// 42 at 160, 47 at 192, 54 at 224, 56-62 at 256 and 66-72 at 320; the model
// picks the fastest width, or one within 1.5% of it, at all nine.
inline int pick_bn(int M, int N, const int* cands, int n_cands) {
    const int cus = device_cu_count();
    int best = cands[0];
    long long best_cost = -1;
    for (int i = 0; i < n_cands; ++i) {
        const int bn = cands[i];
        const long long tiles = (long long)((M + 255) / 256) * ((N + bn - 1) / bn);
        const long long cost = (tiles + cus - 1) / cus * (bn + 92);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = bn;
        }
    }
    return best;
}

template <typename T, bool KN>
int launch_gemm(const GemmParams& p, bool bias, hipStream_t st) {
    // 16-bit weights in [N][K]: six widths; fp32 or WeightT: 256 and 128.
    if constexpr (sizeof(T) == 2 && !KN) {
        static const int cands[] = {320, 224, 256, 192, 160, 128};
        switch (pick_bn(p.M, p.N, cands, 6)) {
        case 320: return launch_cfg<typename ProjTile<T, 320, KN>::C>(p, bias, st);
        case 256: return launch_cfg<typename ProjTile<T, 256, KN>::C>(p, bias, st);
        case 224: return launch_cfg<typename ProjTile<T, 224, KN>::C>(p, bias, st);
        case 192: return launch_cfg<typename ProjTile<T, 192, KN>::C>(p, bias, st);
        case 160: return launch_cfg<typename ProjTile<T, 160, KN>::C>(p, bias, st);
        default: return launch_cfg<typename ProjTile<T, 128, KN>::C>(p, bias, st);
        }
    } else {
        static const int cands[] = {256, 128};
        if (pick_bn(p.M, p.N, cands, 2) == 256) return launch_cfg<typename ProjTile<T, 256, KN>::C>(p, bias, st);
        return launch_cfg<typename ProjTile<T, 128, KN>::C>(p, bias, st);
    }
}

template <typename T> int launch_gemm_layout(const GemmParams& p, int layout, bool bias, hipStream_t st) {
    return layout == KF_WEIGHT_NK ? launch_gemm<T, false>(p, bias, st) : launch_gemm<T, true>(p, bias, st);
}

bool aligned(const void* p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

}  // namespace
}  // namespace kf

extern "C" int kf_proj_gemm(const void* x, const void* weight, const void* bias, void* y, int64_t m, int64_t n,
                            int64_t k, int64_t ldx, int64_t ldy, int weight_layout, int dtype,
                            kf_stream_t stream) {
    using namespace kf;
    clear_error();
    KF_REQUIRE(dtype == KF_BF16 || dtype == KF_F16 || dtype == KF_F32, KF_E_INVALID,
               "kf_proj_gemm: dtype must be bf16, f16 or f32");
    KF_REQUIRE(weight_layout == KF_WEIGHT_NK || weight_layout == KF_WEIGHT_KN, KF_E_INVALID,
               "kf_proj_gemm: weight_layout must be KF_WEIGHT_NK or KF_WEIGHT_KN");
    KF_REQUIRE(m >= 0 && n >= 8 && k >= 8, KF_E_INVALID, "kf_proj_gemm: need m >= 0, n >= 8, k >= 8");
    KF_REQUIRE(n % 8 == 0 && k % 8 == 0, KF_E_INVALID,
               "kf_proj_gemm: n and k must be multiples of 8, got n=%lld k=%lld", (long long)n, (long long)k);
    KF_REQUIRE(ldx >= k && ldx % 8 == 0 && ldy >= n && ldy % 4 == 0, KF_E_INVALID,
               "kf_proj_gemm: need ldx >= k, ldx %% 8 == 0, ldy >= n, ldy %% 4 == 0");
    KF_REQUIRE(m < (1LL << 31) && n < (1LL << 31) && k < (1LL << 31), KF_E_INVALID,
               "kf_proj_gemm: dimensions must fit in 31 bits");
    if (m == 0) return KF_OK;
    KF_REQUIRE(x && weight && y, KF_E_INVALID, "kf_proj_gemm: null pointer");
    const int es = dtype == KF_F32 ? 4 : 2;
    KF_REQUIRE(aligned(x, 16) && aligned(weight, 16) && aligned(y, 4 * es) && (!bias || aligned(bias, es)),
               KF_E_INVALID, "kf_proj_gemm: x and weight must be 16-byte aligned, y aligned to 4 elements");
    GemmParams p{};
    p.x = x;
    p.w = weight;
    p.bias = bias;
    p.y = y;
    p.M = (int)m;
    p.N = (int)n;
    p.K = (int)k;
    p.ldx = ldx;
    p.ldy = ldy;
    p.staged_out = aligned(y, 16) && (ldy * es) % 16 == 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool b = bias != nullptr;
    if (dtype == KF_BF16) return launch_gemm_layout<bf16>(p, weight_layout, b, st);
    if (dtype == KF_F16) return launch_gemm_layout<f16>(p, weight_layout, b, st);
    return launch_gemm_layout<float>(p, weight_layout, b, st);
}
