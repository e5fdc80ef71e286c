// Projection GEMMs of the SANA LiteLA block on gfx950:
//   y[m][n] = dt( sum_k x[m][k] * W[n][k]  (+ bias[n]) )
// with fp32 accumulation on the MFMA pipe and one rounding to the storage
// dtype dt at the end (the bias, when present, is added in fp32 before that
// rounding).  This is the QKV projection (x[B*N][C] times the packed [3C][C]
// weight, no bias) and the bias-fused output projection of
// SANA_LinearAttention/custom.py:23-85 and :457-523.
//
// The weight comes in either layout: [N][K] as torch.nn.Linear stores it
// (K contiguous, the MFMA operand order, read with ds_read_b128), or the
// reference's prepacked WeightT [K][N] (N contiguous, read column-wise: the
// transposing ds_read_b64_tr_b16 for 16-bit types, 4-byte reads for fp32).
//
// Workgroup: 8 wavefronts, a BM x BN output tile, K streamed through LDS in
// stages of 128-byte rows (64 16-bit or 32 fp32 elements) by global_load_lds
// copies (no register staging), STAGES buffers deep.  Each wavefront owns a
// WM x WN sub-tile.  A lane reads one 16-byte chunk per operand block and K
// step (two steps per stage): one v_mfma_f32_16x16x32 for bf16/f16, four
// v_mfma_f32_16x16x4f32 for fp32, whose K slices are taken as {4g + t} so that
// the same chunk read serves all four.  The MFMA computes the transposed
// product (A = weight rows, B = activation rows), so a lane ends with 4
// consecutive output channels of one token: 8- or 16-byte stores along the
// output row.
//
// Tiles are numbered so that each XCD (the hardware sends workgroup i to XCD
// i % 8) receives a contiguous range, and consecutive tiles walk 8 tile rows
// before moving to the next tile column: the 32 workgroups an XCD runs at once
// share 8 activation row panels and 4 weight panels in that XCD's L2.
#include "fa_common.h"

namespace kf {
namespace {

constexpr int kGroupM = 8;         // tile rows walked before the next tile column

struct GemmParams {
    const void* x;     // [M][ldx]
    const void* w;     // [N][K] (NK) or [K][N] (KN), dense
    const void* bias;  // [N] or null
    void* y;           // [M][ldy]
    int M, N, K;
    int64_t ldx, ldy;
    int tiles_m, tiles_n;
};

template <typename T, int BM_, int BN_, int WAVES_M_, int STAGES_, bool KN_, int ROWB_ = 128, int WAVES_ = 8>
struct GemmCfg {
    typedef T Elem;
    static constexpr int BM = BM_, BN = BN_, STAGES = STAGES_;
    static constexpr int WAVES = WAVES_, THREADS = 64 * WAVES;
    static constexpr bool KN = KN_;
    static constexpr int ROWB = ROWB_;                // bytes of K per tile row and stage: 64 or 128
    static constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
    static constexpr int CPR = ROWB / 16;             // chunks per tile row
    static constexpr int BK = ROWB / (int)sizeof(T);  // K elements per stage
    static constexpr int STEPS = ROWB / 64;           // MFMA K steps per stage (64 bytes each)
    static constexpr int RPC = 64 / CPR;              // tile rows per copy instruction
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES / WAVES_M_;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int MB = WM / 16, NB = WN / 16;
    static constexpr int XS = BM * BK, WS = BN * BK;  // elements per stage
    // Copies per wavefront per stage (the fewest any wavefront issues when a
    // tile side is not a whole number of copy rounds).
    static constexpr int XI = BM / (WAVES * RPC), WI = BN / (WAVES * RPC);
    // Workgroups per CU the kernel is shaped for (LDS allows two when a
    // workgroup takes at most half of it).
    static constexpr int OCC = WAVES == 4 ? 2 : 1;
    static constexpr int LDS_BYTES = STAGES * (XS + WS) * (int)sizeof(T);
    static_assert(ROWB == 64 || ROWB == 128, "row geometry");
    static_assert(BM % (WAVES * RPC) == 0 && BN % 16 == 0, "activation tiles are whole copy rounds; 16-row blocks");
    static_assert(WAVES == 8 || WAVES == 4, "workgroup shape");
    static_assert(!KN || BN % 64 == 0, "WeightT tiles are whole copy rounds");
    static_assert(WM % 16 == 0 && WN % 16 == 0, "16x16 MFMA blocks");
    static_assert(!KN || BN == 128 || BN == 256, "the WeightT swizzles need 16..64 chunks per row");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// XCD-aware renumbering: XCD x (= blockIdx % 8) receives a contiguous range
// of logical blocks.
__device__ __forceinline__ int gemm_logical_block() {
    const int nblk = gridDim.x, id = blockIdx.x;
    const int per = nblk >> 3, rem = nblk & 7, xcd = id & 7, slot = id >> 3;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// Logical block -> (tile row, tile column), kGroupM tile rows per column step.
__device__ __forceinline__ void gemm_tile(int blk, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int per_group = kGroupM * tiles_n;
    const int g = blk / per_group, r = blk - g * per_group;
    const int first = g * kGroupM;
    const int gm = min(kGroupM, tiles_m - first);
    tm = first + r % gm;
    tn = r / gm;
}

// K-contiguous tile [R][BK] (rows of CPR 16-byte chunks): logical chunk c of
// row r sits at physical chunk c ^ kswz(r).  An operand read touches 16
// consecutive rows at one logical chunk; 256/(16 CPR) rows share a 256-byte
// bank line, and the map sends the rows of each residue class to distinct
// chunks, so the 16 lanes of a ds_read_b128 cycle hit 16 distinct 16-byte bank
// groups.
template <int CPR> __device__ __forceinline__ int kswz(int r) {
    if constexpr (CPR == 8) return (r >> 1) & 7;
    else return (r >> 2) & 3;
}

// WeightT tile [BK][BN]: logical chunk c of row k sits at c ^ nswz(k).
// 16-bit: a transposing operand read of a 32-lane half touches rows
// {0..3, 8..11} (+4, +32s) at one aligned chunk pair; the (even) map sends
// those 8 rows to 8 distinct pairs of a 256-byte bank line.  fp32: a 4-byte
// read touches rows {t, 4 + t, 8 + t, 12 + t} (+16s) at one 64-byte span; the
// map moves them to 4 distinct 64-byte quarters.
template <typename T> __device__ __forceinline__ int nswz(int k) {
    if constexpr (sizeof(T) == 2) return ((k & 3) | (((k >> 3) & 1) << 2)) << 1;
    else return ((k >> 2) & 3) << 2;
}

// Copy rows row0..row0+R-1 (clamped to rows_valid - 1: those rows only feed
// outputs that are never stored), K columns k0..k0+BK-1 (zero past K) of a
// K-contiguous matrix into a [R][BK] tile.  Instruction i covers tile rows
// RPC i .. RPC i + RPC-1; wavefront w issues i = w, w + 8, ...
template <typename T, typename C, int R>
__device__ __forceinline__ void copy_krows(T* tile, const T* g, int64_t ld, int row0, int rows_valid, int k0,
                                           int K, int wave, int lane) {
    constexpr int NI = R / C::RPC;
#pragma unroll
    for (int j = 0; j < (NI + C::WAVES - 1) / C::WAVES; ++j) {
        const int i = wave + C::WAVES * j;
        if (NI % C::WAVES != 0 && i >= NI) break;
        const int r = C::RPC * i + lane / C::CPR;
        const int c = (lane % C::CPR) ^ kswz<C::CPR>(r);
        const int gr = min(row0 + r, rows_valid - 1);
        const int kk = k0 + C::EPC * c;
        const void* src = kk < K ? static_cast<const void*>(g + (int64_t)gr * ld + kk)
                                 : static_cast<const void*>(g_zero16);
        lds_copy16(src, __builtin_amdgcn_readfirstlane(lds_addr(tile + C::RPC * i * C::BK)));
    }
}

// Copy WeightT rows k0..k0+BK-1 (zero past K), columns n0..n0+BN-1 (zero past
// N) into a [BK][BN] tile.  Instruction i covers 64 / CH rows.
template <typename T, typename C>
__device__ __forceinline__ void copy_kn(T* tile, const T* g, int N, int n0, int k0, int K, int wave, int lane) {
    constexpr int CH = C::BN / C::EPC, RPI = 64 / CH, NI = C::BK / RPI;
    static_assert(NI == C::WAVES * C::WI, "copy rounds");
#pragma unroll
    for (int j = 0; j < NI / C::WAVES; ++j) {
        const int i = wave + C::WAVES * j;
        const int r = RPI * i + lane / CH;
        const int c = (lane % CH) ^ nswz<T>(r);
        const int kk = k0 + r, nn = n0 + C::EPC * c;
        const void* src = (kk < K && nn < N) ? static_cast<const void*>(g + (int64_t)kk * N + nn)
                                             : static_cast<const void*>(g_zero16);
        lds_copy16(src, __builtin_amdgcn_readfirstlane(lds_addr(tile + RPI * i * C::BN)));
    }
}

// Operand chunk from a K-contiguous tile: lane l reads row r0 + l%16, logical
// chunk 4s + l/16 (16 bytes).
template <typename T, typename C>
__device__ __forceinline__ u32x4 op_krows(const T* tile, int r0, int s, int lane) {
    const int r = r0 + (lane & 15);
    const int c = (4 * s + (lane >> 4)) ^ kswz<C::CPR>(r);
    return *reinterpret_cast<const u32x4*>(tile + r * C::BK + c * C::EPC);
}

// The same operand chunk (row = output channel n0 + l%16, the chunk's K
// elements 4s'.. in the K-contiguous order) from a WeightT tile.
template <typename T, typename C>
__device__ __forceinline__ u32x4 op_kn(const T* tile, int n0, int s, int lane) {
    const int g = lane >> 4, j16 = lane & 15;
    if constexpr (sizeof(T) == 2) {
        // Two transposing reads of 4 K rows each: lanes 4q..4q+3 of a 16-lane
        // group address row k + q; lane j16 receives channel n0 + j16.
        const int k = 32 * s + 8 * g + (j16 >> 2);
        const int n = n0 + 4 * (j16 & 3);
        const typename V<T>::x4 lo =
            lds_read_tr(tile + k * C::BN + (((n >> 3) ^ nswz<T>(k)) << 3) + (n & 7));
        const typename V<T>::x4 hi =
            lds_read_tr(tile + (k + 4) * C::BN + (((n >> 3) ^ nswz<T>(k + 4)) << 3) + (n & 7));
        typename V<T>::x8 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[j] = lo[j];
            r[j + 4] = hi[j];
        }
        return __builtin_bit_cast(u32x4, r);
    } else {
        // fp32: K elements 16s + 4g + t, t = 0..3, one 4-byte read each.
        const int n = n0 + j16;
        u32x4 r;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int k = 16 * s + 4 * g + t;
            r[t] = __float_as_uint(tile[k * C::BN + (((n >> 2) ^ nswz<T>(k)) << 2) + (n & 3)]);
        }
        return r;
    }
}

// acc += A-chunk x B-chunk: one 16x16x32 MFMA (16-bit) or four 16x16x4 fp32
// MFMAs over the K slices {4g + t} (g = l/16; the same slices in A and B).
template <typename T> __device__ __forceinline__ f32x4 mma_chunk(u32x4 a, u32x4 b, f32x4 acc) {
    if constexpr (sizeof(T) == 2) {
        return mfma16x16x32(__builtin_bit_cast(typename V<T>::x8, a), __builtin_bit_cast(typename V<T>::x8, b),
                            acc);
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[t]), __uint_as_float(b[t]), acc, 0, 0, 0);
        return acc;
    }
}

// s_waitcnt vmcnt(N) with the expcnt / lgkmcnt fields left at their maxima.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Wait until the copies of stage kt have landed when `ahead` later stages
// (0 .. STAGES-2) have been issued behind it.  Loads retire in order, so
// allowing PER * ahead outstanding (PER = the fewest copies any wavefront
// issues per stage) is sufficient for every wavefront.
template <int STAGES, int PER, int A = STAGES - 2> __device__ __forceinline__ void wait_stage(int ahead) {
    if constexpr (A > 0) {
        if (ahead >= A) {
            wait_vmcnt<A * PER>();
            return;
        }
        wait_stage<STAGES, PER, A - 1>(ahead);
    } else {
        wait_vmcnt<0>();
    }
}

// Accumulate one wavefront's WM x WN sub-tile over the whole K range.
// acc[nb][mb][i] = y[m = wm*WM + 16 mb + l%16][n = wn*WN + 16 nb + 4(l/16) + i].
template <typename T, typename C>
__device__ __forceinline__ void gemm_mainloop(const GemmParams& p, T* lds, int m0, int n0, int wave, int lane,
                                              f32x4 (&acc)[C::NB][C::MB]) {
    constexpr int PER = C::XI + C::WI;
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const T* x = static_cast<const T*>(p.x);
    const T* w = static_cast<const T*>(p.w);
    const int KT = (p.K + C::BK - 1) / C::BK;

    auto issue = [&](int kt) {
        T* xs = lds + (kt % C::STAGES) * (C::XS + C::WS);
        T* ws = xs + C::XS;
        copy_krows<T, C, C::BM>(xs, x, p.ldx, m0, p.M, kt * C::BK, p.K, wave, lane);
        if constexpr (C::KN) copy_kn<T, C>(ws, w, p.N, n0, kt * C::BK, p.K, wave, lane);
        else copy_krows<T, C, C::BN>(ws, w, p.K, n0, p.N, kt * C::BK, p.K, wave, lane);
    };

#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < C::STAGES - 1; ++s)
        if (s < KT) issue(s);

    for (int kt = 0; kt < KT; ++kt) {
        wait_stage<C::STAGES, PER>(min(C::STAGES - 2, KT - 1 - kt));
        __syncthreads();  // stage kt is complete for every wavefront; stage kt-1 is free
        if (kt + C::STAGES - 1 < KT) issue(kt + C::STAGES - 1);
        const T* xs = lds + (kt % C::STAGES) * (C::XS + C::WS);
        const T* ws = xs + C::XS;
#pragma unroll
        for (int s = 0; s < C::STEPS; ++s) {
            u32x4 a[C::NB], b[C::MB];
#pragma unroll
            for (int nb = 0; nb < C::NB; ++nb) {
                if constexpr (C::KN) a[nb] = op_kn<T, C>(ws, wn * C::WN + 16 * nb, s, lane);
                else a[nb] = op_krows<T, C>(ws, wn * C::WN + 16 * nb, s, lane);
            }
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) b[mb] = op_krows<T, C>(xs, wm * C::WM + 16 * mb, s, lane);
#pragma unroll
            for (int nb = 0; nb < C::NB; ++nb)
#pragma unroll
                for (int mb = 0; mb < C::MB; ++mb) acc[nb][mb] = mma_chunk<T>(a[nb], b[mb], acc[nb][mb]);
        }
    }
}

// Four channels of one output row: (+ bias) and one rounding to T.
template <typename T> __device__ __forceinline__ void store4(T* dst, f32x4 v, const float (&bv)[4]) {
    if constexpr (sizeof(T) == 2) {
        u32x2 out;
        out[0] = Pk<T>::cvt(v[0] + bv[0], v[1] + bv[1]);
        out[1] = Pk<T>::cvt(v[2] + bv[2], v[3] + bv[3]);
        *reinterpret_cast<u32x2*>(dst) = out;
    } else {
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0] + bv[0], v[1] + bv[1], v[2] + bv[2], v[3] + bv[3]};
    }
}

template <typename T, typename C, bool BIAS>
__global__ __launch_bounds__(C::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void proj_gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) T lds[C::STAGES * (C::XS + C::WS)];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int tm, tn;
    gemm_tile(gemm_logical_block(), p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;

    f32x4 acc[C::NB][C::MB];
    gemm_mainloop<T, C>(p, lds, m0, n0, wave, lane, acc);

    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    T* y = static_cast<T*>(p.y);
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
            if (m < p.M) store4(y + (int64_t)m * p.ldy + n, acc[nb][mb], bv);
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
// launch takes ceil(tiles / CUs) rounds, and a round costs about BN + 32
// (work proportional to the width plus a fixed per-tile part; this model ranks
// the measured times of every candidate correctly at the SANA shapes).
inline int pick_bn(int M, int N, const int* cands, int n_cands) {
    const int cus = device_cu_count();
    int best = cands[0];
    long long best_cost = -1;
    for (int i = 0; i < n_cands; ++i) {
        const int bn = cands[i];
        const long long tiles = (long long)((M + 255) / 256) * ((N + bn - 1) / bn);
        const long long cost = (tiles + cus - 1) / cus * (bn + 32);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = bn;
        }
    }
    return best;
}

template <typename T, bool KN>
int launch_gemm(const GemmParams& p, bool bias, hipStream_t st) {
    // 16-bit weights in [N][K]: five widths; fp32 or WeightT: 256 and 128.
    if constexpr (sizeof(T) == 2 && !KN) {
        static const int cands[] = {224, 256, 192, 160, 128};
        switch (pick_bn(p.M, p.N, cands, 5)) {
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
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool b = bias != nullptr;
    if (dtype == KF_BF16) return launch_gemm_layout<bf16>(p, weight_layout, b, st);
    if (dtype == KF_F16) return launch_gemm_layout<f16>(p, weight_layout, b, st);
    return launch_gemm_layout<float>(p, weight_layout, b, st);
}
