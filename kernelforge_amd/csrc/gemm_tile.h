// MFMA GEMM tile machinery for gfx950, shared by the projection GEMM
// (proj_gemm.hip) and the fused LiteLA projection kernels (litela_fused.hip).
//
// The product these pieces compute:
//   y[m][n] = sum_k x[m][k] * W[n][k]
// with fp32 accumulation on the MFMA pipe; the kernels that use them round
// and store (or further contract) the accumulators in their own epilogues.
//
// The weight comes in either layout: [N][K] as torch.nn.Linear stores it
// (K contiguous, the MFMA operand order, read with ds_read_b128), or the
// reference's prepacked WeightT [K][N] (N contiguous, read column-wise: the
// transposing ds_read_b64_tr_b16 for 16-bit types, 4-byte reads for fp32).
//
// Workgroup: WAVES wavefronts, a BM x BN output tile, K streamed through LDS
// in stages of 64- or 128-byte rows by global_load_lds copies (no register
// staging), STAGES buffers deep.  Copies of whole stages of in-range rows take
// a scalar base per instruction and one per-lane offset per wavefront, so
// they cost no vector instructions; others compute a clamped address per lane.
// Each wavefront owns a WM x WN sub-tile.  A lane reads one 16-byte chunk per
// operand block and 64-byte K step: one v_mfma_f32_16x16x32 for bf16/f16,
// four v_mfma_f32_16x16x4f32 for fp32, whose K slices are taken as {4g + t}
// so that the same chunk read serves all four.
// The MFMA computes the transposed product (A = weight rows, B = activation
// rows), so a lane ends with 4 consecutive output channels of one token.
//
// Workgroups are renumbered so that each XCD (the hardware sends workgroup i
// to XCD i % 8) receives a contiguous range of logical blocks; the kernels map
// consecutive logical blocks to tiles that share operand panels in that
// XCD's L2.
#pragma once

#include "fa_common.h"

namespace kf {
namespace {

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

// Copy tile rows 0..R-1, K columns k0..k0+BK-1 (zero past K) of a
// K-contiguous matrix into a [R][BK] tile; tile row r comes from global row
// rowf(r) (callers clamp rows past the valid range onto a valid row: those
// rows only feed outputs that are discarded).  Instruction i covers tile rows
// RPC i .. RPC i + RPC-1; wavefront w issues i = w, w + WAVES, ...
template <typename T, typename C, int R, typename RowFn>
__device__ __forceinline__ void copy_krows(T* tile, const T* g, int64_t ld, RowFn rowf, int k0, int K, int wave,
                                           int lane) {
    constexpr int NI = R / C::RPC;
#pragma unroll
    for (int j = 0; j < (NI + C::WAVES - 1) / C::WAVES; ++j) {
        const int i = wave + C::WAVES * j;
        if (NI % C::WAVES != 0 && i >= NI) break;
        const int r = C::RPC * i + lane / C::CPR;
        const int c = (lane % C::CPR) ^ kswz<C::CPR>(r);
        const int64_t gr = rowf(r);
        const int kk = k0 + C::EPC * c;
        const void* src = kk < K ? static_cast<const void*>(g + gr * ld + kk) : static_cast<const void*>(g_zero16);
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

// Workgroup barrier once this wavefront's LDS operations have completed;
// its outstanding LDS copies (vmcnt) are not waited for.
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
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

// Operands of one workgroup's mainloop: activation rows x_row0 + r (clamped
// below x_rows_end) of x[.][ldx]; weight rows wrow(r) of a dense [.][K]
// weight (NK), or columns n0.. of a dense [K][N] WeightT (KN).
template <typename T> struct GemmSrc {
    const T* x;
    int64_t ldx;
    int64_t x_row0, x_rows_end;
    const T* w;
    int K;
    int n0, N;  // KN only
    // NK only: wrow(RPC b + j) == wrow(RPC b) + j for every block b of RPC
    // tile rows (j < RPC), so each copy instruction reads RPC consecutive
    // weight rows and can take a scalar base.
    bool w_rows_linear = false;
};

// Lane byte offset of the scalar-base copies of a K-contiguous [R][BK] tile
// from rows of stride ld: wavefront w issues instructions i = w + WAVES j,
// whose lanes cover tile row RPC i + lane/CPR at logical chunk
// (lane%CPR) ^ kswz(row).  WAVES * RPC is a multiple of 16, so that swizzle
// is the same for every instruction of a wavefront and one offset serves all.
template <typename T, typename C>
__device__ __forceinline__ uint32_t krows_lane_off(int64_t ld, int wave, int lane) {
    static_assert((C::WAVES * C::RPC) % 16 == 0, "one swizzle per wavefront");
    const int r = C::RPC * wave + lane / C::CPR;
    const int c = (lane % C::CPR) ^ kswz<C::CPR>(r);
    return (uint32_t)((int64_t)(lane / C::CPR) * ld * (int64_t)sizeof(T) + c * 16);
}

// Whole-stage copy (K columns k0..k0+BK-1, all < K) of tile rows 0..R-1 whose
// instruction i reads the RPC consecutive rows starting at rowbase(RPC i)
// (stride ld): a scalar base per instruction plus the wavefront's lane
// offset (krows_lane_off); tile_lds is the tile's LDS byte address and wave
// a wavefront-uniform value.
template <typename T, typename C, int R, typename RowBase>
__device__ __forceinline__ void copy_krows_sbase(uint32_t tile_lds, RowBase rowbase, uint32_t voff, int k0,
                                                 int wave) {
    constexpr int NI = R / C::RPC;
#pragma unroll
    for (int j = 0; j < (NI + C::WAVES - 1) / C::WAVES; ++j) {
        const int i = wave + C::WAVES * j;
        if (NI % C::WAVES != 0 && i >= NI) break;
        lds_copy16_sbase(rowbase(C::RPC * i) + k0, voff, tile_lds + (uint32_t)(C::RPC * i * C::BK * (int)sizeof(T)));
    }
}

// Accumulate one wavefront's WM x WN sub-tile over the whole K range.
// acc[nb][mb][i] = y[m = wm*WM + 16 mb + l%16][n = wn*WN + 16 nb + 4(l/16) + i].
//
// Loop schedule: the K range is a sequence of MFMA steps (STEPS per stage),
// and the operand chunks of step q+1 are read from LDS while step q's MFMAs
// run, across stage boundaries too.  Before the first read of stage t each
// wavefront waits for its own copies of stage t and meets the others at one
// barrier; after it stage t-1's buffer is free (every read of it has
// completed), so the copies of stage t + STAGES - 1 go there.  The two
// operand sets alternate between even and odd steps.  A second operand set
// is live throughout, so sub-tiles of more than 28 16x16 blocks (BN = 256,
// which then spills) read each step's operands just before its MFMAs.
template <typename T, typename C, typename WRow>
__device__ __forceinline__ void gemm_mainloop(const GemmSrc<T>& src, WRow wrow, T* lds, int wave, int lane,
                                              f32x4 (&acc)[C::NB][C::MB]) {
    constexpr int PER = C::XI + C::WI;
    constexpr bool kPrefetch = C::NB * C::MB <= 28;
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int KT = (src.K + C::BK - 1) / C::BK;
    const int64_t xr0 = src.x_row0, xlast = src.x_rows_end - 1;
    auto xrow = [xr0, xlast](int r) { return min(xr0 + r, xlast); };

    // Scalar-base copies of whole stages when the tile's activation rows are
    // all in range, its weight rows are linear in 8-row blocks and a lane's
    // offset within an instruction's rows fits the 32-bit offset operand.
    const int swave = __builtin_amdgcn_readfirstlane(wave);
    constexpr int64_t kMaxRowSpan = (int64_t)1 << 31;
    const bool fast = !C::KN && src.w_rows_linear && xr0 + C::BM <= src.x_rows_end &&
                      src.ldx * C::RPC * (int64_t)sizeof(T) < kMaxRowSpan &&
                      (int64_t)src.K * C::RPC * (int64_t)sizeof(T) < kMaxRowSpan;
    const uint32_t x_voff = krows_lane_off<T, C>(src.ldx, swave, lane);
    const uint32_t w_voff = krows_lane_off<T, C>(src.K, swave, lane);
    const uint32_t lds0 = lds_addr(lds);
    const T* xg = src.x + xr0 * src.ldx;
    auto xbase = [xg, &src](int r) { return xg + (int64_t)r * src.ldx; };
    auto wbase = [&src, &wrow](int r) { return src.w + wrow(r) * (int64_t)src.K; };

    auto issue = [&](int kt) {
        const int buf = kt % C::STAGES;
        if (fast && (kt + 1) * C::BK <= src.K) {
            const uint32_t xl = lds0 + (uint32_t)(buf * (C::XS + C::WS) * (int)sizeof(T));
            copy_krows_sbase<T, C, C::BM>(xl, xbase, x_voff, kt * C::BK, swave);
            copy_krows_sbase<T, C, C::BN>(xl + C::XS * (uint32_t)sizeof(T), wbase, w_voff, kt * C::BK, swave);
            return;
        }
        T* xs = lds + buf * (C::XS + C::WS);
        T* ws = xs + C::XS;
        copy_krows<T, C, C::BM>(xs, src.x, src.ldx, xrow, kt * C::BK, src.K, wave, lane);
        if constexpr (C::KN) copy_kn<T, C>(ws, src.w, src.N, src.n0, kt * C::BK, src.K, wave, lane);
        else copy_krows<T, C, C::BN>(ws, src.w, src.K, wrow, kt * C::BK, src.K, wave, lane);
    };
    auto read_ops = [&](int kt, int s, u32x4 (&a)[C::NB], u32x4 (&b)[C::MB]) {
        const T* xs = lds + (kt % C::STAGES) * (C::XS + C::WS);
        const T* ws = xs + C::XS;
#pragma unroll
        for (int nb = 0; nb < C::NB; ++nb) {
            if constexpr (C::KN) a[nb] = op_kn<T, C>(ws, wn * C::WN + 16 * nb, s, lane);
            else a[nb] = op_krows<T, C>(ws, wn * C::WN + 16 * nb, s, lane);
        }
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) b[mb] = op_krows<T, C>(xs, wm * C::WM + 16 * mb, s, lane);
    };
    auto mma_step = [&](const u32x4 (&a)[C::NB], const u32x4 (&b)[C::MB]) {
#pragma unroll
        for (int nb = 0; nb < C::NB; ++nb)
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) acc[nb][mb] = mma_chunk<T>(a[nb], b[mb], acc[nb][mb]);
    };
    // Stage t's copies have landed for every wavefront; stage t-1's buffer
    // takes stage t + STAGES - 1.
    auto enter_stage = [&](int t) {
        wait_stage<C::STAGES, PER>(min(C::STAGES - 2, KT - 1 - t));
        barrier_lds();
        if (t + C::STAGES - 1 < KT) issue(t + C::STAGES - 1);
    };

#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < C::STAGES - 1; ++s)
        if (s < KT) issue(s);

    if constexpr (kPrefetch) {
        const int TS = KT * C::STEPS;
        // Read step q's operands into (a, b), entering its stage first when q
        // is the stage's first step.
        static_assert(C::STEPS == 1 || C::STEPS == 2, "steps per stage");
        auto prepare = [&](int q, u32x4 (&a)[C::NB], u32x4 (&b)[C::MB]) {
            const int t = C::STEPS == 1 ? q : q >> 1, s = C::STEPS == 1 ? 0 : q & 1;
            if (s == 0) enter_stage(t);
            read_ops(t, s, a, b);
        };
        u32x4 a0[C::NB], b0[C::MB], a1[C::NB], b1[C::MB];
        prepare(0, a0, b0);
        for (int q = 0; q < TS; q += 2) {
            if (q + 1 < TS) prepare(q + 1, a1, b1);
            mma_step(a0, b0);
            if (q + 1 < TS) {
                if (q + 2 < TS) prepare(q + 2, a0, b0);
                mma_step(a1, b1);
            }
        }
    } else {
        for (int kt = 0; kt < KT; ++kt) {
            enter_stage(kt);
#pragma unroll
            for (int s = 0; s < C::STEPS; ++s) {
                u32x4 a[C::NB], b[C::MB];
                read_ops(kt, s, a, b);
                mma_step(a, b);
            }
        }
    }
}

// Four channels of one output row: (+ bias) and one rounding to T.  Without
// a bias nothing is added: x + 0 is not folded under IEEE signed zeros, and
// leaving it out keeps an all-(-0) sum at -0, as a plain product gives.
template <bool BIAS, typename T>
__device__ __forceinline__ void store4(T* dst, f32x4 v, const float (&bv)[4]) {
    if constexpr (BIAS) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += bv[i];
    }
    if constexpr (sizeof(T) == 2) {
        u32x2 out;
        out[0] = Pk<T>::cvt(v[0], v[1]);
        out[1] = Pk<T>::cvt(v[2], v[3]);
        *reinterpret_cast<u32x2*>(dst) = out;
    } else {
        *reinterpret_cast<f32x4*>(dst) = v;
    }
}

}  // namespace
}  // namespace kf
