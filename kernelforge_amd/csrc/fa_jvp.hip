// FlashAttention forward, fused forward+JVP, and JVP-from-LSE for gfx950.
//
// Semantics: dense softmax attention (flash_attention_jvp/original.py:6-30),
// its forward-mode derivative, and the single-pass online recurrence of
// flash_attention_jvp/flash-attention-jvp-derivation.md:388-558:
//   S = scale q k^T, tS = scale (tq k^T + q tk^T), E = exp(S - m),
//   l = a l + rowsum(E), U = a U + E v, r = a r + rowsum(E*tS),
//   G = a G + (E*tS) v + E tv;   O = U/l, tO = G/l - (r/l) O, LSE = m + log l.
// The JVP-from-LSE mode recomputes P = exp(S - LSE) (flash_attention_jvp/
// custom.py:88-118) and, unlike the reference, does not use the cached 16-bit
// O in tO = P tv + H v - rowsum(H) O: that term multiplies O's rounding error
// by rowsum(H), which exceeds the bf16 tolerance at D = 128.  It accumulates
// U = P v alongside (one more product) and normalises like the fused mode:
//   tO = (P tv + H v)/l - (rowsum(H)/l) (U/l),  l = rowsum(P) of the rounded P.
//
// Tiling.  A workgroup is 4 wavefronts x 32 query rows (128 rows) of one
// (batch, head); it scans the key axis in tiles of 64 keys.  Per tile each
// wavefront computes the transposed score block S^T = K Q^T with
// v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q held in registers), so lane
// l owns query row l%32 and 16 keys per 32-key block.  That makes every row
// statistic (max, l, r, the rescale factor) lane-local, and the score
// registers are already the B operand of the next product O^T += V^T E^T once
// the keys are enumerated in the order the accumulator holds them:
// k = 8*(j/4) + 4*(l/32) + j%4 for operand element j.  V^T is read from the
// row-major V tile with ds_read_b64_tr_b16 in that same key order.
//
// Memory.  K, V (and tK, tV) tiles stream HBM -> LDS with global_load_lds
// (16 B per lane, no VGPR staging), double buffered, rows XOR-swizzled in
// 16-byte chunks so both the row reads (ds_read_b128) and the transposing
// reads are free of bank conflicts.  Workgroups are renumbered so that all
// query tiles of one head run on one XCD and share its L2.
//
// The running max is only raised when a tile's max exceeds it by more than
// 2^8 (log2 units); E then stays <= 256 and O = U/l, LSE = m + log l remain
// exact because U, l, r, G all use the same reference.
#include <type_traits>

#include "kf_common.h"

namespace kf {
namespace {

enum FaMode { FA_FWD = 0, FA_FWD_JVP = 1, FA_JVP = 2 };

constexpr int kBQ = 128;   // query rows per workgroup
constexpr int kBK = 64;    // keys per tile
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;

// 256 bytes of zeros in global memory: the source of lanes whose chunk is
// outside the tensor (key rows >= Nk, head-dim padding).
__device__ __attribute__((aligned(16))) unsigned g_zero16[64];

struct FaParams {
    const void* q;
    const void* k;
    const void* v;
    const void* tq;
    const void* tk;
    const void* tv;
    void* o;      // output (FWD, FWD_JVP) or cached input (JVP)
    float* lse;   // output (FWD, FWD_JVP) or cached input (JVP)
    void* to;     // output (FWD_JVP, JVP)
    int B, Nq, Nk, Hq, Hkv, D, group, n_qtiles;
    float scale;       // natural units
    float scale_log2;  // scale * log2(e)
    int causal;
};

template <int CH> __device__ __forceinline__ int swz(int row) {
    return (2 * (row & 3) + ((row >> 2) & 1)) & (CH - 1);
}

// Async copy of one [kBK][DP] tile (keys k0.., one kv head) into LDS.
template <typename T, int DP>
__device__ __forceinline__ void load_tile(T* tile, const T* g, int64_t row_stride, int keys_valid,
                                          int D, int wave, int lane) {
    constexpr int CH = DP / 8;
    constexpr int RPI = 64 / CH;
    constexpr int NI = kBK / (RPI * kWaves);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row0 = (i * kWaves + wave) * RPI;
        const int row = row0 + lane / CH;
        const int chunk = (lane % CH) ^ swz<CH>(row);
        const void* src = (row < keys_valid && chunk * 8 < D)
                               ? static_cast<const void*>(g + row * row_stride + chunk * 8)
                               : static_cast<const void*>(g_zero16);
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void*)(tile + row0 * DP), 16, 0, 0);
    }
}

// 8 consecutive elements (one 16-byte chunk) of a tile row.
template <typename T, int DP>
__device__ __forceinline__ typename V<T>::x8 row_chunk(const T* tile, int row, int chunk) {
    return *reinterpret_cast<const typename V<T>::x8*>(
        tile + row * DP + ((chunk ^ swz<DP / 8>(row)) << 3));
}

// Address of element (row, d) with d % 4 == 0, for the transposing read.
template <typename T, int DP>
__device__ __forceinline__ const T* tr_addr(const T* tile, int row, int d) {
    return tile + row * DP + (((d >> 3) ^ swz<DP / 8>(row)) << 3) + (d & 7);
}

// A operand V^T[d][k] for K-step ks2 (keys 16*ks2..) of d-block db, keys in
// accumulator order.
template <typename T, int DP>
__device__ __forceinline__ typename V<T>::x8 vt_operand(const T* tile, int ks2, int db, int lane) {
    const int G = lane >> 4, j16 = lane & 15;
    const int row = 16 * ks2 + 4 * (G >> 1) + (j16 >> 2);
    const int d = 32 * db + 16 * (G & 1) + 4 * (j16 & 3);
    const typename V<T>::x4 lo = lds_read_tr(tr_addr<T, DP>(tile, row, d));
    const typename V<T>::x4 hi = lds_read_tr(tr_addr<T, DP>(tile, row + 8, d));
    typename V<T>::x8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r[j] = lo[j];
        r[j + 4] = hi[j];
    }
    return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T, int DP, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_kernel(const FaParams p) {
    constexpr bool JVP = MODE != FA_FWD;
    constexpr int NT = JVP ? 4 : 2;          // tiles per stage: K, V (, tK, tV)
    constexpr int KS = DP / 16;               // K-steps over the head dim
    constexpr int DB = DP / 32;               // 32-wide d blocks of the output
    __shared__ __attribute__((aligned(16))) T smem[2][NT][kBK * DP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5;

    // XCD-aware renumbering: hardware sends block i to XCD i % 8; give each XCD
    // a contiguous range of logical blocks (consecutive query tiles of a head).
    const int nblk = gridDim.x, id = blockIdx.x;
    const int per = nblk >> 3, rem = nblk & 7, xcd = id & 7, slot = id >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    int qtile = logical % p.n_qtiles;
    const int rest = logical / p.n_qtiles;
    const int hq = rest % p.Hq, b = rest / p.Hq;
    if (p.causal) qtile = p.n_qtiles - 1 - qtile;  // longest scans first
    const int hk = hq / p.group;

    const int q0w = qtile * kBQ + wave * 32;     // first row of this wavefront
    const int qr = q0w + (lane & 31);            // this lane's query row
    const bool row_ok = qr < p.Nq;
    const int64_t q_row_stride = (int64_t)p.Hq * p.D;
    const int64_t kv_row_stride = (int64_t)p.Hkv * p.D;
    const int64_t q_off = ((int64_t)b * p.Nq + qr) * q_row_stride + (int64_t)hq * p.D;
    const int64_t kv_base = (int64_t)b * p.Nk * kv_row_stride + (int64_t)hk * p.D;
    const int diag = p.Nk - p.Nq;                // key j valid for row i iff j <= i + diag

    const bool has_tq = JVP && p.tq != nullptr;
    const bool has_tk = JVP && p.tk != nullptr;
    const bool has_tv = JVP && p.tv != nullptr;

    // Q (and tQ) as B operands: lane l holds row qr, d = 16*ks + 8*h + 0..7.
    typename V<T>::x8 qreg[KS], tqreg[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d = 16 * ks + 8 * h;
        const bool ok = row_ok && d < p.D;
        u32x4 z = {0u, 0u, 0u, 0u};
        u32x4 a = ok ? *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.q) + q_off + d) : z;
        qreg[ks] = __builtin_bit_cast(typename V<T>::x8, a);
        if constexpr (JVP) {
            u32x4 t = (ok && has_tq)
                          ? *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.tq) + q_off + d)
                          : z;
            tqreg[ks] = __builtin_bit_cast(typename V<T>::x8, t);
        }
    }

    float lse2 = 0.f;  // JVP mode: cached LSE in log2 units
    if constexpr (MODE == FA_JVP) {
        lse2 = row_ok ? p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr] * kLog2e : __builtin_inff();
    }

    // Key range of the workgroup.
    int key_stop = p.Nk;
    if (p.causal) key_stop = min(p.Nk, max(0, qtile * kBQ + kBQ + diag));
    const int ntiles = (key_stop + kBK - 1) / kBK;

    f32x16 u[DB], g[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            u[db][i] = 0.f;
            g[db][i] = 0.f;
        }
    // l_run / r_run sum the 16-bit E and H the products consume; l_lse sums
    // the fp32 E for the LSE output.
    float m_run = -__builtin_inff(), l_run = 0.f, r_run = 0.f, l_lse = 0.f;

    auto issue = [&](int tile_idx) {
        const int buf = tile_idx & 1;
        const int k0 = tile_idx * kBK;
        const int kv = p.Nk - k0;
        const int64_t off = kv_base + (int64_t)k0 * kv_row_stride;
        load_tile<T, DP>(smem[buf][0], static_cast<const T*>(p.k) + off, kv_row_stride, kv, p.D, wave, lane);
        load_tile<T, DP>(smem[buf][1], static_cast<const T*>(p.v) + off, kv_row_stride, kv, p.D, wave, lane);
        if constexpr (JVP) {
            if (has_tk)
                load_tile<T, DP>(smem[buf][2], static_cast<const T*>(p.tk) + off, kv_row_stride, kv, p.D, wave, lane);
            if (has_tv)
                load_tile<T, DP>(smem[buf][3], static_cast<const T*>(p.tv) + off, kv_row_stride, kv, p.D, wave, lane);
        }
    };

    if (ntiles > 0) issue(0);
    // The tile loop is instantiated twice: branch-free when every tangent is
    // present (the common case), and with per-tangent checks otherwise.
    auto scan = [&](auto all_tag) {
    constexpr bool ALL = decltype(all_tag)::value;
    const bool use_tq = ALL || has_tq, use_tk = ALL || has_tk, use_tv = ALL || has_tv;
    for (int it = 0; it < ntiles; ++it) {
        const int buf = it & 1;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // tile `it` resident; everyone is done with buffer buf^1
        if (it + 1 < ntiles) issue(it + 1);
        const T* Kt = smem[buf][0];
        const T* Vt = smem[buf][1];
        const T* tKt = smem[buf][2 % NT];
        const T* tVt = smem[buf][3 % NT];
        const int k0 = it * kBK;

        const bool need_mask = (k0 + kBK > p.Nk) || (p.causal && k0 + kBK - 1 > q0w + diag);
        const int klim = p.causal ? min(p.Nk - 1, qr + diag) : p.Nk - 1;

        // The tile is consumed in two 32-key blocks, each run from scores to
        // the P.V products before the next starts (halves the live registers).
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            // ---- scores S^T (and tS^T) ----
            f32x16 s, ts;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s[i] = 0.f;
                ts[i] = 0.f;
            }
            const int krow = 32 * sub + (lane & 31);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const typename V<T>::x8 ka = row_chunk<T, DP>(Kt, krow, 2 * ks + h);
                s = mfma32x32x16(ka, qreg[ks], s);
                if constexpr (JVP) {
                    if (use_tq) ts = mfma32x32x16(ka, tqreg[ks], ts);
                    if (use_tk) {
                        const typename V<T>::x8 tka = row_chunk<T, DP>(tKt, krow, 2 * ks + h);
                        ts = mfma32x32x16(tka, qreg[ks], ts);
                    }
                }
            }

            // ---- scale to log2 units; mask tiles crossing Nk or the diagonal ----
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float x = s[i] * p.scale_log2;
                if (need_mask) {
                    const int key = k0 + 32 * sub + 8 * (i >> 2) + 4 * h + (i & 3);
                    if (key > klim) x = -__builtin_inff();
                }
                s[i] = x;
            }

            // ---- probabilities: E (online, FWD/FWD_JVP) or P (from LSE) ----
            float ref;
            if constexpr (MODE == FA_JVP) {
                ref = lse2;
            } else {
                float mx = -__builtin_inff();
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const bool upd = mx > m_run + kRescaleThreshold;
                if (__any(upd)) {
                    // Rows that keep their reference use alpha = 1 (never
                    // -inf - -inf); a row leaving m = -inf gets alpha = 0 on
                    // its all-zero state.
                    const float m_new = upd ? mx : m_run;
                    const float alpha = upd ? fast_exp2(m_run - m_new) : 1.f;
                    l_run *= alpha;
                    l_lse *= alpha;
#pragma unroll
                    for (int db = 0; db < DB; ++db)
#pragma unroll
                        for (int i = 0; i < 16; ++i) u[db][i] *= alpha;
                    if constexpr (JVP) {
                        r_run *= alpha;
#pragma unroll
                        for (int db = 0; db < DB; ++db)
#pragma unroll
                            for (int i = 0; i < 16; ++i) g[db][i] *= alpha;
                    }
                    m_run = m_new;
                }
                ref = m_run == -__builtin_inff() ? 0.f : m_run;
            }

            // l and r accumulate the same 16-bit E and H values the products
            // consume, so O is an exact convex combination of the V rows and
            // tO = G - r O = sum_j H_j (v_j - O): the rounding of H_j is
            // multiplied by (v_j - O), not by v_j (no cancellation blow-up).
            typename V<T>::x8 eb[2], hb[2];
            float lsum = 0.f, rsum = 0.f, esum = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = fast_exp2(s[i] - ref);
                esum += e;
                const T e16 = (T)e;
                eb[i >> 3][i & 7] = e16;
                lsum += (float)e16;
                if constexpr (JVP) {
                    const T h16 = (T)(e * (ts[i] * p.scale));
                    hb[i >> 3][i & 7] = h16;
                    rsum += (float)h16;
                }
            }
            l_run += lsum;
            r_run += rsum;
            l_lse += esum;

            // ---- O^T += V^T E^T ; G^T += V^T H^T + tV^T E^T ----
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int ks2 = 2 * sub + kk;
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const typename V<T>::x8 va = vt_operand<T, DP>(Vt, ks2, db, lane);
                    u[db] = mfma32x32x16(va, eb[kk], u[db]);
                    if constexpr (JVP) {
                        g[db] = mfma32x32x16(va, hb[kk], g[db]);
                        if (use_tv) {
                            const typename V<T>::x8 tva = vt_operand<T, DP>(tVt, ks2, db, lane);
                            g[db] = mfma32x32x16(tva, eb[kk], g[db]);
                        }
                    }
                }
            }
        }
    }

    };
    if (!JVP || (has_tq && has_tk && has_tv))
        scan(std::true_type{});
    else
        scan(std::false_type{});

    // ---- epilogue ----
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float r_tot = r_run + __shfl_xor(r_run, 32, 64);
    const float l_lse_tot = l_lse + __shfl_xor(l_lse, 32, 64);
    T* orow = static_cast<T*>(p.o) + q_off;
    T* torow = static_cast<T*>(p.to) + q_off;
    {
        const bool empty = !(l_tot > 0.f);
        const float inv = empty ? 0.f : 1.f / l_tot;
        const float rl = r_tot * inv;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int ig = 0; ig < 4; ++ig) {
                const int d = 32 * db + 8 * ig + 4 * h;
                if (row_ok && d < p.D) {
                    typename V<T>::x4 ov, tv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float o = u[db][4 * ig + e] * inv;
                        ov[e] = (T)o;
                        if constexpr (JVP) tv[e] = (T)(g[db][4 * ig + e] * inv - rl * o);
                    }
                    if constexpr (MODE != FA_JVP) *reinterpret_cast<typename V<T>::x4*>(orow + d) = ov;
                    if constexpr (JVP) *reinterpret_cast<typename V<T>::x4*>(torow + d) = tv;
                }
            }
        if (MODE != FA_JVP && h == 0 && row_ok) {
            p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr] =
                empty ? __builtin_inff() : (m_run + log2f(l_lse_tot)) * kLn2;
        }
    }
}

template <typename T, int MODE>
int launch_mode(const FaParams& p, int dp, hipStream_t stream) {
    const int64_t blocks = (int64_t)p.n_qtiles * p.Hq * p.B;
    if (blocks > 0x7fffffff) {
        set_error("fa: grid too large");
        return KF_E_UNSUPPORTED;
    }
    const dim3 grid((unsigned)blocks), block(256);
    switch (dp) {
        case 32: hipLaunchKernelGGL((fa_kernel<T, 32, MODE>), grid, block, 0, stream, p); break;
        case 64: hipLaunchKernelGGL((fa_kernel<T, 64, MODE>), grid, block, 0, stream, p); break;
        case 128: hipLaunchKernelGGL((fa_kernel<T, 128, MODE>), grid, block, 0, stream, p); break;
        default: set_error("fa: head dim %d not supported by this build", p.D); return KF_E_UNSUPPORTED;
    }
    return check_launch("fa_kernel launch");
}

int fa_dispatch(int mode, FaParams p, int dtype, hipStream_t stream) {
    KF_REQUIRE(p.B >= 0 && p.Nq >= 0 && p.Nk >= 0 && p.Hq > 0 && p.Hkv > 0, KF_E_INVALID,
               "fa: bad shape");
    KF_REQUIRE(p.Hq % p.Hkv == 0, KF_E_INVALID, "fa: Hq %% Hkv != 0");
    KF_REQUIRE(p.D > 0 && p.D % 8 == 0 && p.D <= 256, KF_E_INVALID,
               "fa: head dim must be a positive multiple of 8 <= 256, got %d", p.D);
    KF_REQUIRE(p.scale > 0.f && p.scale < __builtin_inff(), KF_E_INVALID,
               "fa: scale must be finite and positive");
    KF_REQUIRE(dtype == KF_F16 || dtype == KF_BF16, KF_E_INVALID, "fa: dtype must be f16 or bf16");
    if (p.B == 0 || p.Nq == 0) return KF_OK;
    KF_REQUIRE(p.q && p.k && p.v && p.o && p.lse && (mode == FA_FWD || p.to), KF_E_INVALID,
               "fa: null pointer");
    KF_REQUIRE(p.D <= 128, KF_E_UNSUPPORTED, "fa: head dim %d > 128 is not supported by this build",
               p.D);
    const int dp = p.D <= 32 ? 32 : p.D <= 64 ? 64 : 128;
    p.group = p.Hq / p.Hkv;
    p.n_qtiles = (p.Nq + kBQ - 1) / kBQ;
    p.scale_log2 = p.scale * kLog2e;
    if (mode != FA_FWD && p.Nk == 0) {
        // No keys: O = 0 and tO = 0 by the empty-row convention; the kernel
        // handles it with zero tiles.
    }
    if (dtype == KF_BF16) {
        switch (mode) {
            case FA_FWD: return launch_mode<bf16, FA_FWD>(p, dp, stream);
            case FA_FWD_JVP: return launch_mode<bf16, FA_FWD_JVP>(p, dp, stream);
            default: return launch_mode<bf16, FA_JVP>(p, dp, stream);
        }
    }
    switch (mode) {
        case FA_FWD: return launch_mode<f16, FA_FWD>(p, dp, stream);
        case FA_FWD_JVP: return launch_mode<f16, FA_FWD_JVP>(p, dp, stream);
        default: return launch_mode<f16, FA_JVP>(p, dp, stream);
    }
}

FaParams make_params(const void* q, const void* k, const void* v, const void* tq, const void* tk,
                     const void* tv, void* o, float* lse, void* to, int64_t B, int64_t Nq,
                     int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D, float scale, int causal) {
    FaParams p{};
    p.q = q; p.k = k; p.v = v; p.tq = tq; p.tk = tk; p.tv = tv;
    p.o = o; p.lse = lse; p.to = to;
    p.B = (int)B; p.Nq = (int)Nq; p.Nk = (int)Nk; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.D = (int)D;
    p.scale = scale; p.causal = causal ? 1 : 0;
    return p;
}

bool dims_fit(int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D) {
    const int64_t lim = 0x3fffffff;
    return B <= lim && Nq <= lim && Nk <= lim && Hq <= lim && Hkv <= lim && D <= lim &&
           B >= 0 && Nq >= 0 && Nk >= 0;
}

}  // namespace
}  // namespace kf

extern "C" int kf_fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                         int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D,
                         float scale, int causal, int dtype, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(dims_fit(B, Nq, Nk, Hq, Hkv, D), KF_E_INVALID, "fa: shape out of range");
    return fa_dispatch(FA_FWD, make_params(q, k, v, nullptr, nullptr, nullptr, o, lse, nullptr, B,
                                           Nq, Nk, Hq, Hkv, D, scale, causal),
                       dtype, static_cast<hipStream_t>(stream));
}

extern "C" int kf_fa_jvp(const void* q, const void* k, const void* v, const void* tq,
                         const void* tk, const void* tv, const void* o, const float* lse, void* to,
                         int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D,
                         float scale, int causal, int dtype, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(dims_fit(B, Nq, Nk, Hq, Hkv, D), KF_E_INVALID, "fa: shape out of range");
    return fa_dispatch(FA_JVP, make_params(q, k, v, tq, tk, tv, const_cast<void*>(o),
                                           const_cast<float*>(lse), to, B, Nq, Nk, Hq, Hkv, D,
                                           scale, causal),
                       dtype, static_cast<hipStream_t>(stream));
}

extern "C" int kf_fa_fwd_jvp(const void* q, const void* k, const void* v, const void* tq,
                             const void* tk, const void* tv, void* o, float* lse, void* to,
                             int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D,
                             float scale, int causal, int dtype, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(dims_fit(B, Nq, Nk, Hq, Hkv, D), KF_E_INVALID, "fa: shape out of range");
    return fa_dispatch(FA_FWD_JVP, make_params(q, k, v, tq, tk, tv, o, lse, to, B, Nq, Nk, Hq,
                                               Hkv, D, scale, causal),
                       dtype, static_cast<hipStream_t>(stream));
}
