// FlashAttention backward (vector-Jacobian product) for gfx950.
//
// Semantics: the reverse-mode derivative of dense softmax attention
// (flash_attention_jvp/original.py:6-30) that the reference obtains from
// flash-attn's _flash_attn_backward (flash_attention_jvp/custom.py:252-267):
//   P = exp(scale q k^T - LSE),  Delta_i = sum_d dO_id O_id,
//   dP = dO v^T,  dS = P * (dP - Delta),
//   dQ = scale dS k,  dK = scale dS^T q,  dV = P^T dO,
// with dK and dV summed over the query heads that share a KV head (GQA/MQA).
// P is recomputed from the forward's natural-log LSE; rows with LSE = +inf
// (no valid key) get P = 0 and contribute nothing.
//
// Two launches, no atomics, deterministic:
//   1. dq kernel, one workgroup per (query tile, batch, query head), shaped
//      like the forward: lane l owns query row l%16 and computes S^T = K Q^T
//      and dP^T = V dO^T over K/V tiles streamed through LDS, then
//      dQ^T += K^T dS^T with K^T read by transposing LDS reads.  It also
//      writes Delta and LSE*log2(e) of its rows to the workspace.
//   2. dkdv kernel, one workgroup per (key tile, batch, KV head), lane l
//      owning key l%16 of each 16-key block; it streams the Q and dO tiles
//      (plus their LSE/Delta entries) of every query head of the group, in a
//      fixed order, computes S = Q K^T and dP = dO V^T with the key as the
//      output column, and accumulates dV^T += dO^T P and dK^T += Q^T dS with
//      dO^T and Q^T read by transposing LDS reads.  Up to D = 128 on grids
//      that fill the chip (causal: D = 64 and 128), each wavefront owns two
//      key blocks (four at D = 32; K in registers, V in LDS), so each
//      transposed operand feeds four (eight) MFMAs; otherwise one block,
//      with K and V in registers.
// Both products of the pair are v_mfma_f32_16x16x32 with the same operand
// enumeration as the forward: the score accumulators of two 16-row blocks
// are directly the B operand of the next product once packed to 16 bits.
#include "fa_common.h"

namespace kf {
namespace {

struct FaBwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const float* lse;
    const void* dout;
    void* dq;
    void* dk;
    void* dv;
    float* ws_lse2;   // [B][Hq][nq_pad]: LSE * log2(e), +inf for rows >= Nq
    float* ws_delta;  // [B][Hq][nq_pad]: Delta, 0 for rows >= Nq
    int B, Nq, Nk, Hq, Hkv, D, group;
    int n_qtiles;  // query tiles of dq_rows() rows (dq grid)
    int n_ktiles;  // key tiles of FaTile::BQ keys (one-block dkdv grid)
    int nq_pad;    // query rows padded to a multiple of FaTile::BQ
    float scale;
    float scale_log2;
    int causal;
};

// XCD-aware renumbering: the hardware sends block i to XCD i % 8; give each
// XCD a contiguous range of logical blocks (consecutive tiles of one head,
// which share K/V or Q/dO rows in that XCD's L2).
__device__ __forceinline__ int xcd_logical_block() {
    const int nblk = gridDim.x, id = blockIdx.x;
    const int per = nblk >> 3, rem = nblk & 7, xcd = id & 7, slot = id >> 3;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// Loads 8 consecutive elements of a row as an MFMA B operand (zero if !ok).
template <typename T>
__device__ __forceinline__ typename V<T>::x8 load_row8(const T* p, bool ok) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    return __builtin_bit_cast(typename V<T>::x8, ok ? *reinterpret_cast<const u32x4*>(p) : z);
}

// ---------------------------------------------------------------------------
// dQ (and the per-row Delta / LSE*log2e workspace).
// ---------------------------------------------------------------------------
// Row blocks of 16 query rows per wavefront: two up to D = 128 (a 256-row
// workgroup), so that every K row and K^T / V operand read from LDS feeds two
// MFMAs and each tile copy serves twice the rows; one at D = 256.
template <int DP> constexpr int dq_row_blocks() { return DP <= 128 ? 2 : 1; }
template <int DP> constexpr int dq_rows() { return FaTile<DP>::BQ * dq_row_blocks<DP>(); }

template <typename T, int DP>
__global__ __launch_bounds__(FaTile<DP>::THREADS)
__attribute__((amdgpu_waves_per_eu(FaTile<DP>::OCC, FaTile<DP>::OCC)))
void fa_bwd_dq_kernel(const FaBwdParams p) {
    constexpr int R = dq_row_blocks<DP>();
    constexpr int kBQ = dq_rows<DP>(), kBK = FaTile<DP>::BK;
    constexpr int DS = DP / 32, DB = DP / 16;
    typedef typename V<T>::x8 x8;
    // Double-buffered K and V tiles, one LDS variable per buffer so that the
    // copies into one buffer are not ordered against reads of the other.
    __shared__ __attribute__((aligned(16))) T kt0[kBK * DP];
    __shared__ __attribute__((aligned(16))) T kt1[kBK * DP];
    __shared__ __attribute__((aligned(16))) T vt0[kBK * DP];
    __shared__ __attribute__((aligned(16))) T vt1[kBK * DP];
    auto lds_tile = [&](auto bufc, auto vsc) -> T* {
        constexpr int buf = decltype(bufc)::value;
        if constexpr (decltype(vsc)::value)
            return buf == 0 ? vt0 : vt1;
        else
            return buf == 0 ? kt0 : kt1;
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4;

    const int logical = p.causal ? causal_tile_order(xcd_logical_block(), p.n_qtiles) : xcd_logical_block();
    int qtile = logical % p.n_qtiles;
    const int rest = logical / p.n_qtiles;
    const int hq = rest % p.Hq, b = rest / p.Hq;
    if (p.causal) qtile = p.n_qtiles - 1 - qtile;  // longest scans first
    const int hk = hq / p.group;

    const int q0w = qtile * kBQ + wave * 16 * R;  // first row of this wavefront
    const int64_t q_row_stride = (int64_t)p.Hq * p.D;
    const int64_t kv_row_stride = (int64_t)p.Hkv * p.D;
    const int64_t kv_base = (int64_t)b * p.Nk * kv_row_stride + (int64_t)hk * p.D;
    const int diag = p.Nk - p.Nq;
    const float c = p.scale_log2;

    // Per row block rb: this lane's row, Q and dO as B operands (d = 32*ds +
    // 8*grp + 0..7), Delta = dO . O and LSE*log2e.
    int qr[R], klim[R];
    bool row_ok[R];
    int64_t q_off[R];
    x8 qreg[R][DS], doreg[R][DS];
    float delta[R], nlse2[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        qr[rb] = q0w + 16 * rb + (lane & 15);
        row_ok[rb] = qr[rb] < p.Nq;
        q_off[rb] = ((int64_t)b * p.Nq + qr[rb]) * q_row_stride + (int64_t)hq * p.D;
        float dot = 0.f;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int d = 32 * ds + 8 * grp;
            const bool ok = row_ok[rb] && d < p.D;
            qreg[rb][ds] = load_row8(static_cast<const T*>(p.q) + q_off[rb] + d, ok);
            doreg[rb][ds] = load_row8(static_cast<const T*>(p.dout) + q_off[rb] + d, ok);
            const x8 ov = load_row8(static_cast<const T*>(p.o) + q_off[rb] + d, ok);
#pragma unroll
            for (int j = 0; j < 8; ++j) dot = fmaf((float)doreg[rb][ds][j], (float)ov[j], dot);
        }
        delta[rb] = row_sum4(dot);
        const float lse2 =
            row_ok[rb] ? p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr[rb]] * kLog2e : __builtin_inff();
        nlse2[rb] = -lse2;
        // The workspace holds nq_pad rows: every row the dK/dV kernel's
        // 64-row tiles read (rows >= Nq get LSE = +inf, Delta = 0).
        if (grp == 0 && qr[rb] < p.nq_pad) {
            const int64_t w = ((int64_t)b * p.Hq + hq) * p.nq_pad + qr[rb];
            p.ws_lse2[w] = lse2;
            p.ws_delta[w] = delta[rb];
        }
        klim[rb] = p.causal ? min(p.Nk - 1, qr[rb] + diag) : p.Nk - 1;
    }

    int key_stop = p.Nk;
    if (p.causal) key_stop = min(p.Nk, max(0, qtile * kBQ + kBQ + diag));
    const int ntiles = (key_stop + kBK - 1) / kBK;

    // Up to D = 128 the K/V tiles use the panel layout (see pswz); at D = 256
    // the row-swizzled layout of fa_common.h.
    constexpr bool kPanels = DP <= 128;
    const PanelLane pl(lane);
    const uint32_t voff = kPanels ? panel_lane_offset<T>(kv_row_stride, lane)
                          : full_tile_shortcut<DP>() ? full_tile_lane_offset<T, DP>(kv_row_stride, wave, lane)
                                                     : 0u;
    const bool dense_rows = p.D == DP;
    const T* const kbase = static_cast<const T*>(p.k) + kv_base;
    const T* const vbase = static_cast<const T*>(p.v) + kv_base;

    auto issue_side = [&](int tile, auto bufc, auto vsc) {
        const int k0 = tile * kBK;
        T* const dst = lds_tile(bufc, vsc);
        const T* const src = (decltype(vsc)::value ? vbase : kbase) + (int64_t)k0 * kv_row_stride;
        if constexpr (kPanels) {
            if (dense_rows && k0 + kBK <= p.Nk)
                load_panels_full<T, DP>(dst, src, kv_row_stride, voff, wave);
            else
                load_panels<T, DP>(dst, src, kv_row_stride, p.Nk - k0, p.D, wave, lane);
            return;
        }
        if constexpr (full_tile_shortcut<DP>()) {
            if (dense_rows && k0 + kBK <= p.Nk) {
                load_tile_full<T, DP>(dst, src, kv_row_stride, voff, wave);
                return;
            }
        }
        load_tile<T, DP>(dst, src, kv_row_stride, p.Nk - k0, p.D, wave, lane);
    };

    f32x4 dq[R][DB];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) dq[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Operand rings (slot st % NR holds step st), as in the forward kernel;
    // the fences are left out at D = 256, whose register budget is tighter.
    constexpr int PF = 2, NR = PF + 1, NSTEP = 2 * DS;
    constexpr bool kFence = DP <= 128;
    x8 kring[NR], vring[NR];

    auto step = [&](int t, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const std::integral_constant<int, buf ^ 1> nbuf;
        const int k0 = t * kBK;
        const bool masked = (k0 + kBK > p.Nk) || (p.causal && k0 + kBK - 1 > q0w + diag);
        const T* Kt = lds_tile(bufc, std::false_type{});
        const T* Vt = lds_tile(bufc, std::true_type{});
        wait_vmem();
        __syncthreads();  // tile t resident; every wavefront is done with tile t-1
        if (t + 1 < ntiles) {
            issue_side(t + 1, nbuf, std::false_type{});
            issue_side(t + 1, nbuf, std::true_type{});
        }
#pragma unroll
        for (int h = 0; h < FaTile<DP>::HALVES; ++h) {
            f32x4 s[R][2], dp[R][2];
            // K and V rows for step st = (key block i2, K-step ds), read PF
            // steps ahead of their MFMAs.
            auto kv_load = [&](int st) {
                if constexpr (kPanels) {
                    kring[st % NR] = panel_chunk(Kt, pl, 16 * (2 * h + st / DS), st % DS);
                    vring[st % NR] = panel_chunk(Vt, pl, 16 * (2 * h + st / DS), st % DS);
                } else {
                    const int krow = 16 * (2 * h + st / DS) + (lane & 15);
                    kring[st % NR] = row_chunk<T, DP>(Kt, krow, 4 * (st % DS) + grp);
                    vring[st % NR] = row_chunk<T, DP>(Vt, krow, 4 * (st % DS) + grp);
                }
            };
            auto kt_load = [&](int db) {
                if constexpr (kPanels)
                    kring[db % NR] = panel_vt_operand(Kt, pl, h, db);
                else
                    kring[db % NR] = vt_operand<T, DP>(Kt, h, db, lane);
            };
            // dP^T accumulates onto -Delta, so it ends as dP - Delta.
#pragma unroll
            for (int rb = 0; rb < R; ++rb)
#pragma unroll
                for (int i2 = 0; i2 < 2; ++i2) {
                    s[rb][i2] = f32x4{0.f, 0.f, 0.f, 0.f};
                    dp[rb][i2] = f32x4{-delta[rb], -delta[rb], -delta[rb], -delta[rb]};
                }
#pragma unroll
            for (int st = 0; st < PF && st < NSTEP; ++st) kv_load(st);
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                if (st + PF < NSTEP) kv_load(st + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const int i2 = st / DS, ds = st % DS;
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    s[rb][i2] = mfma16x16x32(kring[st % NR], qreg[rb][ds], s[rb][i2]);
                    dp[rb][i2] = mfma16x16x32(vring[st % NR], doreg[rb][ds], dp[rb][i2]);
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
            // First K^T operands of the dQ product, in flight during the
            // softmax arithmetic.
#pragma unroll
            for (int db = 0; db < PF && db < DB; ++db) kt_load(db);
            // dS = P (dP - Delta), packed to 16 bits as the B operand of
            // dQ^T += K^T dS^T (keys 4*grp+0..3 of blocks 2h, 2h+1).
            x8 sb[R];
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                if (masked) {
#pragma unroll
                    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (k0 + 16 * (2 * h + i2) + 4 * grp + i > klim[rb]) s[rb][i2][i] = -__builtin_inff();
                }
                u32x2 sw[2];
#pragma unroll
                for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float p0 = fast_exp2(fmaf(s[rb][i2][2 * j], c, nlse2[rb]));
                        const float p1 = fast_exp2(fmaf(s[rb][i2][2 * j + 1], c, nlse2[rb]));
                        sw[i2][j] = Pk<T>::cvt(p0 * dp[rb][i2][2 * j], p1 * dp[rb][i2][2 * j + 1]);
                    }
                sb[rb] = __builtin_bit_cast(x8, u32x4{sw[0][0], sw[0][1], sw[1][0], sw[1][1]});
            }
            // Issue priority over the SIMD's other wavefront for the product
            // phase, so that the MFMA pipe refills first (0.5% at B=2, H=16,
            // N=4096, D=128 on MI355X; likewise in the dK/dV kernel).
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                if (db + PF < DB) kt_load(db + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int rb = 0; rb < R; ++rb) dq[rb][db] = mfma16x16x32(kring[db % NR], sb[rb], dq[rb][db]);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    };
    if (ntiles > 0) {
        issue_side(0, std::integral_constant<int, 0>{}, std::false_type{});
        issue_side(0, std::integral_constant<int, 0>{}, std::true_type{});
    }
    for (int t = 0; t < ntiles; t += 2) {
        step(t, std::integral_constant<int, 0>{});
        if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
    }

    // dQ = scale * dS K; lane holds row qr, d = 16*db + 4*grp + 0..3.
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        T* const dqrow = static_cast<T*>(p.dq) + q_off[rb];
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 16 * db + 4 * grp;
            if (row_ok[rb] && d < p.D) {
                typename V<T>::x4 r;
#pragma unroll
                for (int e = 0; e < 4; ++e) r[e] = (T)(dq[rb][db][e] * p.scale);
                *reinterpret_cast<typename V<T>::x4*>(dqrow + d) = r;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dK, dV: one workgroup per FaTile::BQ keys of one KV head, 16 keys per
// wavefront, scanning query tiles of FaTile::BK rows of every query head of
// the group.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(FaTile<DP>::THREADS)
__attribute__((amdgpu_waves_per_eu(FaTile<DP>::OCC, FaTile<DP>::OCC)))
void fa_bwd_dkdv_kernel(const FaBwdParams p) {
    constexpr int kBKEYS = FaTile<DP>::BQ;  // keys per workgroup
    constexpr int kBR = FaTile<DP>::BK;     // query rows per tile
    constexpr int DS = DP / 32, DB = DP / 16;
    typedef typename V<T>::x8 x8;
    static_assert(FaTile<DP>::WAVES >= 2, "waves 0 and 1 copy the row statistics");
    static_assert(kBR <= 64, "one 64-lane copy holds a tile's row statistics");
    // Double-buffered Q and dO tiles and their rows' [LSE*log2e, Delta].
    __shared__ __attribute__((aligned(16))) T qt0[kBR * DP];
    __shared__ __attribute__((aligned(16))) T qt1[kBR * DP];
    __shared__ __attribute__((aligned(16))) T ot0[kBR * DP];
    __shared__ __attribute__((aligned(16))) T ot1[kBR * DP];
    __shared__ __attribute__((aligned(16))) float rs0[2][64];
    __shared__ __attribute__((aligned(16))) float rs1[2][64];
    auto lds_tile = [&](auto bufc, auto osc) -> T* {
        constexpr int buf = decltype(bufc)::value;
        if constexpr (decltype(osc)::value)
            return buf == 0 ? ot0 : ot1;
        else
            return buf == 0 ? qt0 : qt1;
    };
    auto lds_stats = [&](auto bufc, int i) -> float* {
        return decltype(bufc)::value == 0 ? rs0[i] : rs1[i];
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4;

    const int logical = xcd_logical_block();
    const int ktile = logical % p.n_ktiles;
    const int rest = logical / p.n_ktiles;
    const int hk = rest % p.Hkv, b = rest / p.Hkv;

    const int k0 = ktile * kBKEYS;             // first key of the workgroup
    const int k0w = k0 + wave * 16;            // first key of this wavefront
    const int kr = k0w + (lane & 15);          // this lane's key
    const bool key_ok = kr < p.Nk;
    const int64_t q_row_stride = (int64_t)p.Hq * p.D;
    const int64_t kv_row_stride = (int64_t)p.Hkv * p.D;
    const int64_t kv_off = ((int64_t)b * p.Nk + kr) * kv_row_stride + (int64_t)hk * p.D;
    const int diag = p.Nk - p.Nq;  // key j valid for query i iff j <= i + diag

    // K and V as B operands (lane: key kr, d = 32*ds + 8*grp + 0..7).
    x8 kreg[DS], vreg[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
        const int d = 32 * ds + 8 * grp;
        const bool ok = key_ok && d < p.D;
        kreg[ds] = load_row8(static_cast<const T*>(p.k) + kv_off + d, ok);
        vreg[ds] = load_row8(static_cast<const T*>(p.v) + kv_off + d, ok);
    }

    // Query tiles: causal masks skip the rows before the first one that sees
    // key k0; the same range repeats for each query head of the group.
    const int n_rt = (p.Nq + kBR - 1) / kBR;
    const int rt0 = p.causal ? min(n_rt, max(0, k0 - diag) / kBR) : 0;
    const int per_head = n_rt - rt0;
    const int ntiles = per_head * p.group;
    const float c = p.scale_log2;

    const uint32_t voff = full_tile_shortcut<DP>() ? full_tile_lane_offset<T, DP>(q_row_stride, wave, lane) : 0u;
    const bool dense_rows = p.D == DP;

    auto tile_head = [&](int u) { return u / per_head; };
    auto tile_row0 = [&](int u) { return (rt0 + u % per_head) * kBR; };

    auto issue = [&](int u, auto bufc) {
        const int hq = hk * p.group + tile_head(u);
        const int r0 = tile_row0(u);
        const int64_t off = ((int64_t)b * p.Nq + r0) * q_row_stride + (int64_t)hq * p.D;
        const T* const qsrc = static_cast<const T*>(p.q) + off;
        const T* const osrc = static_cast<const T*>(p.dout) + off;
        T* const qdst = lds_tile(bufc, std::false_type{});
        T* const odst = lds_tile(bufc, std::true_type{});
        bool done = false;
        if constexpr (full_tile_shortcut<DP>()) {
            if (dense_rows && r0 + kBR <= p.Nq) {
                load_tile_full<T, DP>(qdst, qsrc, q_row_stride, voff, wave);
                load_tile_full<T, DP>(odst, osrc, q_row_stride, voff, wave);
                done = true;
            }
        }
        if (!done) {
            load_tile<T, DP>(qdst, qsrc, q_row_stride, p.Nq - r0, p.D, wave, lane);
            load_tile<T, DP>(odst, osrc, q_row_stride, p.Nq - r0, p.D, wave, lane);
        }
        // Row statistics of the tile: rows r0 .. r0+kBR-1 lie below nq_pad.
        if (wave < 2 && (kBR == 64 || lane < kBR)) {
            const float* src = (wave == 0 ? p.ws_lse2 : p.ws_delta) +
                               ((int64_t)b * p.Hq + hq) * p.nq_pad + r0 + lane;
            lds_copy4(src, __builtin_amdgcn_readfirstlane(lds_addr(lds_stats(bufc, wave))));
        }
    };

    f32x4 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dk[db] = f32x4{0.f, 0.f, 0.f, 0.f};
        dv[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Operand rings, as in the dq kernel.
    constexpr int PF = 2, NR = PF + 1, NSTEP = 2 * DS;
    constexpr bool kFence = DP <= 128;
    x8 qring[NR], oring[NR];

    auto step = [&](int u, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const std::integral_constant<int, buf ^ 1> nbuf;
        const int r0 = tile_row0(u);
        // Some (row, key) pair of this wavefront is masked out.
        const bool masked = p.causal && k0w + 15 > r0 + diag;
        const T* Qt = lds_tile(bufc, std::false_type{});
        const T* Ot = lds_tile(bufc, std::true_type{});
        const float* lse2v = lds_stats(bufc, 0);
        const float* deltav = lds_stats(bufc, 1);
        wait_vmem();
        __syncthreads();  // tile u resident; every wavefront is done with tile u-1
        if (u + 1 < ntiles) issue(u + 1, nbuf);
#pragma unroll
        for (int h = 0; h < FaTile<DP>::HALVES; ++h) {
            // S and dP for rows 16*(2h+i2) + 4*grp + i of the tile, key kr.
            f32x4 s[2], dp[2];
            auto qo_load = [&](int st) {
                const int row = 16 * (2 * h + st / DS) + (lane & 15);
                qring[st % NR] = row_chunk<T, DP>(Qt, row, 4 * (st % DS) + grp);
                oring[st % NR] = row_chunk<T, DP>(Ot, row, 4 * (st % DS) + grp);
            };
            // dP accumulates onto -Delta of its rows, so it ends as dP - Delta.
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
                const f32x4 dl = *reinterpret_cast<const f32x4*>(deltav + 16 * (2 * h + i2) + 4 * grp);
                s[i2] = f32x4{0.f, 0.f, 0.f, 0.f};
                dp[i2] = -dl;
            }
#pragma unroll
            for (int st = 0; st < PF && st < NSTEP; ++st) qo_load(st);
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                if (st + PF < NSTEP) qo_load(st + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const int i2 = st / DS, ds = st % DS;
                s[i2] = mfma16x16x32(qring[st % NR], kreg[ds], s[i2]);
                dp[i2] = mfma16x16x32(oring[st % NR], vreg[ds], dp[i2]);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
            // First dO^T and Q^T operands of the dV / dK products.
            auto t_load = [&](int db) {
                oring[db % NR] = vt_operand<T, DP>(Ot, h, db, lane);
                qring[db % NR] = vt_operand<T, DP>(Qt, h, db, lane);
            };
#pragma unroll
            for (int db = 0; db < PF && db < DB; ++db) t_load(db);
            u32x2 pw[2], sw[2];
            // P and dS; the causal test runs only on tiles that cross the
            // diagonal (a uniform branch, so unmasked tiles pay nothing).
            auto probs = [&](auto mkc) {
#pragma unroll
                for (int i2 = 0; i2 < 2; ++i2) {
                    const int rl = 16 * (2 * h + i2) + 4 * grp;
                    const f32x4 l2 = *reinterpret_cast<const f32x4*>(lse2v + rl);
                    float pr[4], dsv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float e = fast_exp2(fmaf(s[i2][i], c, -l2[i]));
                        if constexpr (decltype(mkc)::value) {
                            if (kr > r0 + rl + i + diag) e = 0.f;
                        }
                        pr[i] = e;
                        dsv[i] = e * dp[i2][i];
                    }
                    pw[i2][0] = Pk<T>::cvt(pr[0], pr[1]);
                    pw[i2][1] = Pk<T>::cvt(pr[2], pr[3]);
                    sw[i2][0] = Pk<T>::cvt(dsv[0], dsv[1]);
                    sw[i2][1] = Pk<T>::cvt(dsv[2], dsv[3]);
                }
            };
            if (masked)
                probs(std::true_type{});
            else
                probs(std::false_type{});
            const x8 pb = __builtin_bit_cast(x8, u32x4{pw[0][0], pw[0][1], pw[1][0], pw[1][1]});
            const x8 sb = __builtin_bit_cast(x8, u32x4{sw[0][0], sw[0][1], sw[1][0], sw[1][1]});
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                if (db + PF < DB) t_load(db + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                dv[db] = mfma16x16x32(oring[db % NR], pb, dv[db]);
                dk[db] = mfma16x16x32(qring[db % NR], sb, dk[db]);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    };
    if (ntiles > 0) issue(0, std::integral_constant<int, 0>{});
    for (int u = 0; u < ntiles; u += 2) {
        step(u, std::integral_constant<int, 0>{});
        if (u + 1 < ntiles) step(u + 1, std::integral_constant<int, 1>{});
    }

    // dK = scale * dS^T Q, dV = P^T dO; lane holds key kr, d = 16*db + 4*grp + 0..3.
    T* const dkrow = static_cast<T*>(p.dk) + kv_off;
    T* const dvrow = static_cast<T*>(p.dv) + kv_off;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const int d = 16 * db + 4 * grp;
        if (key_ok && d < p.D) {
            typename V<T>::x4 rk, rv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                rk[e] = (T)(dk[db][e] * p.scale);
                rv[e] = (T)dv[db][e];
            }
            *reinterpret_cast<typename V<T>::x4*>(dkrow + d) = rk;
            *reinterpret_cast<typename V<T>::x4*>(dvrow + d) = rv;
        }
    }
}

// ---------------------------------------------------------------------------
// dK, dV with KB 16-key blocks per wavefront (up to D = 128; KB = 2, and 4
// at D = 32): one workgroup per 16 * KB * WAVES keys of one KV head.  The
// one-block kernel above is bound by its LDS reads: every wavefront reads the
// whole Q^T and dO^T tile through transposing reads to feed two MFMAs per
// operand.  Here each such operand feeds 2 KB (dV and dK of every key
// block).  The registers hold the dK and dV accumulators of all blocks and
// the K operands of the wavefront's keys; V of the workgroup's keys sits in
// LDS and each block reads its V operands once per 32-row half, and the
// blocks' S and dP are computed one after the other so that one block's
// score accumulators are live at a time.
// Its LDS tiles use the panel layout above.
// Per key the products accumulate in the same order as in the one-block
// kernel.
// ---------------------------------------------------------------------------
// 16-key blocks per wavefront: four at D = 32 (7% faster than two at B=2,
// H=16, N=4096-8192 on MI355X), two at D = 64 (three fit the registers, but
// 384-key workgroups leave a partial round and a partial tile: 566 against
// 474 us at N=4096) and at D = 128.
template <int DP> constexpr int dkdv_wide_blocks() { return DP <= 32 ? 4 : 2; }
template <int DP> constexpr int dkdv_wide_keys() { return 16 * FaTile<DP>::WAVES * dkdv_wide_blocks<DP>(); }

template <typename T, int DP>
__global__ __launch_bounds__(FaTile<DP>::THREADS)
__attribute__((amdgpu_waves_per_eu(FaTile<DP>::OCC, FaTile<DP>::OCC)))
void fa_bwd_dkdv_wide_kernel(const FaBwdParams p) {
    static_assert(DP <= 128, "several key blocks per wavefront fit the registers up to D = 128");
    constexpr int kBKEYS = dkdv_wide_keys<DP>();  // keys per workgroup
    constexpr int kBR = FaTile<DP>::BK;           // query rows per tile
    constexpr int KB = dkdv_wide_blocks<DP>();    // 16-key blocks per wavefront
    constexpr int DS = DP / 32, DB = DP / 16;
    typedef typename V<T>::x8 x8;
    constexpr int KW = 16 * KB;                   // keys per wavefront
    static_assert(kBKEYS % kBR == 0, "V is copied in whole tiles");
    static_assert(kBR == 64, "one 64-lane copy holds a tile's row statistics");
    __shared__ __attribute__((aligned(16))) T qt0[kBR * DP];
    __shared__ __attribute__((aligned(16))) T qt1[kBR * DP];
    __shared__ __attribute__((aligned(16))) T ot0[kBR * DP];
    __shared__ __attribute__((aligned(16))) T ot1[kBR * DP];
    __shared__ __attribute__((aligned(16))) T vt[kBKEYS * DP];  // V rows of the workgroup's keys
    __shared__ __attribute__((aligned(16))) float rs0[2][64];
    __shared__ __attribute__((aligned(16))) float rs1[2][64];
    auto lds_tile = [&](auto bufc, auto osc) -> T* {
        constexpr int buf = decltype(bufc)::value;
        if constexpr (decltype(osc)::value)
            return buf == 0 ? ot0 : ot1;
        else
            return buf == 0 ? qt0 : qt1;
    };
    auto lds_stats = [&](auto bufc, int i) -> float* {
        return decltype(bufc)::value == 0 ? rs0[i] : rs1[i];
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4;

    const int n_kt = (p.Nk + kBKEYS - 1) / kBKEYS;
    const int logical = p.causal ? causal_tile_order(xcd_logical_block(), n_kt) : xcd_logical_block();
    const int ktile = logical % n_kt;
    const int rest = logical / n_kt;
    const int hk = rest % p.Hkv, b = rest / p.Hkv;

    const int k0 = ktile * kBKEYS;  // first key of the workgroup
    const int k0w = k0 + wave * KW;  // first key of this wavefront
    const int64_t q_row_stride = (int64_t)p.Hq * p.D;
    const int64_t kv_row_stride = (int64_t)p.Hkv * p.D;
    const int64_t kv_base = (int64_t)b * p.Nk * kv_row_stride + (int64_t)hk * p.D;
    const int diag = p.Nk - p.Nq;  // key j valid for query i iff j <= i + diag

    // V rows k0 .. k0 + kBKEYS - 1 into LDS (zeros past Nk), as kBKEYS/64
    // panel-layout tiles; the first barrier of the scan waits for them.
#pragma unroll
    for (int i = 0; i < kBKEYS / kBR; ++i)
        load_panels<T, DP>(vt + i * kBR * DP,
                           static_cast<const T*>(p.v) + kv_base + (int64_t)(k0 + i * kBR) * kv_row_stride,
                           kv_row_stride, p.Nk - k0 - i * kBR, p.D, wave, lane);

    // K as B operands (lane: key k0w + 16*kb + l%16, d = 32*ds + 8*grp + 0..7).
    x8 kreg[KB][DS];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const int kr = k0w + 16 * kb + (lane & 15);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int d = 32 * ds + 8 * grp;
            kreg[kb][ds] = load_row8(static_cast<const T*>(p.k) + kv_base + (int64_t)kr * kv_row_stride + d,
                                     kr < p.Nk && d < p.D);
        }
    }

    const int n_rt = (p.Nq + kBR - 1) / kBR;
    const int rt0 = p.causal ? min(n_rt, max(0, k0 - diag) / kBR) : 0;
    const int per_head = n_rt - rt0;
    const int ntiles = per_head * p.group;
    const float c = p.scale_log2;

    const uint32_t voff = panel_lane_offset<T>(q_row_stride, lane);
    const bool dense_rows = p.D == DP;

    auto tile_head = [&](int u) { return u / per_head; };
    auto tile_row0 = [&](int u) { return (rt0 + u % per_head) * kBR; };

    auto issue = [&](int u, auto bufc) {
        const int hq = hk * p.group + tile_head(u);
        const int r0 = tile_row0(u);
        const int64_t off = ((int64_t)b * p.Nq + r0) * q_row_stride + (int64_t)hq * p.D;
        const T* const qsrc = static_cast<const T*>(p.q) + off;
        const T* const osrc = static_cast<const T*>(p.dout) + off;
        T* const qdst = lds_tile(bufc, std::false_type{});
        T* const odst = lds_tile(bufc, std::true_type{});
        if (dense_rows && r0 + kBR <= p.Nq) {
            load_panels_full<T, DP>(qdst, qsrc, q_row_stride, voff, wave);
            load_panels_full<T, DP>(odst, osrc, q_row_stride, voff, wave);
        } else {
            load_panels<T, DP>(qdst, qsrc, q_row_stride, p.Nq - r0, p.D, wave, lane);
            load_panels<T, DP>(odst, osrc, q_row_stride, p.Nq - r0, p.D, wave, lane);
        }
        if (wave < 2) {  // 64 rows: one dword per lane
            const float* src = (wave == 0 ? p.ws_lse2 : p.ws_delta) + ((int64_t)b * p.Hq + hq) * p.nq_pad + r0;
            lds_copy4_sbase(src, 4u * lane, __builtin_amdgcn_readfirstlane(lds_addr(lds_stats(bufc, wave))));
        }
    };

    f32x4 dk[KB][DB], dv[KB][DB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            dk[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
            dv[kb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    const PanelLane pl(lane);
    // Operand rings: two deep for the Q/dO chunks of the S/dP steps (one read
    // ahead; the key blocks' V chunks are read at their own step, behind the
    // S products, which keeps the kernel within 256 registers at D = 128),
    // three for the transposed operands (two ahead); the same registers serve
    // both.
    constexpr int PF = 2, NR = PF + 1;
    constexpr bool kFence = true;
    x8 qring[NR], oring[NR];

    auto step = [&](int u, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const std::integral_constant<int, buf ^ 1> nbuf;
        const int r0 = tile_row0(u);
        const T* Qt = lds_tile(bufc, std::false_type{});
        const T* Ot = lds_tile(bufc, std::true_type{});
        const float* lse2v = lds_stats(bufc, 0);
        const float* deltav = lds_stats(bufc, 1);
        wait_vmem();
        __syncthreads();  // tile u (and V) resident; every wavefront is done with tile u-1
        if (u + 1 < ntiles) issue(u + 1, nbuf);
        // Causal: a wavefront none of whose keys any row of the tile sees
        // adds nothing (P = 0) and skips the tile.
        if (p.causal && k0w > r0 + kBR - 1 + diag) return;
#pragma unroll
        for (int h = 0; h < FaTile<DP>::HALVES; ++h) {
            u32x2 pw[KB][2], sw[KB][2];
            // One 16-row block of the half at a time: each Q/dO chunk is read
            // once and feeds the S/dP products of every key block.
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
                const int row16 = 16 * (2 * h + i2);
                const f32x4 dl = *reinterpret_cast<const f32x4*>(deltav + row16 + 4 * grp);
                f32x4 s[KB], dp[KB];
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
                    s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                    dp[kb] = -dl;
                }
                x8 vcur[KB];
                auto qo_load = [&](int ds) {
                    qring[ds % 2] = panel_chunk(Qt, pl, row16, ds);
                    oring[ds % 2] = panel_chunk(Ot, pl, row16, ds);
                };
                auto v_load = [&](int ds) {
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
                        const T* const vtile = vt + ((wave * KW + 16 * kb) / kBR) * kBR * DP;
                        vcur[kb] = panel_chunk(vtile, pl, (wave * KW + 16 * kb) % kBR, ds);
                    }
                };
                qo_load(0);
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    v_load(ds);
                    if (ds + 1 < DS) qo_load(ds + 1);
                    if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb)
                        s[kb] = mfma16x16x32(qring[ds % 2], kreg[kb][ds], s[kb]);
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb)
                        dp[kb] = mfma16x16x32(oring[ds % 2], vcur[kb], dp[kb]);
                    if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                }
                const int rl = row16 + 4 * grp;
                const f32x4 l2 = *reinterpret_cast<const f32x4*>(lse2v + rl);
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
                    const int kr = k0w + 16 * kb + (lane & 15);
                    const bool masked = p.causal && k0w + 16 * kb + 15 > r0 + diag;
                    auto probs = [&](auto mkc) {
                        float pr[4], dsv[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float e = fast_exp2(fmaf(s[kb][i], c, -l2[i]));
                            if constexpr (decltype(mkc)::value) {
                                if (kr > r0 + rl + i + diag) e = 0.f;
                            }
                            pr[i] = e;
                            dsv[i] = e * dp[kb][i];
                        }
                        pw[kb][i2][0] = Pk<T>::cvt(pr[0], pr[1]);
                        pw[kb][i2][1] = Pk<T>::cvt(pr[2], pr[3]);
                        sw[kb][i2][0] = Pk<T>::cvt(dsv[0], dsv[1]);
                        sw[kb][i2][1] = Pk<T>::cvt(dsv[2], dsv[3]);
                    };
                    if (masked)
                        probs(std::true_type{});
                    else
                        probs(std::false_type{});
                }
            }
            x8 pb[KB], sb[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                pb[kb] = __builtin_bit_cast(x8, u32x4{pw[kb][0][0], pw[kb][0][1], pw[kb][1][0], pw[kb][1][1]});
                sb[kb] = __builtin_bit_cast(x8, u32x4{sw[kb][0][0], sw[kb][0][1], sw[kb][1][0], sw[kb][1][1]});
            }
            // dV^T += dO^T P and dK^T += Q^T dS for every key block: each
            // transposed operand feeds KB MFMAs.
            auto t_load = [&](int db) {
                oring[db % NR] = panel_vt_operand(Ot, pl, h, db);
                qring[db % NR] = panel_vt_operand(Qt, pl, h, db);
            };
#pragma unroll
            for (int db = 0; db < PF && db < DB; ++db) t_load(db);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                if (db + PF < DB) t_load(db + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
                    dv[kb][db] = mfma16x16x32(oring[db % NR], pb[kb], dv[kb][db]);
                    dk[kb][db] = mfma16x16x32(qring[db % NR], sb[kb], dk[kb][db]);
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    };
    if (ntiles > 0) issue(0, std::integral_constant<int, 0>{});
    for (int u = 0; u < ntiles; u += 2) {
        step(u, std::integral_constant<int, 0>{});
        if (u + 1 < ntiles) step(u + 1, std::integral_constant<int, 1>{});
    }
    if (ntiles == 0) wait_vmem();  // the V copies land before the workgroup ends

    // dK = scale * dS^T Q, dV = P^T dO; lane holds key k0w + 16*kb + l%16,
    // d = 16*db + 4*grp + 0..3.  The lane index passes through an empty asm
    // statement so that these addresses are formed here rather than shared
    // with the K loads before the scan (which kept them live across it).
    int lane_out = lane;
    asm volatile("" : "+v"(lane_out));
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const int kr = k0w + 16 * kb + (lane_out & 15);
        const int64_t kv_off = kv_base + (int64_t)kr * kv_row_stride;
        T* const dkrow = static_cast<T*>(p.dk) + kv_off;
        T* const dvrow = static_cast<T*>(p.dv) + kv_off;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 16 * db + 4 * (lane_out >> 4);
            if (kr < p.Nk && d < p.D) {
                typename V<T>::x4 rk, rv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    rk[e] = (T)(dk[kb][db][e] * p.scale);
                    rv[e] = (T)dv[kb][db][e];
                }
                *reinterpret_cast<typename V<T>::x4*>(dkrow + d) = rk;
                *reinterpret_cast<typename V<T>::x4*>(dvrow + d) = rv;
            }
        }
    }
}

template <int DP> int64_t nq_pad_of(int64_t Nq) {
    return (Nq + FaTile<DP>::BQ - 1) / FaTile<DP>::BQ * FaTile<DP>::BQ;
}

int64_t padded_rows(int64_t Nq, int64_t D) {
    return D > 128 ? nq_pad_of<256>(Nq) : nq_pad_of<128>(Nq);
}

// key_blocks: 16-key blocks per wavefront of the dK/dV kernel, 0 = chosen per
// shape; 1 or 2 force one kernel (kfm_fa_bwd_blocks, so tests reach both).
template <typename T, int DP>
int launch_bwd(const FaBwdParams& p, int key_blocks, hipStream_t stream) {
    const int64_t qblocks = (int64_t)p.n_qtiles * p.Hq * p.B;
    int64_t kblocks = (int64_t)p.n_ktiles * p.Hkv * p.B;
    // Two key blocks per wavefront (half the workgroups, each doing twice the
    // work at fewer LDS reads per product) once the grid still gives every
    // CU more than half a workgroup; both kernels run one workgroup per CU.
    // Under a causal mask, with the longest key tiles started first
    // (causal_tile_order), it is faster at D = 128 and 64 (B=2, H=16,
    // N=4096 on MI355X: 416 against 470 us and 258 against 296 us for the
    // whole backward) but not at D = 32, whose 512-key workgroups and the
    // wavefronts within one do too unequal work (245 against 229 us).
    bool wide = false;
    if constexpr (DP <= 128) {
        const int64_t wblocks = ((int64_t)p.Nk + dkdv_wide_keys<DP>() - 1) / dkdv_wide_keys<DP>() * p.Hkv * p.B;
        wide = key_blocks ? key_blocks == 2
                                     : (!p.causal || DP > 32) && 2 * wblocks > device_cu_count();
        if (wide) kblocks = wblocks;
    }
    if (qblocks > 0x7fffffff || kblocks > 0x7fffffff) {
        set_error("fa_bwd: grid too large");
        return KF_E_UNSUPPORTED;
    }
    if (qblocks > 0) {
        hipLaunchKernelGGL((fa_bwd_dq_kernel<T, DP>), dim3((unsigned)qblocks), dim3(FaTile<DP>::THREADS), 0,
                           stream, p);
        const int rc = check_launch("fa_bwd_dq_kernel launch");
        if (rc != KF_OK) return rc;
    }
    if (kblocks > 0) {
        if constexpr (DP <= 128) {
            if (wide) {
                hipLaunchKernelGGL((fa_bwd_dkdv_wide_kernel<T, DP>), dim3((unsigned)kblocks),
                                   dim3(FaTile<DP>::THREADS), 0, stream, p);
                return check_launch("fa_bwd_dkdv_wide_kernel launch");
            }
        }
        hipLaunchKernelGGL((fa_bwd_dkdv_kernel<T, DP>), dim3((unsigned)kblocks), dim3(FaTile<DP>::THREADS), 0,
                           stream, p);
        return check_launch("fa_bwd_dkdv_kernel launch");
    }
    return KF_OK;
}

template <typename T>
int launch_bwd_dp(const FaBwdParams& p, int dp, int key_blocks, hipStream_t stream) {
    switch (dp) {
        case 32: return launch_bwd<T, 32>(p, key_blocks, stream);
        case 64: return launch_bwd<T, 64>(p, key_blocks, stream);
        case 128: return launch_bwd<T, 128>(p, key_blocks, stream);
        case 256: return launch_bwd<T, 256>(p, key_blocks, stream);
        default: set_error("fa_bwd: head dim %d not supported by this build", p.D); return KF_E_UNSUPPORTED;
    }
}

bool bwd_dims_fit(int64_t B, int64_t Nq, int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D) {
    const int64_t lim = 0x3fffffff;
    return B >= 0 && Nq >= 0 && Nk >= 0 && B <= lim && Nq <= lim && Nk <= lim && Hq <= lim &&
           Hkv <= lim && D <= lim;
}

}  // namespace
}  // namespace kf

extern "C" int64_t kf_fa_bwd_workspace_bytes(int64_t B, int64_t Nq, int64_t Hq, int64_t D) {
    using namespace kf;
    if (B < 0 || Nq < 0 || Hq <= 0 || D <= 0 || D > 256 || !bwd_dims_fit(B, Nq, 0, Hq, 1, D)) return -1;
    return 2 * (int64_t)sizeof(float) * B * Hq * padded_rows(Nq, D);
}

namespace kf {
namespace {

int fa_bwd_run(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout,
               void* dq, void* dk, void* dv, void* workspace, int64_t workspace_bytes, int64_t B, int64_t Nq,
               int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D, float scale, int causal, int dtype, int key_blocks,
               kf_stream_t stream) {
    KF_REQUIRE(bwd_dims_fit(B, Nq, Nk, Hq, Hkv, D), KF_E_INVALID, "fa_bwd: shape out of range");
    KF_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0, KF_E_INVALID, "fa_bwd: Hq must be a positive multiple of Hkv");
    KF_REQUIRE(D > 0 && D % 8 == 0 && D <= 256, KF_E_INVALID,
               "fa_bwd: head dim must be a positive multiple of 8 <= 256, got %lld", (long long)D);
    KF_REQUIRE(scale > 0.f && scale < __builtin_inff(), KF_E_INVALID, "fa_bwd: scale must be finite and positive");
    KF_REQUIRE(dtype == KF_F16 || dtype == KF_BF16, KF_E_INVALID, "fa_bwd: dtype must be f16 or bf16");
    if (B == 0 || (Nq == 0 && Nk == 0)) return KF_OK;
    const int64_t need = kf_fa_bwd_workspace_bytes(B, Nq, Hq, D);
    KF_REQUIRE(need >= 0 && workspace_bytes >= need && (need == 0 || workspace), KF_E_WORKSPACE,
               "fa_bwd: workspace of %lld bytes needed, %lld given", (long long)need,
               (long long)workspace_bytes);
    KF_REQUIRE(q && k && v && o && lse && dout && dq && dk && dv, KF_E_INVALID, "fa_bwd: null pointer");
    FaBwdParams p{};
    p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse; p.dout = dout;
    p.dq = dq; p.dk = dk; p.dv = dv;
    const int64_t nq_pad = padded_rows(Nq, D);
    p.ws_lse2 = static_cast<float*>(workspace);
    p.ws_delta = static_cast<float*>(workspace) + B * Hq * nq_pad;
    p.B = (int)B; p.Nq = (int)Nq; p.Nk = (int)Nk; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.D = (int)D;
    p.group = (int)(Hq / Hkv);
    const int dp = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
    const int bq = dp > 128 ? FaTile<256>::BQ : FaTile<128>::BQ;
    const int bq_dq = dp > 128 ? dq_rows<256>() : dq_rows<128>();
    p.n_qtiles = (int)((Nq + bq_dq - 1) / bq_dq);
    p.n_ktiles = (int)((Nk + bq - 1) / bq);
    p.nq_pad = (int)nq_pad;
    p.scale = scale;
    p.scale_log2 = scale * kLog2e;
    p.causal = causal ? 1 : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    return dtype == KF_BF16 ? launch_bwd_dp<bf16>(p, dp, key_blocks, s) : launch_bwd_dp<f16>(p, dp, key_blocks, s);
}

}  // namespace
}  // namespace kf

extern "C" int kf_fa_bwd(const void* q, const void* k, const void* v, const void* o,
                         const float* lse, const void* dout, void* dq, void* dk, void* dv,
                         void* workspace, int64_t workspace_bytes, int64_t B, int64_t Nq,
                         int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D, float scale, int causal,
                         int dtype, kf_stream_t stream) {
    return kf::fa_bwd_run(q, k, v, o, lse, dout, dq, dk, dv, workspace, workspace_bytes, B, Nq, Nk, Hq, Hkv, D,
                          scale, causal, dtype, 0, stream);
}

// Test entry point (not in the public header): kf_fa_bwd with the dK/dV
// kernel's 16-key blocks per wavefront forced to one (1) or two (2) for head
// dims up to 128; 0 keeps the per-shape choice.
extern "C" int kfm_fa_bwd_blocks(const void* q, const void* k, const void* v, const void* o,
                                 const float* lse, const void* dout, void* dq, void* dk, void* dv,
                                 void* workspace, int64_t workspace_bytes, int64_t B, int64_t Nq,
                                 int64_t Nk, int64_t Hq, int64_t Hkv, int64_t D, float scale, int causal,
                                 int dtype, int key_blocks, kf_stream_t stream) {
    KF_REQUIRE(key_blocks >= 0 && key_blocks <= 2, KF_E_INVALID, "fa_bwd: key_blocks must be 0, 1 or 2");
    return kf::fa_bwd_run(q, k, v, o, lse, dout, dq, dk, dv, workspace, workspace_bytes, B, Nq, Nk, Hq, Hkv, D,
                          scale, causal, dtype, key_blocks, stream);
}
