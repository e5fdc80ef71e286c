// FlashAttention forward, fused forward+JVP, and JVP-from-LSE for gfx950.
//
// Semantics: dense softmax attention (flash_attention_jvp/original.py:6-30),
// its forward-mode derivative, and the single-pass online recurrence of
// flash_attention_jvp/flash-attention-jvp-derivation.md:388-558:
//   S = scale q k^T, tS = scale (tq k^T + q tk^T), E = exp(S - m),
//   l = sum E, U = E v, r = sum E*tS, G = (E*tS) v + E tv;
//   O = U/l, tO = G/l - (r/l) O, LSE = m + log l.
// The JVP-from-LSE mode recomputes P = exp(S - LSE) (flash_attention_jvp/
// custom.py:88-118) and, like the reference, takes O from the cached 16-bit
// output, five products per key tile:
//   tO = (P tv + H v)/l - (rowsum(H)/l) O,  l = rowsum(P) of the rounded P.
// The second term multiplies O's rounding error (2^-9 relative, plus the
// forward's own rounding of P) by rowsum(H)/l, which a peaked softmax makes
// large enough to break the bf16 tolerance.  So a row is written this way
// only while |rowsum(H)/l| * max(max|O|, 1) <= kCachedOBound; otherwise its
// workgroup redoes all its rows in a second scan that also accumulates
// U = P v (a sixth product) and uses U/l, which carries exactly the rounding
// of the P in the other terms:
//   tO = (P tv + H v)/l - (rowsum(H)/l) (U/l).
//
// Tiling.  A workgroup is 8 wavefronts x 16 query rows (128 rows) of one
// (batch, head), two wavefronts per SIMD so that one wavefront's softmax
// arithmetic runs while the other's matrix products occupy the MFMA pipe.  It
// scans the key axis in tiles of 64 keys (head dims up to 128; D = 256 uses 4
// wavefronts, one per SIMD, and tiles of 32 keys: see FaTile).  Per tile each wavefront computes
// the transposed score blocks S^T = K Q^T with v_mfma_f32_16x16x32 (A = K rows
// from LDS, B = Q held in registers): lane l owns query row l%16 and keys
// 16*kb + 4*(l/16) + i of key block kb.  Those accumulators are directly the
// B operand of O^T += V^T E^T once the K index of each 32-key step is
// enumerated as (keys 4*(l/16)+0..3 of block 2kk, then of block 2kk+1); V^T
// is read from the row-major V tile with ds_read_b64_tr_b16 in that order.
//
// Memory.  K, V (and tK, tV) tiles stream HBM -> LDS with global_load_lds
// (16 B per lane, no VGPR staging), double buffered, rows XOR-swizzled in
// 16-byte chunks so that neither the row reads (ds_read_b128) nor the
// transposing reads (ds_read_b64_tr_b16) conflict in the LDS banks.
// Workgroups are renumbered so that all query tiles of one head run on one
// XCD and share its L2.
//
// Operand pipelining.  The LDS reads of the MFMA operands (K rows, V^T
// columns) run a fixed number of steps ahead of the MFMAs that consume them,
// in small register rings; sched_barrier fences keep the compiler from
// sinking the reads back next to their uses, where each LDS latency would be
// exposed.  The first V^T operands of a half are read before the softmax
// arithmetic, so they arrive while it runs.
//
// Exponent reference.  FWD/FWD_JVP fix each row's reference m at the max of
// its first 32 keys and never raise it, so U and G are never rescaled inside
// the scan.  A later score exceeding m by ~2^7 (log2 units; 2^4 for fp16 E)
// overflows to a non-finite accumulator, which the workgroup detects at the
// end and answers by redoing its rows with a lazily rescaling scan (an
// out-of-line function).  The JVP-from-LSE mode uses -LSE as the reference.
#include "fa_common.h"

namespace kf {
namespace {

// Query tile, head and batch of this workgroup.  XCD-aware renumbering: the
// hardware sends block i to XCD i % 8; give each XCD a contiguous range of
// logical blocks (consecutive query tiles of a head).
struct FaBlock {
    int qtile, hq, b;
};
__device__ __forceinline__ FaBlock fa_block(const FaParams& p) {
    const int nblk = gridDim.x, id = blockIdx.x;
    const int per = nblk >> 3, rem = nblk & 7, xcd = id & 7, slot = id >> 3;
    const int lg = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    const int logical = p.causal ? causal_tile_order(lg, p.n_qtiles) : lg;
    FaBlock r;
    r.qtile = logical % p.n_qtiles;
    const int rest = logical / p.n_qtiles;
    r.hq = rest % p.Hq;
    r.b = rest / p.Hq;
    if (p.causal) r.qtile = p.n_qtiles - 1 - r.qtile;  // longest scans first
    return r;
}

// Row blocks of 16 query rows per wavefront.  The forward has the registers
// for two (a 256-row workgroup): every K row and V^T operand read from LDS
// then feeds two MFMAs, and a tile copy serves twice the rows.
template <int DP, int MODE> constexpr int fa_row_blocks() { return MODE == FA_FWD && DP <= 128 ? 2 : 1; }
template <int DP, int MODE> constexpr int fa_rows() { return FaTile<DP>::BQ * fa_row_blocks<DP, MODE>(); }

// One workgroup's rows: the scan over its key tiles and the epilogue.
// LAZY = false (the fast path): the exponent reference of a row is fixed at
// the max of its first 32 keys.  A later score far above it overflows the
// state; the workgroup then writes NaN into the LSE of its rows (and nothing
// else), and fa_fixup_kernel redoes those rows with LAZY = true, which raises
// the reference whenever a half's max exceeds it by 2^3 and rescales the
// state.  In the JVP-from-LSE mode LAZY = false is the cached-O scan (five
// products): a workgroup with a row past kCachedOBound writes NaN into the
// first tO element of its first row (and nothing else), and fa_fixup_kernel
// redoes its rows with LAZY = true, the scan that recomputes U.  kbuf0/1 and
// vbuf0/1 are the two K-side and V-side LDS buffers, NT tiles each.
template <typename T, int DP, int MODE, bool ALL, bool LAZY>
__device__ __forceinline__ void fa_scan(const FaParams& p, T* kbuf0, T* kbuf1, T* vbuf0, T* vbuf1) {
    constexpr int R = fa_row_blocks<DP, MODE>();
    constexpr int kBQ = fa_rows<DP, MODE>(), kBK = FaTile<DP>::BK;
    constexpr bool JVP = MODE != FA_FWD;
    constexpr bool kCachedO = MODE == FA_JVP && !LAZY;  // O from p.o, no U products
    constexpr int NT = JVP ? 2 : 1;   // tensors per side: K (, tK) and V (, tV)
    constexpr int DS = DP / 32;        // 32-wide K-steps of the score products
    constexpr int DB = DP / 16;        // 16-wide d blocks of the outputs
    constexpr int NSTEP = 2 * DS;      // (key block, K-step) pairs of a half
    // Operand prefetch distance in MFMA steps; the forward has registers to
    // spare for a deeper ring.
    constexpr int PF = JVP ? (DP > 128 ? 0 : 2) : 3;
    constexpr int NR = PF + 1;
    // At D = 256 (one wavefront per SIMD, 512 registers) the fences cost the
    // register allocator more than the ordering gains.
    constexpr bool kFence = DP <= 128;
    typedef typename V<T>::x8 x8;
    auto lds_tile = [&](auto bufc, auto vsc, int i) -> T* {
        constexpr int buf = decltype(bufc)::value;
        if constexpr (decltype(vsc)::value)
            return (buf == 0 ? vbuf0 : vbuf1) + i * (kBK * DP);
        else
            return (buf == 0 ? kbuf0 : kbuf1) + i * (kBK * DP);
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4;  // 16-lane group: key sub-range / d sub-range

    const FaBlock blk = fa_block(p);
    const int qtile = blk.qtile, hq = blk.hq, b = blk.b;
    const int hk = hq / p.group;

    const int q0w = qtile * kBQ + wave * 16 * R;  // first row of this wavefront
    const int64_t q_row_stride = (int64_t)p.Hq * p.D;
    const int64_t kv_row_stride = (int64_t)p.Hkv * p.D;
    const int64_t kv_base = (int64_t)b * p.Nk * kv_row_stride + (int64_t)hk * p.D;
    const int diag = p.Nk - p.Nq;                // key j valid for row i iff j <= i + diag
    // This lane's query row in row block rb.
    int qr[R];
    bool row_ok[R];
    int64_t q_off[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        qr[rb] = q0w + 16 * rb + (lane & 15);
        row_ok[rb] = qr[rb] < p.Nq;
        q_off[rb] = ((int64_t)b * p.Nq + qr[rb]) * q_row_stride + (int64_t)hq * p.D;
    }

    // Tangent presence: ALL instantiations have every tangent; the others
    // skip the products of the NULL ones.
    const bool use_tq = JVP && (ALL || p.tq != nullptr);
    const bool use_tk = JVP && (ALL || p.tk != nullptr);
    const bool use_tv = JVP && (ALL || p.tv != nullptr);

    // Q (and tQ) as B operands: lane l holds row qr, d = 32*ds + 8*grp + 0..7.
    x8 qreg[R][DS], tqreg[R][DS];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int d = 32 * ds + 8 * grp;
            const bool ok = row_ok[rb] && d < p.D;
            const u32x4 z = {0u, 0u, 0u, 0u};
            const u32x4 a = ok ? *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.q) + q_off[rb] + d) : z;
            qreg[rb][ds] = __builtin_bit_cast(x8, a);
            if constexpr (JVP) {
                const u32x4 t = (ok && use_tq)
                                    ? *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.tq) + q_off[rb] + d)
                                    : z;
                tqreg[rb][ds] = __builtin_bit_cast(x8, t);
            }
        }
    // The cached O values this lane's output elements need (d = 16*db +
    // 4*grp + 0..3; D % 8 == 0, so a chunk below D lies wholly below it).
    typename V<T>::x4 ocv[R][kCachedO ? DB : 1];
    if constexpr (kCachedO) {
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const int d = 16 * db + 4 * grp;
                typename V<T>::x4 z;
#pragma unroll
                for (int e = 0; e < 4; ++e) z[e] = (T)0.f;
                ocv[rb][db] = row_ok[rb] && d < p.D
                                  ? *reinterpret_cast<const typename V<T>::x4*>(static_cast<const T*>(p.o) +
                                                                                 q_off[rb] + d)
                                  : z;
            }
    }

    // Key range of the workgroup.
    int key_stop = p.Nk;
    if (p.causal) key_stop = min(p.Nk, max(0, qtile * kBQ + kBQ + diag));
    const int ntiles = (key_stop + kBK - 1) / kBK;
    int klim[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) klim[rb] = p.causal ? min(p.Nk - 1, qr[rb] + diag) : p.Nk - 1;
    const float c = p.scale_log2;

    // Row statistics (each lane holds a quarter of its row's keys).  In the
    // JVP modes l_run and r_run sum the 16-bit E and H values the products
    // consume, so O is an exact convex combination of V rows and
    // tO = sum_j H_j (v_j - O) / l.  l_lse sums the fp32 E for the LSE output;
    // the forward alone also normalises O by it (as flash-attn does), which
    // saves a dot product per pair of keys in its VALU-bound inner loop.
    // m_run is in log2 units.
    float m_run[R], l_run[R], r_run[R], l_lse[R];
    // Exponent offset: -m_run, or -LSE (log2 units) in the JVP mode (+inf LSE
    // -> P = 0).
    float nref[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        m_run[rb] = -__builtin_inff();
        l_run[rb] = r_run[rb] = l_lse[rb] = 0.f;
        nref[rb] = 0.f;
        if constexpr (MODE == FA_JVP) {
            nref[rb] = row_ok[rb] ? -p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr[rb]] * kLog2e : -__builtin_inff();
        }
    }

    // Full tiles (all keys valid, D == DP) take the uniform-address copy.
    const uint32_t voff = full_tile_shortcut<DP>() ? full_tile_lane_offset<T, DP>(kv_row_stride, wave, lane) : 0u;
    const bool dense_rows = p.D == DP;
    const T* const kbase = static_cast<const T*>(p.k) + kv_base;
    const T* const vbase = static_cast<const T*>(p.v) + kv_base;
    const T* const tkbase = use_tk ? static_cast<const T*>(p.tk) + kv_base : nullptr;
    const T* const tvbase = use_tv ? static_cast<const T*>(p.tv) + kv_base : nullptr;
    auto tile_masked = [&](int k0) {
        return (k0 + kBK > p.Nk) || (p.causal && k0 + kBK - 1 > q0w + diag);
    };
    // A tile's keys are consumed in halves of 32 (key blocks 2h, 2h+1).
    auto apply_mask = [&](f32x4 (&s)[2], int k0, int h, int lim) {
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (k0 + 16 * (2 * h + i2) + 4 * grp + i > lim) s[i2][i] = -__builtin_inff();
    };
    auto row_max = [&](const f32x4 (&s)[2]) {
        float mx = s[0][0];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[i2][i]);
        return row_max4(mx) * c;
    };

    // Copies of one side of tile `tile` into its buffer: the K side (K, tK)
    // or the V side (V, tV).  The two sides are issued at different points of
    // the previous tile's work so that the wavefronts of a workgroup do not
    // all queue their copies at the same moment.  `bufc` and `vsc` are
    // compile-time constants (std::integral_constant), so each copy names its
    // destination buffer statically.
    auto issue_side = [&](int tile, auto bufc, auto vsc) {
        constexpr bool vs = decltype(vsc)::value;
        const int k0 = tile * kBK;
        const int64_t off = (int64_t)k0 * kv_row_stride;
        T* const d0 = lds_tile(bufc, vsc, 0);
        T* const d1 = lds_tile(bufc, vsc, NT - 1);
        const T* const s0 = (vs ? vbase : kbase) + off;
        const T* const s1 = (vs ? tvbase : tkbase) + off;
        const bool tan = JVP && (vs ? use_tv : use_tk);
        if constexpr (full_tile_shortcut<DP>()) {
            if (dense_rows && k0 + kBK <= p.Nk) {
                load_tile_full<T, DP, FaTile<DP>::WAVES, JVP>(d0, s0, kv_row_stride, voff, wave);
                if (tan) load_tile_full<T, DP, FaTile<DP>::WAVES, JVP>(d1, s1, kv_row_stride, voff, wave);
                return;
            }
        }
        const int kv = p.Nk - k0;
        load_tile<T, DP>(d0, s0, kv_row_stride, kv, p.D, wave, lane);
        if (tan) load_tile<T, DP>(d1, s1, kv_row_stride, kv, p.D, wave, lane);
    };

    // Operand rings: slot st % NR holds the operands of MFMA step st.
    x8 kring[NR], tkring[NR], vring[NR], tvring[NR];
    // Step st of a half covers key block 2h + i2 at K-step ds.  The forward
    // takes the steps in pairs (both key blocks of one K-step), so that no
    // product waits on the one just issued into the same accumulator
    // (230.5-231 against 233.7-233.8 us at B=2, H=16, N=4096, D=128 on
    // MI355X).  In the JVP modes the same pairing, of the score products,
    // the P.V products or both, ran 0.5-2% slower, so they go key block by
    // key block.
    constexpr bool kPaired = !JVP;
    static_assert(!kPaired || (PF >= 2 && NSTEP % 2 == 0 && DB % 2 == 0), "pairs fit the ring");
    auto step_i2 = [](int st) { return kPaired ? st % 2 : st / DS; };
    auto step_ds = [](int st) { return kPaired ? st / 2 : st % DS; };
    auto k_load = [&](auto bufc, int h, int st) {
        const int i2 = step_i2(st), ds = step_ds(st);
        const int krow = 16 * (2 * h + i2) + (lane & 15);
        kring[st % NR] = row_chunk<T, DP>(lds_tile(bufc, std::false_type{}, 0), krow, 4 * ds + grp);
        if constexpr (JVP) {
            if (use_tk)
                tkring[st % NR] = row_chunk<T, DP>(lds_tile(bufc, std::false_type{}, NT - 1), krow, 4 * ds + grp);
        }
    };
    auto v_load = [&](auto bufc, int h, int db) {
        vring[db % NR] = vt_operand<T, DP>(lds_tile(bufc, std::true_type{}, 0), h, db, lane);
        if constexpr (JVP) {
            if (use_tv) tvring[db % NR] = vt_operand<T, DP>(lds_tile(bufc, std::true_type{}, NT - 1), h, db, lane);
        }
    };

    // S^T (and tS^T) of key blocks 2h, 2h+1 of the tile in buffer bufc, for
    // every row block; ends by reading the first V^T operands of the half.
    auto scores = [&](auto bufc, int h, f32x4 (&s)[R][2], f32x4 (&ts)[R][2]) {
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
                s[rb][i2] = f32x4{0.f, 0.f, 0.f, 0.f};
                ts[rb][i2] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int st = 0; st < PF && st < NSTEP; ++st) k_load(bufc, h, st);
        if constexpr (kPaired) {
            // Both key blocks of a K-step together: s of each, then the two tS
            // terms of each, so no product waits on the one just issued into
            // the same accumulator (each accumulator still sums its terms in
            // the same order).  The ring slot of the pair's first step is
            // refilled only after the pair's products.
#pragma unroll
            for (int sp = 0; sp < NSTEP; sp += 2) {
                if (sp + PF < NSTEP) k_load(bufc, h, sp + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const int ds = sp / 2;
                const x8 k0 = kring[sp % NR], k1 = kring[(sp + 1) % NR];
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    s[rb][0] = mfma16x16x32(k0, qreg[rb][ds], s[rb][0]);
                    s[rb][1] = mfma16x16x32(k1, qreg[rb][ds], s[rb][1]);
                }
                if constexpr (JVP) {
#pragma unroll
                    for (int rb = 0; rb < R; ++rb) {
                        if (use_tq) {
                            ts[rb][0] = mfma16x16x32(k0, tqreg[rb][ds], ts[rb][0]);
                            ts[rb][1] = mfma16x16x32(k1, tqreg[rb][ds], ts[rb][1]);
                        }
                        if (use_tk) {
                            ts[rb][0] = mfma16x16x32(tkring[sp % NR], qreg[rb][ds], ts[rb][0]);
                            ts[rb][1] = mfma16x16x32(tkring[(sp + 1) % NR], qreg[rb][ds], ts[rb][1]);
                        }
                    }
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                if (sp + 1 + PF < NSTEP) k_load(bufc, h, sp + 1 + PF);
            }
        } else {
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                if (st + PF < NSTEP) k_load(bufc, h, st + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const int i2 = st / DS, ds = st % DS;
                const x8 ka = kring[st % NR];
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    s[rb][i2] = mfma16x16x32(ka, qreg[rb][ds], s[rb][i2]);
                    if constexpr (JVP) {
                        if (use_tq) ts[rb][i2] = mfma16x16x32(ka, tqreg[rb][ds], ts[rb][i2]);
                        if (use_tk) ts[rb][i2] = mfma16x16x32(tkring[st % NR], qreg[rb][ds], ts[rb][i2]);
                    }
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int db = 0; db < PF && db < DB; ++db) v_load(bufc, h, db);
    };

    // E = exp2(S*c + nref) and H = E * scale * tS, packed to 16 bits; their
    // rounded values are summed into l and r.
    auto probs = [&](int rb, const f32x4 (&s)[2], const f32x4 (&ts)[2], u32x2 (&ew)[2], u32x2 (&hw)[2]) {
        // The first pair starts the sum: 0 + x is not folded under IEEE
        // signed zeros, and E >= 0 makes the two sums equal bit for bit.
        float esum = 0.f;
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float e0 = fast_exp2(fmaf(s[i2][2 * j], c, nref[rb]));
                const float e1 = fast_exp2(fmaf(s[i2][2 * j + 1], c, nref[rb]));
                if constexpr (MODE != FA_JVP) esum = i2 == 0 && j == 0 ? e0 + e1 : esum + (e0 + e1);
                const unsigned pe = Pk<T>::cvt(e0, e1);
                ew[i2][j] = pe;
                if constexpr (JVP) l_run[rb] = Pk<T>::sum_into(pe, l_run[rb]);
                if constexpr (JVP) {
                    const unsigned ph = Pk<T>::cvt(e0 * (ts[i2][2 * j] * p.scale), e1 * (ts[i2][2 * j + 1] * p.scale));
                    hw[i2][j] = ph;
                    r_run[rb] = Pk<T>::sum_into(ph, r_run[rb]);
                }
            }
        if constexpr (MODE != FA_JVP) l_lse[rb] += esum;
    };

    f32x4 u[R][DB], g[R][DB];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            u[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
            g[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    // O^T += V^T E^T (not in the cached-O scan) ; G^T += V^T H^T + tV^T E^T
    // over the 32 keys of half h
    // of the tile in buffer bufc.
    auto pv = [&](auto bufc, int h, const u32x2 (&ew)[R][2], const u32x2 (&hw)[R][2]) {
        x8 eb[R], hb[R];
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            eb[rb] = __builtin_bit_cast(x8, u32x4{ew[rb][0][0], ew[rb][0][1], ew[rb][1][0], ew[rb][1][1]});
            hb[rb] = __builtin_bit_cast(x8, u32x4{hw[rb][0][0], hw[rb][0][1], hw[rb][1][0], hw[rb][1][1]});
        }
        if constexpr (kPaired) {
            // Two d blocks together: U of each, then the two G terms of each.
#pragma unroll
            for (int db = 0; db < DB; db += 2) {
                if (db + PF < DB) v_load(bufc, h, db + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const x8 v0 = vring[db % NR], v1 = vring[(db + 1) % NR];
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    u[rb][db] = mfma16x16x32(v0, eb[rb], u[rb][db]);
                    u[rb][db + 1] = mfma16x16x32(v1, eb[rb], u[rb][db + 1]);
                }
                if constexpr (JVP) {
#pragma unroll
                    for (int rb = 0; rb < R; ++rb) {
                        g[rb][db] = mfma16x16x32(v0, hb[rb], g[rb][db]);
                        g[rb][db + 1] = mfma16x16x32(v1, hb[rb], g[rb][db + 1]);
                        if (use_tv) {
                            g[rb][db] = mfma16x16x32(tvring[db % NR], eb[rb], g[rb][db]);
                            g[rb][db + 1] = mfma16x16x32(tvring[(db + 1) % NR], eb[rb], g[rb][db + 1]);
                        }
                    }
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                if (db + 1 + PF < DB) v_load(bufc, h, db + 1 + PF);
            }
        } else {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                if (db + PF < DB) v_load(bufc, h, db + PF);
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
                const x8 va = vring[db % NR];
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    if constexpr (!kCachedO) u[rb][db] = mfma16x16x32(va, eb[rb], u[rb][db]);
                    if constexpr (JVP) {
                        g[rb][db] = mfma16x16x32(va, hb[rb], g[rb][db]);
                        if (use_tv) g[rb][db] = mfma16x16x32(tvring[db % NR], eb[rb], g[rb][db]);
                    }
                }
                if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // LAZY: raise the reference of rows whose max grew past m + 2^3 and
    // rescale their state (alpha = 0 for a row leaving m = -inf, whose state
    // is zero).
    auto rebase = [&](int rb, const f32x4 (&s)[2]) {
        const float mx = row_max(s);
        const bool upd = mx > m_run[rb] + kRescaleThreshold;
        if (__any(upd)) {
            const float alpha = upd ? fast_exp2(m_run[rb] - mx) : 1.f;
            if (upd) m_run[rb] = mx;
            l_run[rb] *= alpha;
            r_run[rb] *= alpha;
            l_lse[rb] *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    u[rb][db][i] *= alpha;
                    if constexpr (JVP) g[rb][db][i] *= alpha;
                }
            nref[rb] = m_run[rb] == -__builtin_inff() ? 0.f : -m_run[rb];
        }
    };

    // One key tile; tile t lives in buffer t & 1 == decltype(bufc)::value.
    auto step = [&](int t, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const std::integral_constant<int, buf ^ 1> nbuf;
        const int k0 = t * kBK;
        const bool masked = tile_masked(k0);
        wait_vmem();
        __syncthreads();  // tile t resident; every wavefront is done with tile t-1
        if (t + 1 < ntiles) issue_side(t + 1, nbuf, std::false_type{});
#pragma unroll
        for (int h = 0; h < FaTile<DP>::HALVES; ++h) {
            f32x4 s[R][2], ts[R][2];
            u32x2 ew[R][2], hw[R][2];
#pragma unroll
            for (int rb = 0; rb < R; ++rb) hw[rb][0] = hw[rb][1] = u32x2{0u, 0u};
            scores(bufc, h, s, ts);
            if (h == 0 && t + 1 < ntiles) issue_side(t + 1, nbuf, std::true_type{});
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                if (masked) apply_mask(s[rb], k0, h, klim[rb]);
                if constexpr (MODE != FA_JVP) {
                    if constexpr (LAZY) {
                        rebase(rb, s[rb]);
                    } else if (t == 0 && h == 0) {
                        // Every non-empty row has a valid key among its first
                        // 32 (masks only cut keys off at the end).
                        m_run[rb] = row_max(s[rb]);
                        nref[rb] = m_run[rb] == -__builtin_inff() ? 0.f : -m_run[rb];
                    }
                }
                probs(rb, s[rb], ts[rb], ew[rb], hw[rb]);
            }
            // The wavefront entering its P.V products takes issue priority
            // over the other wavefront of its SIMD (in its softmax arithmetic
            // or score products), so that the MFMA pipe refills first:
            // 0.6-1.1% faster for the JVP modes at B=2, H=16, N=4096,
            // D=128 on MI355X (the forward saw no gain).
            if constexpr (JVP) __builtin_amdgcn_s_setprio(1);
            pv(bufc, h, ew, hw);
            if constexpr (JVP) __builtin_amdgcn_s_setprio(0);
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

    if constexpr (MODE != FA_JVP && !LAZY) {
        // Overflow check, made uniform over the workgroup (the rescaling scan
        // needs every wavefront for its tile copies).
        bool fin = true;
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            fin = fin && __builtin_isfinite(l_lse[rb]) && __builtin_isfinite(r_run[rb]);
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    fin = fin && __builtin_isfinite(u[rb][db][i]);
                    if constexpr (JVP) fin = fin && __builtin_isfinite(g[rb][db][i]);
                }
        }
        if (__syncthreads_or(!fin)) {
#pragma unroll
            for (int rb = 0; rb < R; ++rb)
                if (grp == 0 && row_ok[rb]) p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr[rb]] = __builtin_nanf("");
            return;
        }
    }

    if constexpr (kCachedO) {
        // tO = G/l - (r/l) O with the cached O, unless a row's r/l could
        // amplify O's rounding past the bound: then only the marker is
        // written and fa_fixup_kernel redoes the workgroup's rows with U
        // (uniform over the workgroup: that scan needs every wavefront for its
        // tile copies).
        float inv[R], rl[R];
        bool over = false;
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            const float l_tot = row_sum4(l_run[rb]);
            inv[rb] = l_tot > 0.f ? 1.f / l_tot : 0.f;
            rl[rb] = row_sum4(r_run[rb]) * inv[rb];
            float om = 0.f;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int e = 0; e < 4; ++e) om = fmaxf(om, fabsf((float)ocv[rb][db][e]));
            om = row_max4(om);
            over = over || (row_ok[rb] && fabsf(rl[rb]) * fmaxf(om, 1.f) > kCachedOBound);
        }
        if (__syncthreads_or(over)) {
            // The marker: NaN in the first element of the workgroup's first
            // row (wavefront 0, lane 0; that row always exists).
            if (wave == 0 && lane == 0) static_cast<T*>(p.to)[q_off[0]] = (T)__builtin_nanf("");
            return;
        }
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            T* torow = static_cast<T*>(p.to) + q_off[rb];
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const int d = 16 * db + 4 * grp;
                if (row_ok[rb] && d < p.D) {
                    typename V<T>::x4 tv;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        tv[e] = (T)(g[rb][db][e] * inv[rb] - rl[rb] * (float)ocv[rb][db][e]);
                    *reinterpret_cast<typename V<T>::x4*>(torow + d) = tv;
                }
            }
        }
        return;
    }

    // ---- epilogue: O = U/l, tO = G/l - (r/l) O, LSE = m + log l ----
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        const float l_tot = JVP ? row_sum4(l_run[rb]) : row_sum4(l_lse[rb]);
        const float r_tot = row_sum4(r_run[rb]);
        const float l_lse_tot = row_sum4(l_lse[rb]);
        T* orow = static_cast<T*>(p.o) + q_off[rb];
        T* torow = static_cast<T*>(p.to) + q_off[rb];
        const bool empty = !(l_tot > 0.f);
        const float inv = empty ? 0.f : 1.f / l_tot;
        const float rl = r_tot * inv;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 16 * db + 4 * grp;
            if (row_ok[rb] && d < p.D) {
                typename V<T>::x4 ov, tv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float o = u[rb][db][e] * inv;
                    ov[e] = (T)o;
                    if constexpr (JVP) tv[e] = (T)(g[rb][db][e] * inv - rl * o);
                }
                if constexpr (MODE != FA_JVP) *reinterpret_cast<typename V<T>::x4*>(orow + d) = ov;
                if constexpr (JVP) *reinterpret_cast<typename V<T>::x4*>(torow + d) = tv;
            }
        }
        if (MODE != FA_JVP && grp == 0 && row_ok[rb]) {
            p.lse[((int64_t)b * p.Hq + hq) * p.Nq + qr[rb]] =
                empty ? __builtin_inff() : (m_run[rb] + log2f(l_lse_tot)) * kLn2;
        }
    }
}

// Double-buffered K-side (K, tK) and V-side (V, tV) tiles.  Each buffer is its
// own LDS variable so that the compiler's alias analysis separates the copies
// into one buffer from the reads of the other.
#define FA_LDS_BUFFERS(T, DP, MODE)                                         \
    constexpr int NT_ = (MODE) != FA_FWD ? 2 : 1;                          \
    constexpr int TILE_ = FaTile<DP>::BK * (DP);                           \
    __shared__ __attribute__((aligned(16))) T kside0[NT_ * TILE_];         \
    __shared__ __attribute__((aligned(16))) T kside1[NT_ * TILE_];         \
    __shared__ __attribute__((aligned(16))) T vside0[NT_ * TILE_];         \
    __shared__ __attribute__((aligned(16))) T vside1[NT_ * TILE_]

template <typename T, int DP, int MODE, bool ALL>
__global__ __launch_bounds__(FaTile<DP>::THREADS)
__attribute__((amdgpu_waves_per_eu(FaTile<DP>::OCC, FaTile<DP>::OCC)))
void fa_kernel(const FaParams p) {
    FA_LDS_BUFFERS(T, DP, MODE);
    fa_scan<T, DP, MODE, ALL, false>(p, kside0, kside1, vside0, vside1);
}

// Second launch of every mode: a workgroup whose rows carry the marker redoes
// them with the LAZY = true scan (the rescaling scan in FWD/FWD_JVP, marker NaN
// LSE; the scan that recomputes U in the JVP-from-LSE mode, marker NaN in the
// first tO element of the workgroup's first row); every other workgroup reads
// its markers and exits.  A separate kernel keeps that code out of the fast
// scan's register allocation (inlined, the two scans spill at D = 128).
template <typename T, int DP, int MODE, bool ALL>
__global__ __launch_bounds__(FaTile<DP>::THREADS)
__attribute__((amdgpu_waves_per_eu(FaTile<DP>::OCC, FaTile<DP>::OCC)))
void fa_fixup_kernel(const FaParams p) {
    const FaBlock blk = fa_block(p);
    constexpr int kBQ = fa_rows<DP, MODE>();
    static_assert(kBQ <= FaTile<DP>::THREADS, "one thread per row checks the marker");
    const int row = blk.qtile * kBQ + (int)threadIdx.x;
    bool marked = false;
    if constexpr (MODE == FA_JVP) {
        if (threadIdx.x == 0)
            marked = __builtin_isnan(
                (float)static_cast<const T*>(p.to)[((int64_t)blk.b * p.Nq + row) * p.Hq * p.D + (int64_t)blk.hq * p.D]);
    } else if (threadIdx.x < kBQ && row < p.Nq) {
        marked = __builtin_isnan(p.lse[((int64_t)blk.b * p.Hq + blk.hq) * p.Nq + row]);
    }
    if (!__syncthreads_or(marked)) return;
    FA_LDS_BUFFERS(T, DP, MODE);
    fa_scan<T, DP, MODE, ALL, true>(p, kside0, kside1, vside0, vside1);
}

template <typename T, int MODE, bool ALL>
int launch_variant(const FaParams& p, int dp, hipStream_t stream) {
    const int64_t blocks = (int64_t)p.n_qtiles * p.Hq * p.B;
    if (blocks > 0x7fffffff) {
        set_error("fa: grid too large");
        return KF_E_UNSUPPORTED;
    }
    const dim3 grid((unsigned)blocks);
    auto launch = [&](auto dpc) {
        constexpr int DP = decltype(dpc)::value;
        hipLaunchKernelGGL((fa_kernel<T, DP, MODE, ALL>), grid, dim3(FaTile<DP>::THREADS), 0, stream, p);
        const int rc = check_launch("fa_kernel launch");
        if (rc != KF_OK) return rc;
        hipLaunchKernelGGL((fa_fixup_kernel<T, DP, MODE, ALL>), grid, dim3(FaTile<DP>::THREADS), 0, stream, p);
        return check_launch("fa_fixup_kernel launch");
    };
    switch (dp) {
        case 32: return launch(std::integral_constant<int, 32>{});
        case 64: return launch(std::integral_constant<int, 64>{});
        case 128: return launch(std::integral_constant<int, 128>{});
        case 256: return launch(std::integral_constant<int, 256>{});
        default: set_error("fa: head dim %d not supported by this build", p.D); return KF_E_UNSUPPORTED;
    }
}

// The JVP modes have a branch-free instantiation for the common case of
// three tangents and one that skips the products of NULL tangents.
template <typename T, int MODE>
int launch_mode(const FaParams& p, int dp, hipStream_t stream) {
    if (MODE == FA_FWD || (p.tq && p.tk && p.tv)) return launch_variant<T, MODE, true>(p, dp, stream);
    return launch_variant<T, MODE, false>(p, dp, stream);
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
    const int dp = p.D <= 32 ? 32 : p.D <= 64 ? 64 : p.D <= 128 ? 128 : 256;
    const int bq = dp > 128 ? fa_rows<256, FA_FWD_JVP>() : mode == FA_FWD ? fa_rows<128, FA_FWD>() : fa_rows<128, FA_FWD_JVP>();
    p.group = p.Hq / p.Hkv;
    p.n_qtiles = (p.Nq + bq - 1) / bq;
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
