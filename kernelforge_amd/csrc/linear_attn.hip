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
//   1. linattn_state_kernel   grid (ceil(H/2), splits, B): each workgroup streams
//      one sequence split of two adjacent heads (128 contiguous bytes of K and of
//      V per token) through LDS and accumulates S with v_mfma_f32_32x32x16; the
//      token-major operands are read with ds_read_b64_tr_b16.  z accumulates on
//      the VALU from the same registers.  Partials [B][H][splits][D+1][D] fp32.
//   2. linattn_reduce_kernel  four state elements per thread: sums the partials
//      in split order (fixed order: deterministic, no atomics).
//   3. linattn_out_kernel     grid (ceil(H/4), ceil(N/64), B): one wavefront per
//      head keeps S and z in registers as hi+lo 16-bit pairs (so the products
//      carry ~16 mantissa bits of the fp32 state); relu(q) of 64 tokens x 4
//      heads arrives with whole-line loads, is staged in LDS and read back as
//      the B operand of v_mfma_f32_16x16x32; z is a third A operand whose rows
//      all equal z, so the denominator lands in the same lanes as the
//      numerator.  The normalised rows leave through LDS as whole-line stores.
// Other head dims (128 % D == 0) and fp32 input take a VALU path with the same
// three stages and the same fixed-order split reduction.
#include "kf_common.h"

#include <mutex>

// Device scratch of kf_linattn_fwd_noalloc: the split partials and reduced
// states live here instead of in a caller workspace.  Each GPU the library
// runs on holds its own copy until the process ends; host code reaches it
// only through the per-device address from hipGetSymbolAddress.
constexpr int64_t kLinattnScratchBytes = 16LL << 20;
static __device__ __align__(256) unsigned char scratch[kLinattnScratchBytes];

namespace kf {
namespace {

constexpr int kD = 32;              // head dim of the MFMA path
constexpr int kState = (kD + 1) * kD;
constexpr int kTT = 64;             // tokens per state tile
constexpr int kRS = 72;             // LDS row stride (elements) of a 64-channel row
constexpr int kOutTokens = 64;      // tokens per output workgroup

// --------------------------------------------------------------------------
// 1. Split-state producer (MFMA).
// --------------------------------------------------------------------------
// Workgroup barrier that leaves global loads in flight.  __syncthreads()
// also waits for every outstanding global load (vmcnt(0)), which would drain
// the register prefetch below at each tile; here only this wave's LDS
// traffic is completed (lgkmcnt(0)) before s_barrier.  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_keep_loads() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt untouched
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Global -> register staging of one 64-token tile of a head pair: 4 x 16 B per
// thread.  Chunk c = i*256 + tid: token c/16, part (c/8)%2 (0 = K, 1 = V),
// 16-byte segment c%8 of the 128-byte two-head span, so every load
// instruction of a wave covers 4 tokens x 2 whole 128-byte lines.  Addresses
// are clamped into the split (token t_end-1) and onto the present head, so
// the number of loads never depends on the data; the clamped duplicates are
// zeroed when the tile is stored to LDS.
template <typename T>
__device__ __forceinline__ void state_gload(u32x4 (&reg)[4], const T* __restrict__ qkv, int64_t b,
                                            int N, int64_t C, int h0, int nh, int t0, int t_end,
                                            int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = i * 256 + tid;
        const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
        const int t = min(t0 + tok, t_end - 1);
        const int sg = seg < nh * 4 ? seg : seg - 4;
        const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (1 + part) * C + (int64_t)h0 * kD + sg * 8;
        reg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
}

template <typename T>
__global__ __launch_bounds__(256) void linattn_state_kernel(const T* __restrict__ qkv,
                                                            float* __restrict__ partial, int N,
                                                            int H, int split_len, int splits) {
    // Head pairs vary fastest over the grid, so the workgroups resident at one
    // time read neighbouring 128-byte spans of the same token rows.
    const int g = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t C = (int64_t)H * kD;
    const int h0 = 2 * g;
    const int nh = min(2, H - h0);
    const int t_begin = s * split_len;            // < N: the host sizes the grid
    const int t_end = min(N, t_begin + split_len);

    // [buf][K,V][tok*kRS+ch]; after the scan the same memory combines the
    // two token halves ([head slot][lane][16 accumulators + z]).
    __shared__ __attribute__((aligned(16))) T tile[2][2][kTT * kRS];
    static_assert(sizeof(tile) >= 2 * 64 * 17 * sizeof(float), "combine buffer fits in the tiles");
    float (*comb)[64][17] = reinterpret_cast<float (*)[64][17]>(&tile[0][0][0]);

    // Tile rows at or past t_end are stored as zeros; ReLU is applied to K.
    auto lstore = [&](const u32x4 (&reg)[4], int buf, int t0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * 256 + tid;
            const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
            const u32x4 z = {0u, 0u, 0u, 0u};
            const u32x4 v = t0 + tok < t_end ? (part == 0 ? relu_packed16(reg[i]) : reg[i]) : z;
            *reinterpret_cast<u32x4*>(&tile[buf][part][tok * kRS + seg * 8]) = v;
        }
    };

    // Wave (hw, th): head slot hw, token half th of each 64-token tile.
    const int hw = wave & 1, th = wave >> 1;
    const int G = lane >> 4, j16 = lane & 15;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    float zsum = 0.f;

    auto compute = [&](int buf) {
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
    };

    // Three tiles stay in flight in registers while one is consumed from LDS.
    // Tile j is loaded into register set j % 3 and stored to LDS buffer j % 2
    // one iteration ahead of its use.  The register set is chosen at compile
    // time (the loop is unrolled by three), and every step issues its loads
    // (past the end of the split they re-read row t_end-1), so the compiler's
    // wait before each LDS store is an exact count of younger loads.
    const int ntile = (t_end - t_begin + kTT - 1) / kTT;  // >= 1
    u32x4 r0[4], r1[4], r2[4];
    state_gload<T>(r0, qkv, b, N, C, h0, nh, t_begin, t_end, tid);
    state_gload<T>(r1, qkv, b, N, C, h0, nh, t_begin + kTT, t_end, tid);
    state_gload<T>(r2, qkv, b, N, C, h0, nh, t_begin + 2 * kTT, t_end, tid);
    lstore(r0, 0, t_begin);
    barrier_keep_loads();
    // Step it: LDS buffer it&1 holds tile it; `nx` holds tile it+1; `fr` is
    // free and receives tile it+3.
    auto step = [&](int it, u32x4 (&fr)[4], u32x4 (&nx)[4]) {
        state_gload<T>(fr, qkv, b, N, C, h0, nh, t_begin + (it + 3) * kTT, t_end, tid);
        compute(it & 1);
        lstore(nx, (it + 1) & 1, t_begin + (it + 1) * kTT);
        barrier_keep_loads();
    };
    for (int it = 0; it < ntile; it += 3) {
        step(it, r0, r1);
        if (it + 1 < ntile) step(it + 1, r1, r2);
        if (it + 2 < ntile) step(it + 2, r2, r0);
    }

    // Combine the two token halves of each head, then write the partial.
    __syncthreads();
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
// VEC consecutive state elements of one (batch, head) per thread; the
// partials of all splits are loaded eight at a time (a short last batch is
// padded with zeros, so every batch is one round of independent loads) and
// added in split order (deterministic, no atomics).
template <int VEC>
__global__ __launch_bounds__(256) void linattn_reduce_kernel(const float* __restrict__ partial,
                                                             float* __restrict__ state,
                                                             int64_t n_heads, int splits,
                                                             int state_size) {
    typedef float fv __attribute__((ext_vector_type(VEC)));
    const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
    if (idx >= n_heads * state_size) return;
    const int64_t bh = idx / state_size;
    const int e = (int)(idx - bh * state_size);  // state_size % VEC == 0: one (b, h)
    const float* P = partial + bh * splits * (int64_t)state_size + e;
    fv acc = {};
    for (int s = 0; s < splits; s += 8) {
        fv v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[j] = s + j < splits ? *reinterpret_cast<const fv*>(P + (int64_t)(s + j) * state_size) : fv{};
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += v[j];  // a padded zero leaves acc unchanged
    }
    *reinterpret_cast<fv*>(state + idx) = acc;
}

// Launch of the reduction: four elements per thread when a state is a whole
// number of 16-byte vectors (all head dims but 1 and 2) and the workspace is
// 16-byte aligned.
int launch_reduce(const float* partial, float* state, int64_t n_heads, int splits, int state_size,
                  hipStream_t stream) {
    const int64_t n = n_heads * state_size;
    if (state_size % 4 == 0 && (uintptr_t)partial % 16 == 0) {
        hipLaunchKernelGGL(linattn_reduce_kernel<4>, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0,
                           stream, partial, state, n_heads, splits, state_size);
    } else {
        hipLaunchKernelGGL(linattn_reduce_kernel<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           stream, partial, state, n_heads, splits, state_size);
    }
    return check_launch("linattn_reduce_kernel launch");
}

// --------------------------------------------------------------------------
// 3. Output contraction (MFMA, state in registers).
// --------------------------------------------------------------------------
// Stores of the numerator pair (n0: channels 4kg..4kg+3, n1: 16+4kg..) after
// v_permlane16_swap has exchanged n1 of the even 16-lane groups with n0 of
// the odd ones: an even group then holds channels 4kg..4kg+7, an odd group
// 16+4(kg-1)..16+4(kg-1)+7, so each lane writes 8 consecutive channels.
template <typename TO> struct Store8;
template <> struct Store8<float> {
    __device__ static void run(float* p, f32x4 a, f32x4 b) {
        *reinterpret_cast<f32x4*>(p) = a;
        *reinterpret_cast<f32x4*>(p + 4) = b;
    }
};
template <typename TO> struct Store8 {
    __device__ static void run(TO* p, f32x4 a, f32x4 b) {
        typename V<TO>::x8 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[i] = (TO)a[i];
            o[i + 4] = (TO)b[i];
        }
        *reinterpret_cast<typename V<TO>::x8*>(p) = o;
    }
};

// Output workgroup: 4 wavefronts = 4 consecutive heads (one 256-byte span
// of each token row) x kOutTokens tokens.  q arrives with whole-line loads
// (each wave instruction: 4 tokens x 256 B) and is staged in LDS; each wave
// then reads the MFMA B operand of its own head (16 tokens x 32 channels)
// from LDS.  The normalised rows go back through LDS so that the stores are
// whole lines too.  Loads and stores that split 128-byte lines between
// wavefronts ran at ~60% of the whole-line rate on MI355X.
template <typename T, typename TO>
__global__ __launch_bounds__(256) void linattn_out_kernel(const T* __restrict__ qkv,
                                                          const float* __restrict__ state,
                                                          TO* __restrict__ out, int N, int H,
                                                          float eps) {
    constexpr int TT = kOutTokens;
    constexpr int QR = 4 * kD + 8;            // q tile row stride (elements), padded
    constexpr int OB = 4 * kD * sizeof(TO);   // output bytes per token row of 4 heads
    constexpr int OR = OB + 16;               // out tile row stride (bytes), padded
    __shared__ __attribute__((aligned(16))) T qt[TT * QR];
    __shared__ __attribute__((aligned(16))) unsigned char ot[TT * OR];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.z;
    const int hq0 = blockIdx.x * 4;           // head quads vary fastest over the grid
    const int nhq = min(4, H - hq0);
    const int h = hq0 + wave;
    const int hs = h < H ? h : hq0;           // a missing head computes on head hq0, unstored
    const int64_t C = (int64_t)H * kD;
    const int m16 = lane & 15, kg = lane >> 4;
    const int lr = lane >> 4, lc = lane & 15;  // whole-line load: token row lr, 16-byte chunk lc
    const int lcc = lc < nhq * 4 ? lc : 0;

    // S and z of this wave's head as hi+lo 16-bit A operands: rows
    // r = 16*mb + m16, k = c = 8*kg + j; the third operand repeats z on every
    // row, so the denominator lands in the same lanes as the numerator.
    const float* S = state + (int64_t)(b * H + hs) * kState;
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

    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const int c0 = (kg & 1) ? 16 + 4 * (kg - 1) : 4 * kg;
    constexpr int LPR = OB / 16;              // lanes per output row (16 bf16/f16, 32 fp32)
    constexpr int RPI = 64 / LPR;             // output rows per store instruction
    const int sr = lane / LPR, sc = lane % LPR;
    const bool sc_ok = sc * 16 < nhq * kD * (int)sizeof(TO);

    const int n_blocks = (N + TT - 1) / TT;
    for (int tb = blockIdx.y; tb < n_blocks; tb += gridDim.y) {
        const int t_block = tb * TT;
        const int t_stop = min(N, t_block + TT);
        // Rows past t_stop re-read row t_stop-1; their results are not stored.
        u32x4 qv[TT / 16];
#pragma unroll
        for (int k = 0; k < TT / 16; ++k) {
            const int t = min(t_block + 4 * (4 * k + wave) + lr, t_stop - 1);
            const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (int64_t)hq0 * kD + lcc * 8;
            qv[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
        }
        if (tb != blockIdx.y) __syncthreads();  // the previous block's LDS reads are done
#pragma unroll
        for (int k = 0; k < TT / 16; ++k) {
            const int row = 4 * (4 * k + wave) + lr;
            *reinterpret_cast<u32x4*>(&qt[row * QR + lc * 8]) = relu_packed16(qv[k]);
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TT / 16; ++u) {
            const int row = 16 * u + m16;
            const typename V<T>::x8 bq =
                *reinterpret_cast<const typename V<T>::x8*>(&qt[row * QR + wave * kD + 8 * kg]);
            f32x4 n0 = mfma16x16x32(shi[0], bq, zero);
            n0 = mfma16x16x32(slo[0], bq, n0);
            f32x4 n1 = mfma16x16x32(shi[1], bq, zero);
            n1 = mfma16x16x32(slo[1], bq, n1);
            f32x4 dn = mfma16x16x32(zhi, bq, zero);
            dn = mfma16x16x32(zlo, bq, dn);
            const float inv = 1.0f / (dn[0] + eps);
            f32x4 lo, hi;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(n0[i] * inv),
                                                                __float_as_uint(n1[i] * inv), false, false);
                lo[i] = __uint_as_float(r[0]);
                hi[i] = __uint_as_float(r[1]);
            }
            // Even groups now hold (n0 own, n0 of the odd partner) = channels
            // 4kg..4kg+7; odd groups (n1 of the even partner, n1 own) = channels
            // 16+4(kg-1)..16+4(kg-1)+7.
            Store8<TO>::run(reinterpret_cast<TO*>(&ot[row * OR + (wave * kD + c0) * sizeof(TO)]), lo, hi);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < TT / (4 * RPI); ++k) {
            const int row = RPI * (4 * k + wave) + sr;
            const int t = t_block + row;
            if (t < t_stop && sc_ok) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(&ot[row * OR + sc * 16]);
                unsigned char* dst = reinterpret_cast<unsigned char*>(out + ((int64_t)b * N + t) * C + (int64_t)hq0 * kD);
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + sc * 16));
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
    const int h = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
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
    const int h = blockIdx.x, b = blockIdx.z;
    const int64_t C = (int64_t)H * DG;
    __shared__ float st[SS];
    __shared__ float qt[TPI][DG];
    const float* S = state + (int64_t)(b * H + h) * SS;
    for (int i = threadIdx.x; i < SS; i += 256) st[i] = S[i];
    const int n_blocks = (N + kOutTokens - 1) / kOutTokens;
    for (int tb = blockIdx.y; tb < n_blocks; tb += gridDim.y) {
    const int t_block = tb * kOutTokens;
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
}

// --------------------------------------------------------------------------
// Host side.
// --------------------------------------------------------------------------
// Token-block dimension of the output grids (the kernels loop past 65535).
unsigned out_grid_y(int N) {
    const int blocks = (N + kOutTokens - 1) / kOutTokens;
    return (unsigned)(blocks < 65535 ? blocks : 65535);
}

int64_t split_len_for(int64_t N, int64_t splits, int64_t align) {
    int64_t len = (N + splits - 1) / splits;
    return (len + align - 1) / align * align;
}

template <typename T, typename TO>
int run_mfma(const void* qkv, void* out, float* partial, float* state, int B, int N, int H,
             int splits, int split_len, float eps, hipStream_t stream) {
    hipLaunchKernelGGL((linattn_state_kernel<T>), dim3((H + 1) / 2, splits, B), dim3(256), 0,
                       stream, static_cast<const T*>(qkv), partial, N, H, split_len, splits);
    if (int rc = check_launch("linattn_state_kernel launch")) return rc;
    if (int rc = launch_reduce(partial, state, (int64_t)B * H, splits, kState, stream)) return rc;
    hipLaunchKernelGGL((linattn_out_kernel<T, TO>),
                       dim3((H + 3) / 4, out_grid_y(N), B), dim3(256), 0,
                       stream, static_cast<const T*>(qkv), state, static_cast<TO*>(out), N, H, eps);
    return check_launch("linattn_out_kernel launch");
}

template <typename T, typename TO, int DG>
int run_generic(const void* qkv, void* out, float* partial, float* state, int B, int N, int H,
                int splits, int split_len, float eps, hipStream_t stream) {
    hipLaunchKernelGGL((linattn_state_generic<T, DG>), dim3(H, splits, B), dim3(256), 0, stream,
                       static_cast<const T*>(qkv), partial, N, H, split_len, splits);
    if (int rc = check_launch("linattn_state_generic launch")) return rc;
    if (int rc = launch_reduce(partial, state, (int64_t)B * H, splits, (DG + 1) * DG, stream)) return rc;
    hipLaunchKernelGGL((linattn_out_generic<T, TO, DG>),
                       dim3(H, out_grid_y(N), B), dim3(256), 0, stream,
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
    // Aim for about 1.75 state workgroups per CU, each streaming at least 64
    // tokens (one tile) of a head pair.  A sweep of the whole pipeline on
    // MI355X (B=2/N=4096 and B=1/N=16384, 70 heads) found its minimum at 1.6-1.9
    // workgroups per CU: fewer, longer streams beat four short ones per CU by
    // 4-7%, and fewer than one per CU leaves CUs idle.
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 1;
    const int64_t groups = dim == kf::kD ? batch * ((heads + 1) / 2) : batch * heads;
    const int64_t target = (7 * (int64_t)kf::device_cu_count() + 3) / 4;
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

namespace kf {
namespace {

// Validates the request, resolves the split count and runs the three
// stages with `workspace` holding the partials and the reduced states.
int linattn_run(const void* qkv, void* out, void* workspace, int64_t workspace_bytes, int64_t batch,
                int64_t seq_len, int64_t heads, int64_t dim, int64_t splits, float eps, int in_dtype,
                int out_dtype, hipStream_t s) {
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
    // The split index is the y grid dimension (at most 65535 blocks).
    const int64_t split_len = split_len_for(seq_len, splits < 65535 ? splits : 65535, mfma ? kTT : kGT);
    const int64_t eff_splits = (seq_len + split_len - 1) / split_len;
    KF_REQUIRE(eff_splits <= 65535, KF_E_UNSUPPORTED, "linattn: too many splits");
    const int64_t state_size = (dim + 1) * dim;
    float* partial = static_cast<float*>(workspace);
    float* state = partial + batch * heads * state_size * splits;
    const int B = (int)batch, N = (int)seq_len, H = (int)heads, D = (int)dim;
    const int S = (int)eff_splits, L = (int)split_len;
    switch (in_dtype) {
        case KF_BF16: return run_in<bf16>(out_dtype, mfma, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
        case KF_F16: return run_in<f16>(out_dtype, mfma, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
        default: return run_in<float>(out_dtype, false, D, qkv, out, partial, state, B, N, H, S, L, eps, s);
    }
}

// Per-device address of `scratch`, resolved once per device with that
// device current (each GPU holds its own copy at its own address).
int scratch_for_current_device(void** ptr) {
    static std::mutex lock;
    static void* addr[64] = {};
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return hip_failure(err, "linattn: hipGetDevice");
    KF_REQUIRE(dev >= 0 && dev < 64, KF_E_UNSUPPORTED, "linattn: device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> guard(lock);
    if (!addr[dev]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_failure(err, "linattn: hipGetSymbolAddress(scratch)");
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return KF_OK;
}

}  // namespace
}  // namespace kf

extern "C" int kf_linattn_fwd(const void* qkv, void* out, void* workspace, int64_t workspace_bytes,
                              int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                              int64_t splits, float eps, int in_dtype, int out_dtype,
                              kf_stream_t stream) {
    return kf::linattn_run(qkv, out, workspace, workspace_bytes, batch, seq_len, heads, dim, splits, eps,
                           in_dtype, out_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int64_t kf_linattn_noalloc_max_bytes(void) { return kLinattnScratchBytes; }

extern "C" int kf_linattn_fwd_noalloc(const void* qkv, void* out, int64_t batch, int64_t seq_len,
                                      int64_t heads, int64_t dim, int64_t splits, float eps, int in_dtype,
                                      int out_dtype, kf_stream_t stream) {
    using namespace kf;
    // Size check first, so an oversized request fails before any device call.
    int64_t eff = splits <= 0 ? kf_linattn_default_splits(batch, heads, dim, seq_len) : splits;
    if (eff > seq_len && seq_len > 0) eff = seq_len;
    const int64_t need = kf_linattn_workspace_bytes(batch, heads, dim, eff);
    KF_REQUIRE(need <= kLinattnScratchBytes, KF_E_WORKSPACE,
               "linattn noalloc: %lld bytes of scratch needed for B=%lld H=%lld D=%lld splits=%lld, "
               "the static scratch holds %lld; use fewer splits or kf_linattn_fwd with a workspace",
               (long long)need, (long long)batch, (long long)heads, (long long)dim, (long long)eff,
               (long long)kLinattnScratchBytes);
    if (batch <= 0 || seq_len <= 0 || heads <= 0)
        return linattn_run(qkv, out, nullptr, 0, batch, seq_len, heads, dim, eff, eps, in_dtype, out_dtype,
                           static_cast<hipStream_t>(stream));
    void* ws = nullptr;
    if (int rc = scratch_for_current_device(&ws)) return rc;
    return linattn_run(qkv, out, ws, kLinattnScratchBytes, batch, seq_len, heads, dim, eff, eps, in_dtype,
                       out_dtype, static_cast<hipStream_t>(stream));
}
