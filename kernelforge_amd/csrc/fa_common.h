// Device helpers shared by the FlashAttention kernels (forward / JVP in
// fa_jvp.hip, backward in fa_bwd.hip) for gfx950: workgroup shapes, the
// HBM -> LDS tile copies (global_load_lds), the XOR chunk swizzle and the LDS
// operand reads for v_mfma_f32_16x16x32, and 16-lane-group row reductions.
//
// The HBM -> LDS copies are issued from inline assembly.  The compiler models
// a global_load_lds it emits itself as a FLAT access of both VMEM and LDS and,
// while one is outstanding, turns the next wait for any LDS read or global
// load into vmcnt(0) lgkmcnt(0): the wavefront then stalls until the copy of
// the NEXT tile has landed, which defeats the double buffering.  Issued from
// assembly, the copies are invisible to that model; the kernels wait for them
// explicitly (wait_vmem) before the barrier that publishes a buffer, and the
// "memory" clobber keeps the compiler from moving LDS accesses across them.
#pragma once

#include <type_traits>

#include "kf_common.h"

namespace kf {
namespace {

enum FaMode { FA_FWD = 0, FA_FWD_JVP = 1, FA_JVP = 2 };

// Byte address of an LDS location, as the M0 register of an LDS copy takes it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// HBM -> LDS copy of 16 bytes per lane: lane i's bytes at `src` land at LDS
// address m0 + 16 i.  m0 must be wavefront-uniform.  The s_nop covers the
// wait state an LDS copy needs after M0 is written.
__device__ __forceinline__ void lds_copy16(const void* src, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// The same from a wavefront-uniform base (SGPRs) plus a per-lane 32-bit byte
// offset: lane i's 16 bytes at sbase + voff land at m0 + 16 i.  The address
// arithmetic per instruction is then scalar.
__device__ __forceinline__ void lds_copy16_sbase(const void* sbase, uint32_t voff, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// The same with 4 bytes per lane (lane i's dword lands at m0 + 4 i).
__device__ __forceinline__ void lds_copy4(const void* src, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// 4 bytes per lane from a wavefront-uniform base plus a per-lane byte offset.
__device__ __forceinline__ void lds_copy4_sbase(const void* sbase, uint32_t voff, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// Workgroup shape per padded head dim.  Up to D = 128: 8 wavefronts x 16
// query rows, 64-key tiles, two wavefronts per SIMD.  D = 256 doubles the Q and
// accumulator registers per row: 4 wavefronts x 16 rows, 32-key tiles (the
// double-buffered K/V/tK/tV tiles still take 128 KiB of LDS), one wavefront
// per SIMD with its 512 registers.
template <int DP> struct FaTile {
    static constexpr int BQ = DP > 128 ? 64 : 128;  // query rows per workgroup
    static constexpr int BK = DP > 128 ? 32 : 64;   // keys per tile
    static constexpr int WAVES = BQ / 16;           // 16 query rows each
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int HALVES = BK / 32;          // 32-key halves per tile
    static constexpr int OCC = DP > 128 ? 1 : 2;    // wavefronts per SIMD
};
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // lazy rescale step of the rescaling scan (log2)
// The JVP-from-LSE mode writes tO = G/l - (r/l) O with the cached O only for
// rows where |r/l| * max(max|O|, 1) is at most this: O's rounding (a few
// 2^-9 relative) then moves tO by at most ~2^-8 of it, about a fifth of the
// 2e-2 tolerance (a CPU emulation of every rounding point over D = 32-128,
// N = 64-2048 and scales 0.05-1.3 measured at most 0.24 of it).  At scale
// 1/sqrt(D) on unit-normal inputs the product stays below ~0.4 at 4096 keys
// (~0.8 at 256-512 keys, where fewer keys average less).
constexpr float kCachedOBound = 1.0f;

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

// Physical 16-byte chunk = logical chunk ^ swz(row), for CH chunks per row.
// Chosen (by enumerating the XOR-linear maps of row % 16 and checking them
// against measured LDS conflict counts) so that neither the ds_read_b128 of a
// K block (16 consecutive rows at one logical chunk) nor the
// ds_read_b64_tr_b16 of a V^T operand (8 consecutive rows x an aligned pair of
// chunks) has bank conflicts; swz depends on row % 16 only.  For 32 chunks
// (512-byte rows) the 16-chunk map is also conflict-free for both patterns in
// a 64-bank model of the LDS.
template <int CH> __device__ __forceinline__ int swz(int r) {
    if constexpr (CH == 16 || CH == 32) return (r & 15) ^ ((r & 1) * 12);
    else if constexpr (CH == 8) return (r & 7) ^ ((r & 1) << 2);
    else return ((r >> 1) & 1) | ((((r >> 1) ^ (r >> 2)) & 1) << 1);
}

// Async copy of one [BK][DP] tile (keys k0.., one kv head) into LDS.  A tile
// is NI = BK*DP/512 copy instructions of 64 lanes x 16 B (RPI rows each);
// wavefront w of the W issuing ones issues instructions w, w + W, ...
template <typename T, int DP, int W = FaTile<DP>::WAVES>
__device__ __forceinline__ void load_tile(T* tile, const T* g, int64_t row_stride, int keys_valid,
                                          int D, int wave, int lane) {
    constexpr int CH = DP / 8;
    constexpr int RPI = 64 / CH;
    constexpr int NI = FaTile<DP>::BK / RPI;
#pragma unroll
    for (int j = 0; j < (NI + W - 1) / W; ++j) {
        const int i = wave + j * W;
        if (NI % W == 0 || i < NI) {
            const int row0 = i * RPI;
            const int row = row0 + lane / CH;
            const int chunk = (lane % CH) ^ swz<CH>(row);
            const void* src = (row < keys_valid && chunk * 8 < D)
                                   ? static_cast<const void*>(g + row * row_stride + chunk * 8)
                                   : static_cast<const void*>(g_zero16);
            lds_copy16(src, __builtin_amdgcn_readfirstlane(lds_addr(tile + row0 * DP)));
        }
    }
}

// Byte offset, within a full tile, of the 16-byte chunk lane `lane` copies.
// The rows a lane copies are wave*RPI + lane/CH plus multiples of W*RPI;
// when that is a multiple of 16 (full_tile_shortcut), their swizzle (a
// function of row % 16) is the same for every instruction and one offset
// serves them all.
template <int DP, int W = FaTile<DP>::WAVES> constexpr bool full_tile_shortcut() {
    return (W * (64 / (DP / 8))) % 16 == 0;
}
template <typename T, int DP>
__device__ __forceinline__ uint32_t full_tile_lane_offset(int64_t row_stride, int wave, int lane) {
    constexpr int CH = DP / 8;
    constexpr int RPI = 64 / CH;
    const int row = wave * RPI + lane / CH;
    const int chunk = (lane % CH) ^ swz<CH>(row);
    return (uint32_t)(((int64_t)(lane / CH) * row_stride + chunk * 8) * (int64_t)sizeof(T));
}

// Async copy of a tile whose 64 rows are all valid and whose rows hold exactly
// DP elements: a uniform base per instruction plus one per-lane offset.  With
// SBASE the base stays in SGPRs (scalar address arithmetic, LDS addresses from
// one conversion of the tile pointer); otherwise each instruction forms a
// 64-bit per-lane address.  SBASE trades VALU for SALU instructions: 0.5-1.5%
// faster for the JVP modes and the backward at B=2, H=16, N=4096, D=128 on
// MI355X, 1.5% slower for the forward, whose loop is VALU-bound already.
template <typename T, int DP, int W = FaTile<DP>::WAVES, bool SBASE = true>
__device__ __forceinline__ void load_tile_full(T* tile, const T* g, int64_t row_stride, uint32_t voff,
                                               int wave) {
    constexpr int CH = DP / 8;
    constexpr int RPI = 64 / CH;
    constexpr int NI = FaTile<DP>::BK / RPI;
    static_assert(full_tile_shortcut<DP, W>(), "one lane offset serves every instruction");
    const uint32_t t0 = SBASE ? __builtin_amdgcn_readfirstlane(lds_addr(tile)) : 0u;
#pragma unroll
    for (int j = 0; j < (NI + W - 1) / W; ++j) {
        const int i = wave + j * W;
        if (NI % W == 0 || i < NI) {
            const int row0 = i * RPI;
            if constexpr (SBASE) {
                lds_copy16_sbase(g + (int64_t)row0 * row_stride, voff, t0 + row0 * DP * (uint32_t)sizeof(T));
            } else {
                const char* src = reinterpret_cast<const char*>(g + (int64_t)row0 * row_stride) + voff;
                lds_copy16(src, __builtin_amdgcn_readfirstlane(lds_addr(tile + row0 * DP)));
            }
        }
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

// A operand V^T[d][k] of the 32-key step kk and 16-wide d block db: lane l
// (g = l/16) holds d = 16*db + l%16 and keys 32*kk + 4*g + 0..3 (elements
// 0..3) and 32*kk + 16 + 4*g + 0..3 (elements 4..7).  In ds_read_b64_tr_b16
// lanes 4q..4q+3 of each 16-lane group address row q's 16 elements; lane j of
// the group then receives element j of rows 0..3.
template <typename T, int DP>
__device__ __forceinline__ typename V<T>::x8 vt_operand(const T* tile, int kk, int db, int lane) {
    const int g = lane >> 4, j16 = lane & 15;
    const int row = 32 * kk + 4 * g + (j16 >> 2);
    const int d = 16 * db + 4 * (j16 & 3);
    const typename V<T>::x4 lo = lds_read_tr(tr_addr<T, DP>(tile, row, d));
    const typename V<T>::x4 hi = lds_read_tr(tr_addr<T, DP>(tile, row + 16, d));
    typename V<T>::x8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r[j] = lo[j];
        r[j + 4] = hi[j];
    }
    return r;
}

// ---------------------------------------------------------------------------
// Panel layout of [64][DP] LDS tiles of the backward kernels (up to D = 128):
// DP/32 panels of [64 rows][32 elements] (64-byte rows); element (r, d) sits
// in panel d/32, row r, 16-byte chunk ((d % 32) / 8) ^ pswz(r), element d % 8,
// with pswz(r) = (r1 ^ r2 ^ r3, r2) for row bits r1..r3.  Every operand read
// is then one per-lane base plus a compile-time offset, where the row-swizzled
// layout above needs a separate lane offset per 16-byte column, which the
// compiler keeps in registers (16-35 VGPRs per kernel).  One copy instruction
// fills 16 rows of one panel (1024 contiguous LDS bytes) from 64-byte row
// segments.  The forward kernels ran 0.5-2% slower with this layout, and
// keep the row layout.  pswz was found by enumerating the XOR-linear maps of the
// row bits: with it neither the 16-byte reads (16 rows at one logical chunk)
// nor the transposing reads (rows 4g + q, 32 bytes each) meet a bank conflict
// in any of the LDS models the row swizzle is conflict-free in: 128 banks
// with 32-lane passes for 16-byte reads and one pass for 8-byte reads (the
// one the hardware counters agree with: a map that is clean only in the two
// narrower models measured two conflict cycles per read), 64 banks with 16-
// and 32-lane passes, and 32 banks with 8- and 16-lane passes.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int pswz(int r) {
    const int r1 = (r >> 1) & 1, r2 = (r >> 2) & 1, r3 = (r >> 3) & 1;
    return ((r1 ^ r2 ^ r3) << 1) | r2;
}

template <typename T, int DP>
__device__ __forceinline__ void load_panels(T* tile, const T* g, int64_t row_stride, int rows_valid, int D,
                                            int wave, int lane) {
    constexpr int NI = DP / 8, W = FaTile<DP>::WAVES;
    const int r16 = lane >> 2;
    const int cs = (lane & 3) ^ pswz(r16);
#pragma unroll
    for (int j = 0; j < (NI + W - 1) / W; ++j) {
        const int i = wave + j * W;
        if (NI % W == 0 || i < NI) {
            const int rb = i & 3, pnl = i >> 2;
            const int row = 16 * rb + r16;
            const int d = 32 * pnl + 8 * cs;
            const void* src = (row < rows_valid && d < D) ? static_cast<const void*>(g + row * row_stride + d)
                                                           : static_cast<const void*>(g_zero16);
            lds_copy16(src, __builtin_amdgcn_readfirstlane(lds_addr(tile + pnl * 64 * 32 + 16 * rb * 32)));
        }
    }
}

// Byte offset of the 16-byte chunk lane `lane` copies within each 16-row
// block of a panel (the same for every copy instruction of a full tile).
template <typename T>
__device__ __forceinline__ uint32_t panel_lane_offset(int64_t row_stride, int lane) {
    const int r16 = lane >> 2;
    return (uint32_t)(((int64_t)r16 * row_stride + 8 * ((lane & 3) ^ pswz(r16))) * (int64_t)sizeof(T));
}

// A tile whose 64 rows are all valid and hold exactly DP elements: a uniform
// base per instruction plus the one lane offset, the base in SGPRs with SBASE
// (as load_tile_full).
template <typename T, int DP, bool SBASE = true>
__device__ __forceinline__ void load_panels_full(T* tile, const T* g, int64_t row_stride, uint32_t voff, int wave) {
    constexpr int NI = DP / 8, W = FaTile<DP>::WAVES;
    const uint32_t t0 = __builtin_amdgcn_readfirstlane(lds_addr(tile));
#pragma unroll
    for (int j = 0; j < (NI + W - 1) / W; ++j) {
        const int i = wave + j * W;
        if (NI % W == 0 || i < NI) {
            const int rb = i & 3, pnl = i >> 2;
            const uint32_t m0 = t0 + (uint32_t)((pnl * 64 * 32 + 16 * rb * 32) * sizeof(T));
            const T* src = g + (int64_t)(16 * rb) * row_stride + 32 * pnl;
            if constexpr (SBASE)
                lds_copy16_sbase(src, voff, m0);
            else
                lds_copy16(reinterpret_cast<const char*>(src) + voff, m0);
        }
    }
}

// Per-lane element offsets of the operand reads of a panel-layout tile.
struct PanelLane {
    int nat;  // 16-byte read: row l%16 (plus a multiple of 16), logical chunk l/16 of a panel
    int tr0;  // transposing read (see vt_operand): row 4g + q, even chunk pair of a panel
    __device__ __forceinline__ explicit PanelLane(int lane) {
        const int j16 = lane & 15, g = lane >> 4;
        nat = j16 * 32 + 8 * (g ^ pswz(j16));
        const int trq = 4 * g + (j16 >> 2);
        tr0 = trq * 32 + 8 * (((j16 >> 1) & 1) ^ pswz(trq)) + 4 * (j16 & 1);
    }
};

// row_chunk(tile, row16 + l%16, 4*ds + l/16) of a panel-layout tile.
template <typename T>
__device__ __forceinline__ typename V<T>::x8 panel_chunk(const T* tile, const PanelLane& pl, int row16, int ds) {
    return *reinterpret_cast<const typename V<T>::x8*>(tile + ds * 64 * 32 + row16 * 32 + pl.nat);
}

// vt_operand(tile, kk, db, lane) of a panel-layout tile; the odd chunk pair
// of a panel is the even one's physical chunk ^ 2 (element offset ^ 16).
template <typename T>
__device__ __forceinline__ typename V<T>::x8 panel_vt_operand(const T* tile, const PanelLane& pl, int kk, int db) {
    const T* base = tile + (db >> 1) * 64 * 32 + 32 * kk * 32 + ((db & 1) ? (pl.tr0 ^ 16) : pl.tr0);
    const typename V<T>::x4 lo = lds_read_tr(base);
    const typename V<T>::x4 hi = lds_read_tr(base + 16 * 32);
    typename V<T>::x8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r[j] = lo[j];
        r[j + 4] = hi[j];
    }
    return r;
}

// Causal grids, where a head's tiles are numbered longest first: the logical
// block numbers of one XCD (a contiguous range, consecutive tiles of a head)
// dealt round-robin over that range's heads, so that the XCD starts every
// head's longest tile before any head's shorter ones (longest-processing-time
// order; one head after another leaves the longest tiles of the last heads
// for the end).  The XCD keeps the same heads.  Applies when every XCD range
// holds whole heads; otherwise the order is left as it is.
__device__ __forceinline__ int causal_tile_order(int logical, int n_tiles) {
    const int nblk = gridDim.x;
    if (nblk & 7) return logical;
    const int per = nblk >> 3;
    if (per % n_tiles) return logical;
    const int heads = per / n_tiles, s = logical % per;
    return logical - s + (s % heads) * n_tiles + s / heads;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Packed 16-bit pairs: round-to-nearest-even conversion of two floats and a
// two-term fp32 dot product with (1, 1), used to sum the rounded values.
template <typename T> struct Pk;
template <> struct Pk<bf16> {
    typedef __bf16 x2 __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ unsigned cvt(float a, float b) {
        const f32x2 v = {a, b};
        return __builtin_bit_cast(unsigned, __builtin_convertvector(v, x2));
    }
    static __device__ __forceinline__ float sum_into(unsigned pk, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(x2, pk),
                                               __builtin_bit_cast(x2, 0x3f803f80u), acc, false);
    }
};
template <> struct Pk<f16> {
    typedef _Float16 x2 __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ unsigned cvt(float a, float b) {
        const f32x2 v = {a, b};
        return __builtin_bit_cast(unsigned, __builtin_convertvector(v, x2));
    }
    static __device__ __forceinline__ float sum_into(unsigned pk, float acc) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(x2, pk), __builtin_bit_cast(x2, 0x3c003c00u),
                                      acc, false);
    }
};

// Wait until this thread's global->LDS copies (and any other vector memory
// operation) have completed (vmcnt = 0); the LDS and scalar counters are left
// alone.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Reduce x over the four lanes l%16 + 16*g (g = 0..3) that share a query row.
// v_permlane16_swap / v_permlane32_swap exchange the odd 16-lane (32-lane)
// groups of their first operand with the even groups of the second; with both
// operands x, op(r0, r1) combines each lane with its partner in the same
// operand order in every lane, so all four lanes end with the same value.
__device__ __forceinline__ float row_sum4(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_max4(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

}  // namespace
}  // namespace kf
