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
// D = 32 with bf16/f16 input runs one fused kernel (linattn_fused_kernel):
// each workgroup streams one sequence split of two adjacent heads, builds
// the split's partial state on MFMA, waits at its (batch, head pair) group's
// counter for the other splits, sums the group's partials in split order
// (deterministic, no atomics on data) and contracts the state with the
// split's relu(q) on MFMA.  Counters live in the workspace's control words.
// Other head dims (128 % D == 0) and fp32 input take a VALU path in three
// launches (split states, fixed-order split reduction, output).
#include "kf_common.h"

#include <atomic>
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
constexpr int kTT = 128;            // tokens per tile (state and output phases)
constexpr int kWaves = 8;           // wavefronts per fused workgroup: (head of the pair) x (32-token quarter)
constexpr int kThreads = 64 * kWaves;
// Tiles held in registers (in flight) per thread: three of each.  Deeper
// rings (4-7) ran 2-20% slower on MI355X, as did 16-wave workgroups and
// wave-private pipelines without the per-tile barrier.
constexpr int KV_RING = 3;
constexpr int Q_RING = 3;
constexpr int kOutTokens = 64;      // tokens per output workgroup of the generic path
constexpr int kSpinLimit = 1 << 20; // polls of the group counter before giving up

// --------------------------------------------------------------------------
// Control words at the start of the workspace (uint32):
//   [0]          ticket counter (start order of the fused kernel's workgroups)
//   [1]          error word: 1 = a group barrier timed out, 2 = control words
//                not zero on entry (a ticket beyond the grid, or a group
//                counter above its member count)
//   [64 + 64g]   arrivals of group g (one (batch, head pair)) at its barrier
//   [64 + 64g+1] departures of group g from it (each group's words share no
//                cache line with another group's, so polls do not collide)
// The region has a fixed size (kCtrlBytes), so a workspace reused for other
// shapes keeps its control words apart from its partials.  They must be zero
// before the first call; every call returns them to zero.
// --------------------------------------------------------------------------
constexpr int kCtrlHeader = 64;
constexpr int kCtrlStride = 64;            // words per group: each group's counters own a 256-byte line
constexpr int kMaxGroupsPerLaunch = 4096;  // larger problems take several launches
constexpr int64_t kCtrlBytes = (int64_t)(kCtrlHeader + kCtrlStride * kMaxGroupsPerLaunch) * 4;
static_assert(kCtrlBytes % 256 == 0, "partials stay 256-byte aligned");

// Workgroup barrier that leaves global loads in flight.  __syncthreads()
// also waits for every outstanding global load (vmcnt(0)), which would drain
// the register prefetch at each tile; here only this wave's LDS traffic is
// completed (lgkmcnt(0)) before s_barrier.  The empty asm statements keep
// the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_keep_loads() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt untouched
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS byte offsets.  The swizzles below were found by enumerating the
// XOR-linear maps of the row bits against every access pattern of the tiles,
// in three LDS bank models: 128 banks with 32-lane passes for 16-byte
// accesses and one pass for 8-byte ones (the model the hardware's conflict
// counter agrees with), 64 banks with 16- and 32-lane passes, and 32 banks
// with 8- and 16-lane passes.
//
// K/V tile: one 256-byte row per token holding the pair's 64 K channels and
// 64 V channels: 16-byte chunk L = 8*part + ch/8 (part 0 = K, 1 = V) sits at
// L ^ kvswz(tok), kvswz(t) = (t0 ^ t3, t1, t0, 0) in chunk bits 3..0.  A
// 16-lane store group (one token's K and V) and a transposing read (rows
// 4g + q, 8 rows x 64 bytes) meet no conflict.
__device__ __forceinline__ int kvswz(int t) {
    return (((t ^ (t >> 3)) & 1) << 3) | (((t >> 1) & 1) << 2) | ((t & 1) << 1);
}
__device__ __forceinline__ int kv_off(int tok, int part, int ch) {
    return tok * 256 + (((8 * part + (ch >> 3)) ^ kvswz(tok)) << 4) + (ch & 7) * 2;
}
// q and 16-bit output tiles: 128-byte rows (the pair's 64 channels), 16-byte
// chunk index xor rswz(row) = (r0 ^ r3, r1 ^ r2, r2) in chunk bits 2..0: 16
// consecutive rows at one chunk (an MFMA operand read), 16 rows at the chunk
// pairs the output staging writes, and 2 rows x 8 chunks (a whole-line
// access) meet no conflict.
__device__ __forceinline__ int rswz(int r) {
    return (((r ^ (r >> 3)) & 1) << 2) | ((((r >> 1) ^ (r >> 2)) & 1) << 1) | ((r >> 2) & 1);
}
__device__ __forceinline__ int r128_off(int row, int chunk) { return row * 128 + ((chunk ^ rswz(row)) << 4); }
// fp32 output tile: 256-byte rows, chunk index xor (row & 15).
__device__ __forceinline__ int r256_off(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }

template <typename TO> struct OutTile {
    static constexpr int ROW = 2 * kD * (int)sizeof(TO);   // bytes per token row of the pair
    static constexpr int CHUNKS = ROW / 16;
    __device__ static int off(int row, int chunk) {
        if constexpr (ROW == 128) return r128_off(row, chunk);
        else return r256_off(row, chunk);
    }
};

struct FusedParams {
    const void* qkv;
    void* out;
    float* partial;     // [B][H][S][D+1][D]
    unsigned* ctrl;
    int N, H, npairs, S, split_len;
    int g0;             // first group (batch * npairs + pair) of this launch
    int total;          // workgroups of this launch: groups * S
    int use_ticket;     // 1: number workgroups by ticket (more than the device holds at once)
    int spin_limit;     // polls of a group counter before a member gives up
    float eps;
};

// Global -> register staging of one 128-token K/V tile of a head pair: 4 x 16 B
// per thread.  Chunk c = i*512 + tid: token c/16, part (c/8)%2 (0 = K, 1 = V),
// 16-byte segment c%8 of the pair's 128-byte span, so every load instruction
// of a wave covers 4 tokens x 2 whole 128-byte lines.  Addresses are clamped
// into the split (token t_end-1) and onto a present head, so the number of
// loads never depends on the data; the clamped duplicates are zeroed when the
// tile is stored to LDS.
template <typename T>
__device__ __forceinline__ void kv_gload(u32x4 (&reg)[4], const T* __restrict__ qkv, int64_t b, int N,
                                         int64_t C, int h0, int nh, int t0, int t_end, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = i * kThreads + tid;
        const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
        const int t = min(t0 + tok, t_end - 1);
        const int sg = seg < nh * 4 ? seg : seg - 4;
        const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (1 + part) * C + (int64_t)h0 * kD + sg * 8;
        reg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
}

// One 128-token q tile of the pair: 2 x 16 B per thread, chunk c = i*512+tid:
// token c/8, segment c%8 (whole 128-byte lines), clamped like kv_gload.
template <typename T>
__device__ __forceinline__ void q_gload(u32x4 (&reg)[2], const T* __restrict__ qkv, int64_t b, int N,
                                        int64_t C, int h0, int nh, int t0, int t_end, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = i * kThreads + tid;
        const int tok = c >> 3, seg = c & 7;
        const int t = min(t0 + tok, t_end - 1);
        const int sg = seg < nh * 4 ? seg : seg - 4;
        const T* src = qkv + ((int64_t)b * N + t) * 3 * C + (int64_t)h0 * kD + sg * 8;
        reg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
}

// Stores of the numerator pair (n0: channels 4kg..4kg+3, n1: 16+4kg..) after
// v_permlane16_swap has exchanged n1 of the even 16-lane groups with n0 of
// the odd ones: an even group then holds channels 4kg..4kg+7, an odd group
// 16+4(kg-1)..16+4(kg-1)+7, so each lane writes 8 consecutive channels.
template <typename TO>
__device__ __forceinline__ void store8_lds(unsigned char* tile, int row, int ch0, f32x4 a, f32x4 b) {
    if constexpr (sizeof(TO) == 4) {
        *reinterpret_cast<f32x4*>(tile + OutTile<TO>::off(row, ch0 / 4)) = a;
        *reinterpret_cast<f32x4*>(tile + OutTile<TO>::off(row, ch0 / 4 + 1)) = b;
    } else {
        typename V<TO>::x8 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[i] = (TO)a[i];
            o[i + 4] = (TO)b[i];
        }
        *reinterpret_cast<typename V<TO>::x8*>(tile + OutTile<TO>::off(row, ch0 / 8)) = o;
    }
}

// Barrier of the workgroups of one group (the `members` sequence splits of one
// (batch, head pair)): every writer's partial has completed at the device
// coherence point (device-coherent stores, then a wait for them) before the
// workgroup barrier that precedes this call; thread 0 counts the arrival,
// polls until all members have arrived (at most `spin_limit` polls, then it
// sets the error word and goes on, so no wave can wait forever), counts the
// departure, and the last member to leave resets both counters to zero for
// the next call.  Returns true, in every thread, when the wait gave up: the
// partials are then incomplete and the caller writes NaN instead of a result.  The members then read the partials with plain loads (see
// phase 2 for why they are current).  Agent-scope fences are not used: their L2 write-backs and
// invalidations, once per workgroup, cost more than the rest of the kernel
// on MI355X (write-backs ~67 us, invalidations ~10 us of a 37 us launch at
// B=2, H=70, N=4096).
__device__ __forceinline__ bool group_barrier(unsigned* ctrl, int g, unsigned members, int spin_limit,
                                              int* late_flag) {
    if (threadIdx.x == 0) {
        unsigned* arrive = ctrl + kCtrlHeader + kCtrlStride * g;
        unsigned* depart = arrive + 1;
        __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int polls = 0, late = 0;
        unsigned seen;
        while ((seen = __hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < members) {
            if (++polls > spin_limit) {
                __hip_atomic_store(ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                late = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
        const unsigned departed = __hip_atomic_fetch_add(depart, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (departed == members - 1) {
            __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(depart, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // Counts no valid call produces (at most `members` arrivals and
        // departures per call, both reset by the last to leave): the control
        // words were not zero on entry.  Reported like a stale ticket; the
        // partials may be incomplete, so this member writes NaN.
        if (seen > members || departed >= members) {
            __hip_atomic_store(ctrl + 1, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            late = 1;
        }
        *late_flag = late;
    }
    __syncthreads();
    return *late_flag != 0;
}

// --------------------------------------------------------------------------
// The fused kernel (D = 32, 16-bit input).  One workgroup per (batch, head
// pair, sequence split).  A launch whose workgroups all fit on the device at
// once (the default split counts keep it so) numbers them by workgroup
// index: alone on the device, every member a waiting workgroup needs then
// holds a slot or gets one, whatever order the hardware starts them in.
// (Beside other launches that hold slots, index numbering relies on the
// hardware starting a launch's workgroups in index order, as MI355X's
// dispatcher does, to keep complete groups resident; ticket numbering does
// not.  Out of order and oversubscribed, members could wait on each other
// until the poll limit, and would then report it.)  A larger launch numbers
// them by a ticket taken at start, so the members of a group start
// consecutively: a member can only wait for members that started before it
// or will start next, and at most one group is partly started at any time.
// Workgroups of fully started groups wait for nobody who has not started, so
// they finish and free their slots; the partly started group's waiting
// members hold at most S - 1 slots, and the host keeps S within the slots the
// device offers (invariant 3 below), so its remaining members always find a
// slot and every wait ends.  (The ticket is one atomic counter for the whole
// launch: 210 workgroups taking it cost ~2 us at B=2, H=70, N=4096 on MI355X,
// so the smaller launches skip it.)  Only other work holding the device's
// slots for longer than the poll limit can make a member give up (then it
// reports it: see group_barrier).
//   Phase 1: stream the split's K and V (three 128-token tiles in flight in
//            registers, LDS double buffer), accumulate the partial state
//            S = V^T relu(K) with v_mfma_f32_32x32x16 and z = sum relu(K),
//            write it to the workspace.
//   Barrier: wait for the group's other splits.
//   Phase 2: sum the group's partials in split order (fixed order: the same
//            state in every member, deterministic), then stream the split's
//            q tiles: out = S relu(q) / (z . relu(q) + eps) on
//            v_mfma_f32_16x16x32 with S and z held as hi+lo 16-bit pairs,
//            rows leaving through LDS as whole-line stores.
// Waves: (hw, th) = (head of the pair, 32-token quarter of each tile).
// Where the time goes (MI355X, B=2, H=70, N=4096, 3 splits, per-workgroup
// timestamps, medians): phase 1 11.5 us, the hand-over between the phases
// 4.6 us (combining the quarters and storing the partial 1.9, the group wait
// 1.3, summing the partials 1.4: round trips to the coherence point that all
// workgroups make at once), phase 2 9.6 us; the last workgroup ends 2.3 us
// after the median one.
// OT (fp32 output only) writes out[b][h*D + r][t] -- LiteLA.attn_matmul's
// [B, h, d, N] result -- instead of out[b][t][h*D + r].
//
// Memory-model invariants the group barrier and phase 2 rely on (any change
// to either phase must keep them):
//   1. Partials are written only with device-coherent (agent-scope) stores,
//      and each writer waits for them (vmcnt(0)) before its workgroup
//      barrier, which precedes its arrival count.
//   2. Nothing reads a partial before the group barrier in a launch, and
//      each (batch, head, split) partial starts on its own 128-byte line
//      (kState floats are a whole number of lines), so no cache can hold a
//      line of another group's or an earlier launch's partial: caches are
//      invalidated at every kernel start.  Phase 2's plain loads therefore
//      miss to the coherence point and see the stores of invariant 1.
//   3. A group has at most as many members as can be resident at once
//      (the host clamps the split count to the kernel's occupancy times the
//      CU count), so the members a waiting workgroup needs can always start.
// --------------------------------------------------------------------------
static_assert(kState * 4 % 128 == 0, "each partial starts on its own cache line");
template <typename T, typename TO, bool OT = false>
__global__ __launch_bounds__(kThreads) void linattn_fused_kernel(FusedParams p) {
    static_assert(!OT || sizeof(TO) == 4, "the transposed output is fp32");
    constexpr int KV_BYTES = 2 * kTT * 256;                          // double-buffered K/V tile
    constexpr int Q_BYTES = kTT * 128;
    constexpr int O_BYTES = kTT * OutTile<TO>::ROW;
    constexpr int P2_BYTES = 2 * (Q_BYTES + O_BYTES);                // double-buffered q and out tiles
    constexpr int LDS_BYTES = KV_BYTES > P2_BYTES ? KV_BYTES : P2_BYTES;
    static_assert(LDS_BYTES >= 2 * 3 * 64 * 17 * 4, "combine buffer fits");
    __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
    __shared__ int sh_ticket;
    __shared__ int sh_late;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int ticket = blockIdx.x;
    if (p.use_ticket) {
        if (tid == 0) {
            const int t = (int)__hip_atomic_fetch_add(p.ctrl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (t == p.total - 1) __hip_atomic_store(p.ctrl, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sh_ticket = t;
        }
        __syncthreads();
        ticket = sh_ticket;
        if (ticket >= p.total) {
            // Control words that were not zero on entry: flag it and touch
            // nothing (the group barriers of the other workgroups then time out).
            if (tid == 0) __hip_atomic_store(p.ctrl + 1, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    const int g = ticket / p.S, s = ticket - g * p.S;  // group within this launch, split
    const int gg = p.g0 + g;
    const int b = gg / p.npairs, pair = gg - b * p.npairs;
    const T* __restrict__ qkv = static_cast<const T*>(p.qkv);
    const int N = p.N, H = p.H;
    const int64_t C = (int64_t)H * kD;
    const int h0 = 2 * pair;
    const int nh = min(2, H - h0);
    const int t_begin = s * p.split_len;          // < N: the host sizes the splits
    const int t_end = min(N, t_begin + p.split_len);
    const int ntile = (t_end - t_begin + kTT - 1) / kTT;  // >= 1
    const int hw = wave & 1, th = wave >> 1;
    const int G = lane >> 4, j16 = lane & 15;

    // ---------------- Phase 1: partial state of this split ----------------
    // ReLU on K only and zeros past t_end, as masks (no divergent branches).
    const unsigned sign_bits = ((tid >> 3) & 1) ? 0u : 0x00010001u;  // part = (c/8)%2 = (tid/8)%2
    auto kv_store = [&](const u32x4 (&reg)[4], int buf, int t0) {
        unsigned char* base = lds + buf * (kTT * 256);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * kThreads + tid;
            const int tok = c >> 4, part = (c >> 3) & 1, seg = c & 7;
            const unsigned keep = t0 + tok < t_end ? 0xffffffffu : 0u;
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const unsigned neg = (reg[i][e] >> 15) & sign_bits;
                v[e] = reg[i][e] & ~(neg * 0xffffu) & keep;
            }
            *reinterpret_cast<u32x4*>(base + kv_off(tok, part, seg * 8)) = v;
        }
    };
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    float zsum = 0.f;
    auto accumulate = [&](int buf) {
        const unsigned char* base = lds + buf * (kTT * 256);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int row = 32 * th + 16 * ks + 8 * (G >> 1) + (j16 >> 2);
            const int col = hw * 32 + 16 * (G & 1) + 4 * (j16 & 3);
            const T* v0 = reinterpret_cast<const T*>(base + kv_off(row, 1, col));
            const T* v1 = reinterpret_cast<const T*>(base + kv_off(row + 4, 1, col));
            const T* k0 = reinterpret_cast<const T*>(base + kv_off(row, 0, col));
            const T* k1 = reinterpret_cast<const T*>(base + kv_off(row + 4, 0, col));
            typename V<T>::x4 a0 = lds_read_tr(v0), a1 = lds_read_tr(v1);
            typename V<T>::x4 b0 = lds_read_tr(k0), b1 = lds_read_tr(k1);
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
    {
        // Tile j is loaded into register set j % KV_RING and stored to LDS
        // buffer j % 2 one step ahead of its use, so KV_RING - 1 tiles are in
        // flight while a step waits for the next one.  The register set is
        // chosen at compile time (the loop body is KV_RING steps, unrolled),
        // and every step issues its loads (past the end they re-read row
        // t_end-1), so the compiler's wait before each LDS store is an exact
        // count.
        u32x4 ring[KV_RING][4];
#pragma unroll
        for (int j = 0; j < KV_RING; ++j) kv_gload<T>(ring[j], qkv, b, N, C, h0, nh, t_begin + j * kTT, t_end, tid);
        kv_store(ring[0], 0, t_begin);
        barrier_keep_loads();
        // Step it: LDS buffer it&1 holds tile it; ring[(it+1) % KV_RING] holds
        // tile it+1; ring[it % KV_RING] is free and receives tile it+KV_RING.
        auto step = [&](int it, u32x4 (&fr)[4], u32x4 (&nx)[4]) {
            kv_gload<T>(fr, qkv, b, N, C, h0, nh, t_begin + (it + KV_RING) * kTT, t_end, tid);
            accumulate(it & 1);
            kv_store(nx, (it + 1) & 1, t_begin + (it + 1) * kTT);
            barrier_keep_loads();
        };
        // Whole rounds of KV_RING steps in the loop, the remainder after it,
        // so the loop's back edge always follows a full round.
        int it = 0;
        for (; it + KV_RING <= ntile; it += KV_RING) {
#pragma unroll
            for (int r = 0; r < KV_RING; ++r) step(it + r, ring[r], ring[(r + 1) % KV_RING]);
        }
#pragma unroll
        for (int r = 0; r < KV_RING - 1; ++r)
            if (it + r < ntile) step(it + r, ring[r], ring[(r + 1) % KV_RING]);
    }
    // Combine the four token quarters of each head (in quarter order), then
    // write the partial.
    __syncthreads();
    float (*comb)[3][64][17] = reinterpret_cast<float (*)[3][64][17]>(lds);
    if (th > 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) comb[hw][th - 1][lane][i] = acc[i];
        comb[hw][th - 1][lane][16] = zsum;
    }
    __syncthreads();
    if (th == 0) {
#pragma unroll
        for (int q = 0; q < 3; ++q) {
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] += comb[hw][q][lane][i];
            zsum += comb[hw][q][lane][16];
        }
        zsum += __shfl_xor(zsum, 32, 64);  // lanes l and l+32 hold the same channel
        if (hw < nh) {
            // Device-coherent stores (sc1: written through to the coherence
            // point shared by all XCDs), so no L2 write-back is needed before
            // the other members read them.
            float* P = p.partial + ((int64_t)(b * H + h0 + hw) * p.S + s) * kState;
            const int c = lane & 31;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                __hip_atomic_store(P + r * kD + c, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (lane < 32) __hip_atomic_store(P + kD * kD + c, zsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // The stores have completed at the coherence point before this wave
        // reaches the workgroup barrier that precedes the arrival count.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // The first Q_RING q tiles are requested before the barrier, so their
    // latency overlaps the wait for the other splits.
    u32x4 qring[Q_RING][2];
#pragma unroll
    for (int j = 0; j < Q_RING; ++j) q_gload<T>(qring[j], qkv, b, N, C, h0, nh, t_begin + j * kTT, t_end, tid);
    barrier_keep_loads();
    const bool late = group_barrier(p.ctrl, g, (unsigned)p.S, p.spin_limit, &sh_late);

    // ---------------- Phase 2: the group's state, then the outputs --------
    // The group's partials of both heads (2 x 1056 floats, 528 16-byte
    // vectors) are summed in split order by all 512 threads into LDS (inside
    // the first out buffer, which is first written after the phase-2 loop's
    // first barrier, when every wave has read its state), eight splits' loads
    // in flight at a time.  Plain loads
    // see the partials: they were written with device-coherent stores that
    // completed before their writers arrived, and no cache holds a line of
    // them from before the barrier (nothing reads them earlier in a launch,
    // and caches start every launch invalidated).
    // The sums keep 36-float rows in LDS: the operand reads below take row
    // m16 = 0..15 at one column in 16 lanes, which 32-float rows would put on
    // eight banks; 36 spreads them over all 64.
    constexpr int kRowPad = kD + 4, kPadState = (kD + 1) * kRowPad;
    float* sums = reinterpret_cast<float*>(lds + 2 * Q_BYTES);
    static_assert(2 * Q_BYTES + 2 * kPadState * 4 <= LDS_BYTES, "state sums fit");
    {
        constexpr int NV = 2 * kState / 4;  // 16-byte vectors of the pair's state
        const float* P0 = p.partial + (int64_t)(b * H + h0) * p.S * kState;
        const float* P1 = nh > 1 ? P0 + (int64_t)p.S * kState : P0;
        for (int v = tid; v < NV; v += kThreads) {
            const int e = 4 * v;
            const float* P = e < kState ? P0 + e : P1 + (e - kState);
            f32x4 acc4 = {0.f, 0.f, 0.f, 0.f};
            for (int s0 = 0; s0 < p.S; s0 += 8) {
                f32x4 part4[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    part4[j] = s0 + j < p.S ? *reinterpret_cast<const f32x4*>(P + (int64_t)(s0 + j) * kState)
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 8; ++j) acc4 += part4[j];  // split order; padding adds zero
            }
            const int hh = e >= kState, rem = e - hh * kState;  // 4 floats of one row
            *reinterpret_cast<f32x4*>(sums + hh * kPadState + (rem / kD) * kRowPad + rem % kD) = acc4;
        }
    }
    barrier_keep_loads();
    // S and z of head hw as hi+lo 16-bit A operands: rows r = 16*mb + m16,
    // k = c = 8*kg + j; the third operand repeats z on every row, so the
    // denominator lands in the same lanes as the numerator.
    const int m16 = lane & 15, kg = lane >> 4;
    float sv[2][8], zv[8];
    {
        const float* S0 = sums + hw * kPadState;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sv[0][j] = S0[m16 * kRowPad + 8 * kg + j];
            sv[1][j] = S0[(16 + m16) * kRowPad + 8 * kg + j];
            zv[j] = S0[kD * kRowPad + 8 * kg + j];
        }
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
    // A member that stopped waiting holds an incomplete state: NaN rather than
    // a silently wrong result.
    const float eps = late ? __builtin_nanf("") : p.eps * scale;

    TO* __restrict__ out = static_cast<TO*>(p.out);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const int ch0 = (kg & 1) ? 16 + 4 * (kg - 1) : 4 * kg;  // first channel a lane stores
    constexpr int OCH = OutTile<TO>::CHUNKS;                  // 16-byte chunks per token row
    constexpr int OROUNDS = kTT * OCH / kThreads;             // store rounds per tile
    const int valid_chunks = nh * OCH / 2;
    auto qbuf = [&](int i) { return lds + (i & 1) * Q_BYTES; };
    auto obuf = [&](int i) { return lds + 2 * Q_BYTES + (i & 1) * O_BYTES; };
    auto q_store = [&](const u32x4 (&reg)[2], int i) {
        unsigned char* base = qbuf(i);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int c = k * kThreads + tid;
            *reinterpret_cast<u32x4*>(base + r128_off(c >> 3, c & 7)) = relu_packed16(reg[k]);
        }
    };
    auto out_tile = [&](int i) {
        const unsigned char* qb = qbuf(i);
        unsigned char* ob = obuf(i);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int row = 32 * th + 16 * u + m16;
            const typename V<T>::x8 bq = *reinterpret_cast<const typename V<T>::x8*>(qb + r128_off(row, 4 * hw + kg));
            f32x4 n0 = mfma16x16x32(shi[0], bq, zero);
            n0 = mfma16x16x32(slo[0], bq, n0);
            f32x4 n1 = mfma16x16x32(shi[1], bq, zero);
            n1 = mfma16x16x32(slo[1], bq, n1);
            f32x4 dn = mfma16x16x32(zhi, bq, zero);
            dn = mfma16x16x32(zlo, bq, dn);
            const float inv = 1.0f / (dn[0] + eps);
            f32x4 lo, hi;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(n0[k] * inv),
                                                                __float_as_uint(n1[k] * inv), false, false);
                lo[k] = __uint_as_float(r[0]);
                hi[k] = __uint_as_float(r[1]);
            }
            store8_lds<TO>(ob, row, hw * kD + ch0, lo, hi);
        }
    };
    auto out_store = [&](int i, int t0) {
        const unsigned char* ob = obuf(i);
        if constexpr (OT) {
            // Channel rows of out[b][c][t]: thread (tid % 128) owns token
            // t0 + tid % 128 and channels (tid / 128) + 4k, so each store
            // instruction of a wave writes 64 consecutive tokens (256 bytes)
            // of one channel.
            const int tok = tid & (kTT - 1), cq = tid >> 7;
            if (t0 + tok < t_end) {
                float* dst = reinterpret_cast<float*>(out) + ((int64_t)b * C + (int64_t)h0 * kD) * N + t0 + tok;
#pragma unroll
                for (int k = 0; k < 2 * kD / 4; ++k) {
                    const int ch = cq + 4 * k;
                    if (ch < nh * kD) {
                        const float v = *reinterpret_cast<const float*>(ob + OutTile<TO>::off(tok, ch >> 2) +
                                                                        (ch & 3) * 4);
                        __builtin_nontemporal_store(v, dst + (int64_t)ch * N);
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < OROUNDS; ++k) {
            const int c = k * kThreads + tid;
            const int tok = c / OCH, chunk = c % OCH;
            if (t0 + tok < t_end && chunk < valid_chunks) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(ob + OutTile<TO>::off(tok, chunk));
                unsigned char* dst = reinterpret_cast<unsigned char*>(out + ((int64_t)b * N + t0 + tok) * C +
                                                                      (int64_t)h0 * kD);
                // Plain (cached) stores: 4% faster than nontemporal ones at
                // B=1, N=16384 on MI355X (54.7 against 56.9 us), the same at
                // B=2, N=4096; nontemporal loads stay faster for q and K/V.
                *reinterpret_cast<u32x4*>(dst + chunk * 16) = v;
            }
        }
    };
    // Tile i: q registers -> LDS q buffer i&1, barrier, MFMA -> LDS out buffer
    // i&1, barrier, whole-line stores; the double buffers make two barriers
    // per tile enough.  Q_RING q tiles stay in flight in registers.
    auto pstep = [&](int it, u32x4 (&cur)[2]) {
        const int t0 = t_begin + it * kTT;
        q_store(cur, it);
        q_gload<T>(cur, qkv, b, N, C, h0, nh, t0 + Q_RING * kTT, t_end, tid);
        barrier_keep_loads();
        out_tile(it);
        barrier_keep_loads();
        out_store(it, t0);
    };
    int it = 0;
    for (; it + Q_RING <= ntile; it += Q_RING) {
#pragma unroll
        for (int r = 0; r < Q_RING; ++r) pstep(it + r, qring[r]);
    }
#pragma unroll
    for (int r = 0; r < Q_RING - 1; ++r)
        if (it + r < ntile) pstep(it + r, qring[r]);
}

// --------------------------------------------------------------------------
// Fixed-order reduction of the split partials (generic path).
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

// Zeroes n words (the control words of a fresh workspace).
__global__ __launch_bounds__(256) void linattn_zero_kernel(unsigned* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
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
                                                           float eps, int out_tn) {
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
                // out[b][t][c], or out[b][c][t] (LiteLA.attn_matmul's [B, h, d, N]) when out_tn.
                const int64_t c_out = (int64_t)h * DG + r;
                const int64_t o = out_tn ? ((int64_t)b * C + c_out) * N + t : ((int64_t)b * N + t) * C + c_out;
                out[o] = from_f32<TO>(num / (den + eps));
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

// Split plan of a request: `splits` (>= 1 after the default is applied) is
// cut to the sequence length and to `max_members` (the fused kernel's
// resident-workgroup capacity, or the generic path's grid limit), then each
// split gets a whole number of `align`-token tiles; `eff` is the number of
// non-empty splits that gives, never more than the cut request.
void split_plan(int64_t N, int64_t splits, int64_t align, int64_t max_members, int64_t* len, int64_t* eff) {
    if (splits > N) splits = N;
    if (splits > max_members) splits = max_members;
    if (splits < 1) splits = 1;
    *len = split_len_for(N, splits, align);
    *eff = (N + *len - 1) / *len;
}

// Workspace regions: control words, split partials, reduced states (the
// generic path's; the fused kernel keeps its state in registers).
struct Workspace {
    unsigned* ctrl;
    float* partial;
    float* state;
};

// One resolved call.
struct Launch {
    const void* qkv;
    void* out;
    Workspace ws;
    int B, N, H, D, S, L;  // S splits of L tokens
    float eps;
    int spin_limit;
    bool force_ticket;     // number workgroups by ticket even when all fit at once
    bool out_tn;           // out[b][c][t] instead of out[b][t][c]
    hipStream_t stream;
};

// Workgroups of one fused-kernel instantiation that the current device holds
// at once: the occupancy per CU (LDS and registers decide it: one for fp32
// output, whose phase-2 tiles take 96 KiB of LDS) times the CU count.
template <typename T, typename TO, bool OT>
int64_t fused_slots() {
    static std::atomic<int> per_cu[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = per_cu[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, linattn_fused_kernel<T, TO, OT>, kThreads, 0) !=
                hipSuccess ||
            blocks < 1) {
            (void)hipGetLastError();
            blocks = 1;  // the query failed: assume the least
        }
        per_cu[dev].store(blocks, std::memory_order_relaxed);
        n = blocks;
    }
    return (int64_t)n * device_cu_count();
}

int64_t fused_slots_for(int in_dt, int out_dt, bool ot) {
    if (in_dt == KF_BF16) {
        if (ot) return fused_slots<bf16, float, true>();
        return out_dt == KF_F32 ? fused_slots<bf16, float, false>()
               : out_dt == KF_F16 ? fused_slots<bf16, f16, false>() : fused_slots<bf16, bf16, false>();
    }
    if (ot) return fused_slots<f16, float, true>();
    return out_dt == KF_F32 ? fused_slots<f16, float, false>()
           : out_dt == KF_F16 ? fused_slots<f16, f16, false>() : fused_slots<f16, bf16, false>();
}

template <typename T, typename TO, bool OT>
int run_mfma(const Launch& a) {
    FusedParams p;
    p.qkv = a.qkv;
    p.out = a.out;
    p.partial = a.ws.partial;
    p.ctrl = a.ws.ctrl;
    p.N = a.N;
    p.H = a.H;
    p.npairs = (a.H + 1) / 2;
    p.S = a.S;
    p.split_len = a.L;
    p.spin_limit = a.spin_limit;
    p.eps = a.eps;
    const int64_t groups = (int64_t)a.B * p.npairs;
    const int64_t slots = fused_slots<T, TO, OT>();
    // Groups per launch: the control region holds kMaxGroupsPerLaunch groups,
    // and a launch's workgroup count stays below 2^31.
    int64_t per = kMaxGroupsPerLaunch;
    if (per * a.S > 0x7fffffffLL) per = 0x7fffffffLL / a.S;
    for (int64_t g0 = 0; g0 < groups; g0 += per) {
        const int64_t n = groups - g0 < per ? groups - g0 : per;
        p.g0 = (int)g0;
        p.total = (int)(n * a.S);
        p.use_ticket = p.total > slots || a.force_ticket ? 1 : 0;
        hipLaunchKernelGGL((linattn_fused_kernel<T, TO, OT>), dim3((unsigned)p.total), dim3(kThreads), 0, a.stream,
                           p);
        if (int rc = check_launch("linattn_fused_kernel launch")) return rc;
    }
    return KF_OK;
}

template <typename T, typename TO, int DG>
int run_generic(const Launch& a) {
    hipLaunchKernelGGL((linattn_state_generic<T, DG>), dim3(a.H, a.S, a.B), dim3(256), 0, a.stream,
                       static_cast<const T*>(a.qkv), a.ws.partial, a.N, a.H, a.L, a.S);
    if (int rc = check_launch("linattn_state_generic launch")) return rc;
    if (int rc = launch_reduce(a.ws.partial, a.ws.state, (int64_t)a.B * a.H, a.S, (DG + 1) * DG, a.stream))
        return rc;
    hipLaunchKernelGGL((linattn_out_generic<T, TO, DG>), dim3(a.H, out_grid_y(a.N), a.B), dim3(256), 0, a.stream,
                       static_cast<const T*>(a.qkv), a.ws.state, static_cast<TO*>(a.out), a.N, a.H, a.eps,
                       a.out_tn ? 1 : 0);
    return check_launch("linattn_out_generic launch");
}

template <typename T, typename TO>
int run_generic_d(const Launch& a) {
#define KF_GENERIC_CASE(DD) \
    case DD: return run_generic<T, TO, DD>(a);
    switch (a.D) {
        KF_GENERIC_CASE(1) KF_GENERIC_CASE(2) KF_GENERIC_CASE(4) KF_GENERIC_CASE(8)
        KF_GENERIC_CASE(16) KF_GENERIC_CASE(32) KF_GENERIC_CASE(64) KF_GENERIC_CASE(128)
        default: set_error("linattn: unsupported head dim %d", a.D); return KF_E_UNSUPPORTED;
    }
#undef KF_GENERIC_CASE
}

template <typename T>
int run_in(int out_dt, bool mfma, const Launch& a) {
    if (mfma) {
        if constexpr (sizeof(T) == 2) {
            if (a.out_tn) return run_mfma<T, float, true>(a);  // fp32 output only (checked by the caller)
            switch (out_dt) {
                case KF_F32: return run_mfma<T, float, false>(a);
                case KF_F16: return run_mfma<T, f16, false>(a);
                case KF_BF16: return run_mfma<T, bf16, false>(a);
            }
        }
    }
    switch (out_dt) {
        case KF_F32: return run_generic_d<T, float>(a);
        case KF_F16: return run_generic_d<T, f16>(a);
        case KF_BF16: return run_generic_d<T, bf16>(a);
    }
    set_error("linattn: unknown output dtype %d", out_dt);
    return KF_E_INVALID;
}

bool valid_dim(int64_t D) { return D > 0 && D <= 128 && 128 % D == 0; }

// Argument checks shared by every entry point, before any device call.
int validate(int64_t batch, int64_t seq_len, int64_t heads, int64_t dim, int in_dtype, int out_dtype) {
    KF_REQUIRE(batch >= 0 && seq_len >= 0 && heads >= 0, KF_E_INVALID,
               "linattn: negative shape B=%lld N=%lld H=%lld", (long long)batch,
               (long long)seq_len, (long long)heads);
    KF_REQUIRE(valid_dim(dim), KF_E_INVALID, "linattn: dim must divide 128 and be at most 128, got %lld",
               (long long)dim);
    KF_REQUIRE(in_dtype == KF_F32 || in_dtype == KF_F16 || in_dtype == KF_BF16, KF_E_INVALID,
               "linattn: unknown input dtype %d", in_dtype);
    KF_REQUIRE(out_dtype == KF_F32 || out_dtype == KF_F16 || out_dtype == KF_BF16, KF_E_INVALID,
               "linattn: unknown output dtype %d", out_dtype);
    KF_REQUIRE(batch <= 65535 && heads <= 65535 && seq_len <= 0x3fffffff, KF_E_UNSUPPORTED,
               "linattn: shape exceeds grid limits");
    return KF_OK;
}

// The fused kernel is the candidate for head dim 32 and 16-bit input (it also
// needs 16-byte aligned buffers, which only the run itself can check).
bool fused_candidate(int64_t dim, int in_dtype) { return dim == kD && in_dtype != KF_F32; }

// Effective split count of a validated, non-empty request: the default for
// splits <= 0, then the split plan, with the fused kernel's group size kept
// within the workgroups the device holds at once (invariant 3 of the fused
// kernel); `len` receives the split length.
int64_t resolve_splits(int64_t batch, int64_t seq_len, int64_t heads, int64_t dim, int64_t splits, int in_dtype,
                       int out_dtype, bool out_tn, int64_t* len) {
    if (splits <= 0) splits = kf_linattn_default_splits(batch, heads, dim, seq_len);
    const bool fused = fused_candidate(dim, in_dtype) && (!out_tn || out_dtype == KF_F32);
    int64_t max_members = 65535;  // the generic path's split index is a y grid dimension
    if (fused) {
        const int64_t slots = fused_slots_for(in_dtype, out_dtype, out_tn);
        if (slots < max_members) max_members = slots;
    }
    int64_t eff = 1;
    split_plan(seq_len, splits, fused ? kTT : kGT, max_members, len, &eff);
    return eff;
}

// Zeroes the first `bytes` of a workspace (rounded down to whole words).
int zero_words(void* ws, int64_t bytes, hipStream_t s) {
    const int64_t n = bytes / 4;
    if (n <= 0) return KF_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(linattn_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<unsigned*>(ws), n);
    return check_launch("linattn_zero_kernel launch");
}

// Runs a validated, non-empty request with `workspace` holding the control
// words, the partials and (generic path) the reduced states.
int linattn_run(const void* qkv, void* out, void* workspace, int64_t workspace_bytes, int64_t batch,
                int64_t seq_len, int64_t heads, int64_t dim, int64_t splits, float eps, int in_dtype,
                int out_dtype, bool out_tn, int spin_limit, hipStream_t s, bool force_ticket = false) {
    KF_REQUIRE(qkv && out, KF_E_INVALID, "linattn: null pointer");
    int64_t split_len = 0;
    const int64_t eff = resolve_splits(batch, seq_len, heads, dim, splits, in_dtype, out_dtype, out_tn, &split_len);
    const int64_t need = kf_linattn_workspace_bytes(batch, heads, dim, eff);
    KF_REQUIRE(workspace && workspace_bytes >= need, KF_E_WORKSPACE,
               "linattn: workspace of %lld bytes needed, %lld given", (long long)need,
               (long long)workspace_bytes);
    KF_REQUIRE((uintptr_t)workspace % 256 == 0, KF_E_WORKSPACE, "linattn: workspace must be 256-byte aligned");
    const bool mfma = fused_candidate(dim, in_dtype) && (!out_tn || out_dtype == KF_F32) &&
                      (uintptr_t)qkv % 16 == 0 && (uintptr_t)out % 16 == 0;
    if (!mfma && fused_candidate(dim, in_dtype)) {
        // Unaligned buffers (or 16-bit transposed output): the generic path,
        // with its own tile alignment and at most `eff` splits.
        int64_t eff_generic = 0;
        split_plan(seq_len, eff, kGT, 65535, &split_len, &eff_generic);
    }
    Launch a;
    a.qkv = qkv;
    a.out = out;
    a.ws.ctrl = static_cast<unsigned*>(workspace);
    a.ws.partial = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + kCtrlBytes);
    a.B = (int)batch;
    a.N = (int)seq_len;
    a.H = (int)heads;
    a.D = (int)dim;
    a.L = (int)split_len;
    a.S = (int)((seq_len + split_len - 1) / split_len);  // <= eff
    a.ws.state = a.ws.partial + batch * heads * (dim + 1) * dim * a.S;
    a.eps = eps;
    a.spin_limit = spin_limit;
    a.force_ticket = force_ticket;
    a.out_tn = out_tn;
    a.stream = s;
    switch (in_dtype) {
        case KF_BF16: return run_in<bf16>(out_dtype, mfma, a);
        case KF_F16: return run_in<f16>(out_dtype, mfma, a);
        default: return run_in<float>(out_dtype, false, a);
    }
}

// Per-device address of `scratch`, resolved once per device with that
// device current (each GPU holds its own copy at its own address).  The
// first call on a device also zeroes the scratch's control words on the
// caller's stream (the array starts zeroed at load; this makes it explicit).
int scratch_for_current_device(void** ptr, hipStream_t stream) {
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
        if (int rc = zero_words(p, kCtrlBytes, stream)) return rc;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return KF_OK;
}

// Reads the error word of a control region after `stream` has drained; when
// it is set, clears the whole control region (a ticket counter may be left
// over too) and reports what happened.
int check_ctrl(unsigned* ctrl, hipStream_t stream) {
    unsigned word = 0;
    hipError_t err = hipMemcpyAsync(&word, ctrl + 1, sizeof(word), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return hip_failure(err, "linattn check: reading the error word");
    if (word == 0) return KF_OK;
    if (int rc = zero_words(ctrl, kCtrlBytes, stream)) return rc;
    err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return hip_failure(err, "linattn check: clearing the control words");
    if (word == 1)
        set_error("linattn: split workgroups of a (batch, head pair) stopped waiting for the rest of their "
                  "group (other work held the device's slots past the poll limit); their outputs are NaN");
    else
        set_error("linattn: the workspace's control words were not zero on entry (error word %u); "
                  "outputs are incomplete", word);
    return KF_E_INCOMPLETE;
}

// Validates, then runs kf_linattn_fwd's request on the static scratch.
int noalloc_run(const void* qkv, void* out, int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                int64_t splits, float eps, int in_dtype, int out_dtype, hipStream_t s) {
    if (int rc = validate(batch, seq_len, heads, dim, in_dtype, out_dtype)) return rc;
    if (batch == 0 || seq_len == 0 || heads == 0) return KF_OK;
    // Size check before any device work.
    int64_t len = 0;
    const int64_t eff = resolve_splits(batch, seq_len, heads, dim, splits, in_dtype, out_dtype, false, &len);
    const int64_t need = kf_linattn_workspace_bytes(batch, heads, dim, eff);
    KF_REQUIRE(need <= kLinattnScratchBytes, KF_E_WORKSPACE,
               "linattn noalloc: %lld bytes of scratch needed for B=%lld H=%lld D=%lld splits=%lld, "
               "the static scratch holds %lld; use fewer splits or kf_linattn_fwd with a workspace",
               (long long)need, (long long)batch, (long long)heads, (long long)dim, (long long)eff,
               (long long)kLinattnScratchBytes);
    KF_REQUIRE(qkv && out, KF_E_INVALID, "linattn: null pointer");
    void* ws = nullptr;
    if (int rc = scratch_for_current_device(&ws, s)) return rc;
    return linattn_run(qkv, out, ws, kLinattnScratchBytes, batch, seq_len, heads, dim, eff, eps, in_dtype,
                       out_dtype, false, kSpinLimit, s);
}

}  // namespace
}  // namespace kf

extern "C" int64_t kf_linattn_default_splits(int64_t batch, int64_t heads, int64_t dim,
                                             int64_t seq_len) {
    // D = 32 (the fused kernel): one workgroup per CU at most, each streaming
    // at least one 128-token tile of a head pair.  The members of a group meet
    // at a barrier, so every member waits for the slowest: a grid that leaves
    // some CUs with two workgroups and others with one ran 10-20% slower on
    // MI355X than one workgroup per CU (B=2, H=70, N=4096: 36.3 us at 3 splits
    // = 210 workgroups, 41.8 us at 4 = 280; B=1, N=16384: 57.6 us at 7 = 245,
    // 74.1 us at 8 = 280).  Other head dims: about 1.75 workgroups per CU.
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 1;
    const int64_t cus = kf::device_cu_count();
    int64_t splits;
    if (dim == kf::kD) {
        const int64_t groups = batch * ((heads + 1) / 2);
        splits = cus / groups;
    } else {
        const int64_t groups = batch * heads;
        splits = ((7 * cus + 3) / 4 + groups - 1) / groups;
    }
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
    return kf::kCtrlBytes + (int64_t)sizeof(float) * batch * heads * state * (splits + 1);
}

extern "C" int kf_linattn_workspace_init(void* workspace, int64_t workspace_bytes, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(workspace_bytes >= 0, KF_E_INVALID, "linattn: negative workspace size");
    KF_REQUIRE(workspace || workspace_bytes == 0, KF_E_INVALID, "linattn: null workspace");
    const int64_t n = workspace_bytes < kCtrlBytes ? workspace_bytes : kCtrlBytes;
    return zero_words(workspace, n, static_cast<hipStream_t>(stream));
}

extern "C" int kf_linattn_fwd(const void* qkv, void* out, void* workspace, int64_t workspace_bytes,
                              int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                              int64_t splits, float eps, int in_dtype, int out_dtype,
                              kf_stream_t stream) {
    using namespace kf;
    if (int rc = validate(batch, seq_len, heads, dim, in_dtype, out_dtype)) return rc;
    if (batch == 0 || seq_len == 0 || heads == 0) return KF_OK;
    return linattn_run(qkv, out, workspace, workspace_bytes, batch, seq_len, heads, dim, splits, eps, in_dtype,
                       out_dtype, false, kSpinLimit, static_cast<hipStream_t>(stream));
}

extern "C" int kf_linattn_attn_matmul(const void* qkv, float* out, void* workspace, int64_t workspace_bytes,
                                      int64_t batch, int64_t seq_len, int64_t heads, int64_t dim,
                                      int64_t splits, float eps, int in_dtype, kf_stream_t stream) {
    using namespace kf;
    if (int rc = validate(batch, seq_len, heads, dim, in_dtype, KF_F32)) return rc;
    if (batch == 0 || seq_len == 0 || heads == 0) return KF_OK;
    return linattn_run(qkv, out, workspace, workspace_bytes, batch, seq_len, heads, dim, splits, eps, in_dtype,
                       KF_F32, true, kSpinLimit, static_cast<hipStream_t>(stream));
}

extern "C" int kf_linattn_check(void* workspace, int64_t workspace_bytes, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(workspace && workspace_bytes >= kCtrlBytes, KF_E_WORKSPACE,
               "linattn check: a workspace of at least %lld bytes is needed", (long long)kCtrlBytes);
    return check_ctrl(static_cast<unsigned*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int64_t kf_linattn_noalloc_max_bytes(void) { return kLinattnScratchBytes; }

extern "C" int kf_linattn_fwd_noalloc(const void* qkv, void* out, int64_t batch, int64_t seq_len,
                                      int64_t heads, int64_t dim, int64_t splits, float eps, int in_dtype,
                                      int out_dtype, kf_stream_t stream) {
    return kf::noalloc_run(qkv, out, batch, seq_len, heads, dim, splits, eps, in_dtype, out_dtype,
                           static_cast<hipStream_t>(stream));
}

extern "C" int kf_linattn_noalloc_check(kf_stream_t stream) {
    using namespace kf;
    void* ws = nullptr;
    if (int rc = scratch_for_current_device(&ws, static_cast<hipStream_t>(stream))) return rc;
    return check_ctrl(static_cast<unsigned*>(ws), static_cast<hipStream_t>(stream));
}

// Test entry points (not in the public header).
//
// kf_linattn_fwd with the number of polls a member of the fused kernel makes
// at its group's counter before giving up (and writing NaN); polls <= 0 or
// above the default take the default.  A cut limit also selects ticket
// numbering.  Lets a test drive the give-up path from the host without any
// global state.
extern "C" int kfm_linattn_fwd_spin(const void* qkv, void* out, void* workspace, int64_t workspace_bytes,
                                    int64_t batch, int64_t seq_len, int64_t heads, int64_t dim, int64_t splits,
                                    float eps, int in_dtype, int out_dtype, int64_t polls, kf_stream_t stream) {
    using namespace kf;
    if (int rc = validate(batch, seq_len, heads, dim, in_dtype, out_dtype)) return rc;
    if (batch == 0 || seq_len == 0 || heads == 0) return KF_OK;
    const int spin = polls <= 0 || polls > kSpinLimit ? kSpinLimit : (int)polls;
    // A cut poll limit also numbers the workgroups by ticket, as a launch
    // beyond the device's capacity does: the members of a group then start
    // one after another, so the early ones reach the limit while waiting.
    return linattn_run(qkv, out, workspace, workspace_bytes, batch, seq_len, heads, dim, splits, eps, in_dtype,
                       out_dtype, false, spin, static_cast<hipStream_t>(stream), spin != kSpinLimit);
}

// The split plan's arithmetic (no device call): plan[0] = split length,
// plan[1] = effective split count.
extern "C" int kfm_linattn_split_plan(int64_t seq_len, int64_t splits, int64_t align, int64_t max_members,
                                      int64_t* plan) {
    if (seq_len <= 0 || align <= 0 || max_members <= 0 || !plan) return KF_E_INVALID;
    kf::split_plan(seq_len, splits, align, max_members, &plan[0], &plan[1]);
    return KF_OK;
}
