// Measurement kernels: the attainable HBM stream rate and dense bf16 MFMA
// rate of the device the library runs on.  bench.py reports them next to the
// hot-path kernels as the ceilings those kernels are compared with.  They
// compute nothing for a caller, so they are exported with the kfm_ prefix
// and are not part of the public C ABI header.
#include "kf_common.h"

namespace kf {
namespace {

// Stream copy: thread t of a block of BS threads moves the 16-byte vectors
// (b * VPT + i) * BS + t, i < VPT, so every load and store instruction of a
// wavefront covers one contiguous 1 KiB span, the access shape of the
// RMSNorm kernel.  All VPT loads are issued before the first store.  POL
// selects the cache policy: bit 0 plain (cached) loads instead of
// nontemporal ones, bit 1 plain stores.  On MI355X one-wavefront blocks with
// one vector per lane and nontemporal loads and stores stream fastest (3-5%
// above 256-thread blocks at 64-256 MiB; the sweep of `bench.py --only
// copy_sweep` covers block sizes, vectors per lane, cache policies and
// occupancy limits).
template <int VPT, int BS, int POL = 0>
__global__ __launch_bounds__(BS) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                  int64_t nvec) {
    const int64_t base = (int64_t)blockIdx.x * BS * VPT + threadIdx.x;
    const u32x4* s = src + base;
    u32x4* d = dst + base;
    u32x4 v[VPT];
    if (base + (int64_t)(VPT - 1) * BS < nvec) {
        // Whole block in range: no per-vector guards (they cost registers).
#pragma unroll
        for (int i = 0; i < VPT; ++i) v[i] = (POL & 1) ? s[i * BS] : __builtin_nontemporal_load(s + i * BS);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            if constexpr (POL & 2) d[i * BS] = v[i];
            else __builtin_nontemporal_store(v[i], d + i * BS);
        }
        return;
    }
    for (int i = 0; i < VPT; ++i) {
        if (base + (int64_t)i * BS >= nvec) break;
        const u32x4 x = (POL & 1) ? s[i * BS] : __builtin_nontemporal_load(s + i * BS);
        if constexpr (POL & 2) d[i * BS] = x;
        else __builtin_nontemporal_store(x, d + i * BS);
    }
}

// Dynamic LDS of `lds` bytes per block limits the blocks a CU holds at once.
template <int BS, int POL>
int launch_copy(int vpt, const u32x4* in, u32x4* o, int64_t nvec, int lds, hipStream_t s) {
    const int64_t blocks = (nvec + (int64_t)BS * vpt - 1) / ((int64_t)BS * vpt);
    KF_REQUIRE(blocks <= 0x7fffffff, KF_E_UNSUPPORTED, "copy: too many blocks");
    const dim3 g((unsigned)blocks), b(BS);
    switch (vpt) {
        case 1: hipLaunchKernelGGL((copy_kernel<1, BS, POL>), g, b, lds, s, in, o, nvec); break;
        case 2: hipLaunchKernelGGL((copy_kernel<2, BS, POL>), g, b, lds, s, in, o, nvec); break;
        case 4: hipLaunchKernelGGL((copy_kernel<4, BS, POL>), g, b, lds, s, in, o, nvec); break;
        case 8: hipLaunchKernelGGL((copy_kernel<8, BS, POL>), g, b, lds, s, in, o, nvec); break;
        default: set_error("copy: vectors_per_thread must be 1, 2, 4 or 8, got %d", vpt); return KF_E_INVALID;
    }
    return check_launch("copy_kernel launch");
}

template <int POL>
int launch_copy_bs(int bs, int vpt, const u32x4* in, u32x4* o, int64_t nvec, int lds, hipStream_t s) {
    switch (bs) {
        case 64: return launch_copy<64, POL>(vpt, in, o, nvec, lds, s);
        case 256: return launch_copy<256, POL>(vpt, in, o, nvec, lds, s);
        case 1024: return launch_copy<1024, POL>(vpt, in, o, nvec, lds, s);
    }
    set_error("copy: threads_per_block must be 64, 256 or 1024, got %d", bs);
    return KF_E_INVALID;
}

int copy_run(const void* src, void* dst, int64_t bytes, int vpt, int bs, int policy, int lds, hipStream_t s) {
    KF_REQUIRE(bytes >= 0 && bytes % 16 == 0, KF_E_INVALID, "copy: bytes %lld not a multiple of 16",
               (long long)bytes);
    KF_REQUIRE(bytes == 0 || (src && dst && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0),
               KF_E_INVALID, "copy: null or unaligned pointer");
    KF_REQUIRE(bs == 64 || bs == 256 || bs == 1024, KF_E_INVALID,
               "copy: threads_per_block must be 64, 256 or 1024, got %d", bs);
    KF_REQUIRE(policy >= 0 && policy <= 3, KF_E_INVALID, "copy: policy must be 0..3, got %d", policy);
    KF_REQUIRE(lds >= 0 && lds <= 65536, KF_E_INVALID, "copy: lds_bytes must be 0..65536, got %d", lds);
    if (bytes == 0) return KF_OK;
    const int64_t nvec = bytes / 16;
    const u32x4* in = static_cast<const u32x4*>(src);
    u32x4* o = static_cast<u32x4*>(dst);
    switch (policy) {
        case 0: return launch_copy_bs<0>(bs, vpt, in, o, nvec, lds, s);
        case 1: return launch_copy_bs<1>(bs, vpt, in, o, nvec, lds, s);
        case 2: return launch_copy_bs<2>(bs, vpt, in, o, nvec, lds, s);
        default: return launch_copy_bs<3>(bs, vpt, in, o, nvec, lds, s);
    }
}

// Dense bf16 MFMA issue rate: each wavefront runs `iters` rounds of two
// independent v_mfma_f32_32x32x16_bf16 chains (32768 flops each).  On MI355X
// this shape issues at 97-98% of the published dense peak from two
// wavefronts per SIMD up; a loop of four or more 16x16x32 chains reads lower
// only because the compiler then shuffles the accumulators between
// registers every round.  The result is stored so the chains are not removed.
__global__ __launch_bounds__(256) void mfma_kernel(float* __restrict__ out, int iters) {
    V<bf16>::x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (bf16)(threadIdx.x * 0.001f + i);
        b[i] = (bf16)(i * 0.5f);
    }
    f32x16 c0, c1;
#pragma unroll
    for (int i = 0; i < 16; ++i) c0[i] = c1[i] = 0.f;
    for (int it = 0; it < iters; ++it) {
        c0 = mfma32x32x16(a, b, c0);
        c1 = mfma32x32x16(a, b, c1);
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace
}  // namespace kf

// Copy `bytes` (a multiple of 16, both pointers 16-byte aligned) from src to
// dst with VPT = vectors_per_thread in {1, 2, 4, 8} 16-byte vectors per lane
// and threads_per_block in {64, 256}.
extern "C" int kfm_copy(const void* src, void* dst, int64_t bytes, int vectors_per_thread, int threads_per_block,
                        kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(threads_per_block == 64 || threads_per_block == 256, KF_E_INVALID,
               "copy: threads_per_block must be 64 or 256, got %d", threads_per_block);
    return copy_run(src, dst, bytes, vectors_per_thread, threads_per_block, 0, 0, static_cast<hipStream_t>(stream));
}

// The copy with every variable of the ceiling sweep: threads_per_block 64,
// 256 or 1024; policy bit 0 = plain loads, bit 1 = plain stores (else
// nontemporal); lds_bytes of dynamic LDS per block (0..65536) to cap the
// blocks per CU.
extern "C" int kfm_copy_ex(const void* src, void* dst, int64_t bytes, int vectors_per_thread, int threads_per_block,
                           int policy, int lds_bytes, kf_stream_t stream) {
    return kf::copy_run(src, dst, bytes, vectors_per_thread, threads_per_block, policy, lds_bytes,
                        static_cast<hipStream_t>(stream));
}

// Run the MFMA loop on `blocks` blocks of 256 threads for `iters` rounds;
// out must hold blocks * 256 floats.  Flops = blocks * 4 * iters * 2 * 32768.
extern "C" int kfm_mfma_bf16(float* out, int64_t blocks, int iters, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(out && blocks > 0 && blocks <= 0x7fffffff && iters > 0, KF_E_INVALID,
               "mfma: bad arguments");
    hipLaunchKernelGGL(mfma_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       out, iters);
    return check_launch("mfma_kernel launch");
}
