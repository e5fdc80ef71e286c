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
// RMSNorm kernel.  All VPT loads are issued before the first store.  On
// MI355X one-wavefront blocks with one vector per lane stream fastest (3-5%
// above 256-thread blocks at 64-256 MiB; more vectors per lane, larger
// blocks and other block-to-XCD orders were slower).
template <int VPT, int BS>
__global__ __launch_bounds__(BS) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                  int64_t nvec) {
    const int64_t base = (int64_t)blockIdx.x * BS * VPT + threadIdx.x;
    u32x4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int64_t j = base + (int64_t)i * BS;
        v[i] = j < nvec ? __builtin_nontemporal_load(src + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int64_t j = base + (int64_t)i * BS;
        if (j < nvec) __builtin_nontemporal_store(v[i], dst + j);
    }
}

template <int BS>
int launch_copy(int vpt, const u32x4* in, u32x4* o, int64_t nvec, hipStream_t s) {
    const int64_t blocks = (nvec + (int64_t)BS * vpt - 1) / ((int64_t)BS * vpt);
    KF_REQUIRE(blocks <= 0x7fffffff, KF_E_UNSUPPORTED, "copy: too many blocks");
    switch (vpt) {
        case 1: hipLaunchKernelGGL((copy_kernel<1, BS>), dim3((unsigned)blocks), dim3(BS), 0, s, in, o, nvec); break;
        case 2: hipLaunchKernelGGL((copy_kernel<2, BS>), dim3((unsigned)blocks), dim3(BS), 0, s, in, o, nvec); break;
        case 4: hipLaunchKernelGGL((copy_kernel<4, BS>), dim3((unsigned)blocks), dim3(BS), 0, s, in, o, nvec); break;
        case 8: hipLaunchKernelGGL((copy_kernel<8, BS>), dim3((unsigned)blocks), dim3(BS), 0, s, in, o, nvec); break;
        default: set_error("copy: vectors_per_thread must be 1, 2, 4 or 8, got %d", vpt); return KF_E_INVALID;
    }
    return check_launch("copy_kernel launch");
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
    KF_REQUIRE(bytes >= 0 && bytes % 16 == 0, KF_E_INVALID, "copy: bytes %lld not a multiple of 16",
               (long long)bytes);
    KF_REQUIRE(bytes == 0 || (src && dst && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0),
               KF_E_INVALID, "copy: null or unaligned pointer");
    KF_REQUIRE(threads_per_block == 64 || threads_per_block == 256, KF_E_INVALID,
               "copy: threads_per_block must be 64 or 256, got %d", threads_per_block);
    if (bytes == 0) return KF_OK;
    const int64_t nvec = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const u32x4* in = static_cast<const u32x4*>(src);
    u32x4* o = static_cast<u32x4*>(dst);
    return threads_per_block == 64 ? launch_copy<64>(vectors_per_thread, in, o, nvec, s)
                                   : launch_copy<256>(vectors_per_thread, in, o, nvec, s);
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
