// Hardware probes behind the issue-rate and LDS-rate figures in the design
// notes: how much VALU work a wavefront issues under its own MFMAs, and the
// LDS read rate per CU.  They are measurement code only, built into their
// own library (libkernelforge_amd_probes.so) that `bench.py --only
// coissue|lds_rate` loads; the product library does not contain them.
#include "../kf_common.h"

namespace kf {
namespace {

// Co-issue probe: one wavefront per SIMD (256-thread blocks, one per CU)
// runs `iters` rounds of 8 v_mfma_f32_32x32x16_bf16 on two independent
// accumulators (one when ONE: each MFMA waits for the previous one's result),
// with K independent VALU instructions (v_fma_f32, or v_exp_f32
// when EXP) after each MFMA; sched_barrier fences keep that order.  Each
// wavefront's lane 0 stores the shader-clock cycles of its loop in
// cycles[block * 4 + wave].  Compared with K = 0, the cycles per MFMA show how
// much of a wavefront's own VALU work issues in the shadow of its MFMAs.
template <int K, bool EXP, bool ONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void coissue_kernel(float* __restrict__ out, long long* __restrict__ cycles, int iters) {
    V<bf16>::x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (bf16)(threadIdx.x * 0.001f + i);
        b[i] = (bf16)(i * 0.5f);
    }
    f32x16 c0 = {}, c1 = {};
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = threadIdx.x * 1e-3f + i * 1e-2f;
    const float m = 0.999f + threadIdx.x * 1e-9f;
    auto valu = [&]() {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if constexpr (EXP)
                x[i % 8] = __builtin_amdgcn_exp2f(x[i % 8]);
            else
                x[i % 8] = __builtin_fmaf(x[i % 8], m, 0.5f);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
    const long long t0 = clock64();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            c0 = mfma32x32x16(a, b, c0);
            __builtin_amdgcn_sched_barrier(0);
            valu();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (ONE)
                c0 = mfma32x32x16(a, b, c0);
            else
                c1 = mfma32x32x16(a, b, c1);
            __builtin_amdgcn_sched_barrier(0);
            valu();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const long long t1 = clock64();
    __builtin_amdgcn_sched_barrier(0);
    if ((threadIdx.x & 63) == 0) cycles[(int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)] = t1 - t0;
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) r += c0[i] + c1[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) r += x[i];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = r;
}

// LDS read-rate probe: each wavefront issues `iters` rounds of 8 reads of a
// 64 KiB LDS buffer at addresses free of bank conflicts (16 lanes x 16 bytes
// on 16 rows for ds_read_b128; 4-lane groups on 32 contiguous bytes of one
// row each for ds_read_b64_tr_b16), folding the data into one value.  Each
// wavefront's lane 0 stores the shader-clock cycles of its loop in
// cycles[block * waves + wave].
template <bool TR>
__global__ __launch_bounds__(1024) void lds_rate_kernel(unsigned* __restrict__ out, long long* __restrict__ cycles,
                                                        int iters) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[65536];
    for (int i = threadIdx.x; i < 65536 / 16; i += blockDim.x)
        reinterpret_cast<u32x4*>(lds)[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 acc = {0u, 0u, 0u, 0u};
    __builtin_amdgcn_sched_barrier(0);
    const long long t0 = clock64();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int tile = ((it * 8 + j + wave * 5) & 15) * 4096;
            if constexpr (TR) {
                const int row = lane >> 2, seg = ((lane & 3) + 4 * ((j + wave) & 1)) * 8;
                const int off = tile + row * 256 + ((seg + 32 * (row & 7)) & 255);
                typedef short s4 __attribute__((ext_vector_type(4)));
                const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(lds + off));
                acc[j & 3] ^= (unsigned)(unsigned short)v[0] ^ ((unsigned)(unsigned short)v[1] << 16) ^
                              (unsigned)(unsigned short)v[2] ^ (unsigned)(unsigned short)v[3];
            } else {
                const int row = lane & 15, ch = (lane >> 4) ^ row;
                const int off = tile + row * 256 + (((ch + 4 * (j & 3)) & 15) << 4);
                acc ^= *reinterpret_cast<const u32x4*>(lds + off);
            }
        }
    }
    const unsigned folded = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    const long long t1 = clock64();
    __builtin_amdgcn_sched_barrier(0);
    if (lane == 0) cycles[(int64_t)blockIdx.x * (blockDim.x >> 6) + wave] = t1 - t0;
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = folded;
}

}  // namespace
}  // namespace kf

// Co-issue probe (see coissue_kernel): `blocks` blocks of 256 threads, each
// wavefront issuing 8 * iters MFMAs; valu_per_mfma in {0, 1, 2, 3, 4, 6, 8},
// exp != 0 for v_exp_f32 instead of v_fma_f32, chains 1 or 2 accumulators
// (1 only with valu_per_mfma = 0); out must hold blocks * 256 floats and
// cycles blocks * 4 values.
extern "C" int kfm_coissue(float* out, long long* cycles, int64_t blocks, int iters, int valu_per_mfma, int exp,
                           int chains, kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(out && cycles && blocks > 0 && blocks <= 0x7fffffff && iters > 0 &&
                   (chains == 2 || (chains == 1 && valu_per_mfma == 0)),
               KF_E_INVALID, "coissue: bad arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 g((unsigned)blocks), t(256);
#define KF_COISSUE(K)                                                                  \
    case K:                                                                            \
        if (exp)                                                                       \
            hipLaunchKernelGGL((coissue_kernel<K, true, false>), g, t, 0, s, out, cycles, iters);   \
        else                                                                           \
            hipLaunchKernelGGL((coissue_kernel<K, false, false>), g, t, 0, s, out, cycles, iters);   \
        break;
    if (chains == 1) {
        hipLaunchKernelGGL((coissue_kernel<0, false, true>), g, t, 0, s, out, cycles, iters);
        return check_launch("coissue_kernel launch");
    }
    switch (valu_per_mfma) {
        KF_COISSUE(0) KF_COISSUE(1) KF_COISSUE(2) KF_COISSUE(3) KF_COISSUE(4) KF_COISSUE(6) KF_COISSUE(8)
        default: set_error("coissue: valu_per_mfma %d not built", valu_per_mfma); return KF_E_INVALID;
    }
#undef KF_COISSUE
    return check_launch("coissue_kernel launch");
}

// LDS read-rate probe (see lds_rate_kernel): `blocks` blocks of 64 * waves
// threads (waves in 1..16), transposing != 0 for ds_read_b64_tr_b16; out must
// hold blocks * 64 * waves words and cycles blocks * waves values.  Bytes
// read = blocks * waves * 64 * iters * 8 * (16 or 8).
extern "C" int kfm_lds_rate(unsigned* out, long long* cycles, int64_t blocks, int waves, int iters, int transposing,
                            kf_stream_t stream) {
    using namespace kf;
    KF_REQUIRE(out && cycles && blocks > 0 && blocks <= 0x7fffffff && waves >= 1 && waves <= 16 && iters > 0, KF_E_INVALID,
               "lds_rate: bad arguments");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (transposing)
        hipLaunchKernelGGL(lds_rate_kernel<true>, dim3((unsigned)blocks), dim3(64 * waves), 0, s, out, cycles, iters);
    else
        hipLaunchKernelGGL(lds_rate_kernel<false>, dim3((unsigned)blocks), dim3(64 * waves), 0, s, out, cycles, iters);
    return check_launch("lds_rate_kernel launch");
}
