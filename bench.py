"""Benchmark of the kernelforge_amd hot paths on one MI355X.

Prints ONE JSON line.  The headline ("value") is BASELINE config 1: RMSNorm
bf16 on x[16384, 4096] (one step = one RMSNorm pass), in HBM GB/s of
algorithmic traffic (read x once, write y once, read w).  The same line
carries, under "results", every BASELINE config measured the same way:
the RMSNorm hidden sweep {2048, 4096, 8192}, SANA linear attention at both
shapes (HBM GB/s and TFLOP/s), and FlashAttention at B=2, H=16, N=4096,
D=128 (fused forward+JVP, standalone JVP from LSE, forward, backward), in
TFLOP/s against the bf16 dense MFMA peak.

Timing: each workload is timed as the median of 5 batches of K launches
(the per-batch times are in "repeats_us"); the headline RMSNorm line times
exactly one batch of K steps.  Inputs are resident in HBM before the timed region; input/output
sets rotate so that the bytes touched between two uses of a buffer exceed
the 256 MB Infinity Cache; the timed region is bracketed by
torch.cuda.synchronize() and measured with HIP events recorded on the
stream the kernels are launched on (torch's current stream).  Warm-up: the W
untimed launches, then more untimed launches until 100 ms of the workload
have run on the GPU, because the clocks keep ramping for tens of
milliseconds after an idle period (measured on MI355X: the first 9 ms after
a 10-launch warm-up ran 4-6% slower than the steady state, the first ~90 ms
of the fused FA kernel 7% slower; the rate after that stayed within 0.3%
over two seconds of back-to-back launches).  The line reports the requested
W as "warmup", and the headline's untimed launches in total (W plus the
settling ones) as "warmup_launches".

The CPU baseline times the oracle (a plain-torch restatement of the
reference original.py, test infrastructure) on the host cores on a bounded
sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu] [--settle-ms MS]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

BASELINE_METRIC = "RMSNorm HBM GB/s; lin-attn & FA-JVP TFLOP/s as % roofline; speedup vs ref"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 * 2**20


def _sets_for(bytes_per_set: int) -> int:
    """Number of rotating buffer sets so that a full rotation exceeds 2x the MALL."""
    return max(2, min(16, -(-2 * MALL_BYTES // max(1, bytes_per_set)) + 1))


SETTLE_MS = 100.0
# Timed batches per workload (the median is reported, the batches are kept in
# `repeats_us`); the headline RMSNorm line times exactly one batch of K steps.
REPEATS = 5
LAST_REPEATS: list = []


def _time_launches(fn, n_sets: int, steps: int, warmup: int, repeats: int | None = None) -> tuple[float, int]:
    """(microseconds per launch of fn(set_index), untimed launches before the
    timed ones): `warmup` launches, then batches of about 10 ms each until
    SETTLE_MS of GPU time has run, then `repeats` timed batches of `steps`
    launches each; the result is the median batch.  The per-batch figures are
    kept in LAST_REPEATS."""
    global LAST_REPEATS
    repeats = REPEATS if repeats is None else repeats
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_warm = 0
    for _ in range(warmup):
        fn(n_warm % n_sets)
        n_warm += 1
    torch.cuda.synchronize()
    settled, batch = 0.0, 1
    while settled < SETTLE_MS:
        start.record()
        for _ in range(batch):
            fn(n_warm % n_sets)
            n_warm += 1
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        settled += ms
        batch = max(1, min(4 * batch, int(batch * 10.0 / max(ms, 1e-3))))
    per = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            fn(i % n_sets)
        end.record()
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) * 1000.0 / steps)
    LAST_REPEATS = per
    return sorted(per)[len(per) // 2], n_warm


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# Workloads (GPU).  Each returns a dict with the per-launch time and rates.
# ---------------------------------------------------------------------------
def bench_rmsnorm(hidden: int, steps: int, warmup: int, rows: int = 16384, repeats: int | None = None) -> dict:
    from kernelforge_amd import _lib

    lib = _lib.load()
    bytes_per_launch = 2 * rows * hidden * 2 + hidden * 2
    n_sets = _sets_for(bytes_per_launch)
    g = _gen(hidden)
    xs = [torch.randn(rows, hidden, generator=g).to(torch.bfloat16).to("cuda") for _ in range(n_sets)]
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to("cuda")
    ys = [torch.empty_like(x) for x in xs]
    stream = _lib.stream_of(xs[0])
    args = [(_lib.ptr(xs[i]), _lib.ptr(w), _lib.ptr(ys[i])) for i in range(n_sets)]
    fnc = lib.kf_rmsnorm_fwd

    def launch(i):
        x, wp, y = args[i]
        rc = fnc(x, wp, y, rows, hidden, 1e-6, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_rmsnorm_fwd")

    us, n_warm = _time_launches(launch, n_sets, steps, warmup, repeats)
    gbs = bytes_per_launch / (us * 1e-6) / 1e9
    return dict(kernel="rmsnorm_vec_kernel", workload=f"rmsnorm_bf16_{rows}x{hidden}", us=us,
                warmup_launches=n_warm, steps=steps,
                bytes=bytes_per_launch, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, sets=n_sets)


def bench_sana(B: int, H: int, N: int, steps: int, warmup: int, D: int = 32) -> dict:
    from kernelforge_amd import _lib

    lib = _lib.load()
    C = H * D
    bytes_per_launch = 3 * B * N * C * 2 + B * N * C * 2
    flops = 4 * B * H * N * D * (D + 1)
    n_sets = _sets_for(bytes_per_launch)
    g = _gen(N + B)
    qkvs = [torch.randn(B, N, 3, C, generator=g).to(torch.bfloat16).to("cuda") for _ in range(n_sets)]
    outs = [torch.empty(B, N, C, device="cuda", dtype=torch.bfloat16) for _ in range(n_sets)]
    splits = int(lib.kf_linattn_default_splits(B, H, D, N))
    ws_bytes = int(lib.kf_linattn_workspace_bytes(B, H, D, splits))
    ws = torch.empty(ws_bytes, device="cuda", dtype=torch.uint8)
    stream = _lib.stream_of(ws)
    _lib.check(lib.kf_linattn_workspace_init(_lib.ptr(ws), ws_bytes, stream), "kf_linattn_workspace_init")
    args = [(_lib.ptr(qkvs[i]), _lib.ptr(outs[i])) for i in range(n_sets)]
    wsp = _lib.ptr(ws)
    fnc = lib.kf_linattn_fwd

    def launch(i):
        q, o = args[i]
        rc = fnc(q, o, wsp, ws_bytes, B, N, H, D, splits, 1e-15, _lib.KF_BF16, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_linattn_fwd")

    us, n_warm = _time_launches(launch, n_sets, steps, warmup)
    gbs = bytes_per_launch / (us * 1e-6) / 1e9
    tflops = flops / (us * 1e-6) / 1e12
    return dict(kernel="linattn_fused_kernel", workload=f"sana_bf16_B{B}_H{H}_D{D}_N{N}", us=us,
                warmup_launches=n_warm, steps=steps,
                bytes=bytes_per_launch, flops=flops, gbs=gbs, tflops=tflops,
                roofline_frac=gbs / HBM_PEAK_GBS, mfma_frac=tflops / BF16_PEAK_TFLOPS, splits=splits,
                sets=n_sets)


def bench_fa(mode: str, steps: int, warmup: int, B=2, H=16, N=4096, D=128) -> dict:
    from kernelforge_amd import _lib

    lib = _lib.load()
    g = _gen(7)
    shape = (B, N, H, D)
    q, k, v, tq, tk, tv = (torch.randn(shape, generator=g).to(torch.bfloat16).to("cuda") for _ in range(6))
    o = torch.empty_like(q)
    to = torch.empty_like(q)
    lse = torch.empty(B, H, N, device="cuda", dtype=torch.float32)
    scale = D ** -0.5
    stream = _lib.stream_of(q)
    P = [_lib.ptr(x) for x in (q, k, v, tq, tk, tv, o, lse, to)]
    dims = (B, N, N, H, H, D, scale, 0, _lib.KF_BF16, stream)
    if mode == "fwd_jvp":
        fnc, a = lib.kf_fa_fwd_jvp, (*P, *dims)
        gemms, executed, name = 6, 6, "fa_kernel<bf16,128,FWD_JVP>"
    elif mode == "jvp":
        # JVP from the cached O and LSE: 5 GEMM-equivalents (S, tq.k, q.tk,
        # H.v, P.tv), as executed.  Rows whose rowsum(H)/l could amplify the
        # cached O's rounding past the kernel's bound are redone by the second
        # launch with U = P.v recomputed; at scale 1/sqrt(D) on unit-normal
        # inputs no row reaches the bound, so that launch only reads markers.
        rc = lib.kf_fa_fwd(P[0], P[1], P[2], P[6], P[7], *dims)
        _lib.check(rc, "kf_fa_fwd")
        fnc, a = lib.kf_fa_jvp, (*P, *dims)
        gemms, executed, name = 5, 5, "fa_kernel<bf16,128,JVP>"
    elif mode == "bwd":
        # Backward from the forward's O and LSE: dq kernel + dkdv kernel.  The
        # algorithmic count is the usual 5 GEMM-equivalents (S recomputed
        # once, dP, dV, dK, dQ); the kernels recompute S and dP twice.
        rc = lib.kf_fa_fwd(P[0], P[1], P[2], P[6], P[7], *dims)
        _lib.check(rc, "kf_fa_fwd")
        dout = torch.randn(shape, generator=g).to(torch.bfloat16).to("cuda")
        grads = [torch.empty_like(x) for x in (q, k, v)]
        ws_bytes = lib.kf_fa_bwd_workspace_bytes(B, N, H, D)
        ws = torch.empty(ws_bytes, device="cuda", dtype=torch.uint8)
        fnc = lib.kf_fa_bwd
        a = (P[0], P[1], P[2], P[6], P[7], _lib.ptr(dout), *(_lib.ptr(x) for x in grads), _lib.ptr(ws),
             ws_bytes, *dims)
        gemms, executed, name = 5, 7, "fa_bwd_dq_kernel+fa_bwd_dkdv_wide_kernel<bf16,128>"
    else:
        fnc, a = lib.kf_fa_fwd, (P[0], P[1], P[2], P[6], P[7], *dims)
        gemms, executed, name = 2, 2, "fa_kernel<bf16,128,FWD>"

    def launch(_):
        rc = fnc(*a)
        if rc:
            _lib.check(rc, name)

    us, n_warm = _time_launches(launch, 1, steps, warmup)
    flops = 2 * gemms * B * H * N * N * D
    tflops = flops / (us * 1e-6) / 1e12
    return dict(kernel=name, workload=f"fa_{mode}_bf16_B{B}_H{H}_N{N}_D{D}", us=us, flops=flops,
                warmup_launches=n_warm, steps=steps,
                gemm_equivalents=gemms, executed_gemm_equivalents=executed,
                executed_tflops=tflops * executed / gemms, tflops=tflops,
                roofline_frac=tflops / BF16_PEAK_TFLOPS)


def bench_proj(kind: str, B: int, N: int, C: int, steps: int, warmup: int) -> dict:
    """SANA projection GEMM (kf_proj_gemm, nn.Linear weight layout): "qkv" is
    x[B*N, C] . W[3C, C]^T without bias, "out" is x . W[C, C]^T + bias.  The
    same product through torch.matmul / torch.addmm (hipBLASLt) is timed
    beside it as "library_us" (a reference point, not part of this build)."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    M, K = B * N, C
    n_out = 3 * C if kind == "qkv" else C
    g = _gen(11)
    w = (torch.randn(n_out, K, generator=g) / K ** 0.5).to(torch.bfloat16).to("cuda")
    bias = torch.randn(n_out, generator=g).to(torch.bfloat16).to("cuda") if kind == "out" else None
    n_sets = _sets_for(M * K * 2 + M * n_out * 2)
    xs = [torch.randn(M, K, generator=g).to(torch.bfloat16).to("cuda") for _ in range(n_sets)]
    ys = [torch.empty(M, n_out, device="cuda", dtype=torch.bfloat16) for _ in range(n_sets)]
    stream = _lib.stream_of(xs[0])
    bp = _lib.ptr(bias)

    def launch(i):
        rc = lib.kf_proj_gemm(_lib.ptr(xs[i]), _lib.ptr(w), bp, _lib.ptr(ys[i]), M, n_out, K, K, n_out,
                              _lib.KF_WEIGHT_NK, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_proj_gemm")

    us, n_warm = _time_launches(launch, n_sets, steps, warmup)
    kernel_repeats = list(LAST_REPEATS)
    wt = w.t()

    def library(i):
        if bias is None:
            torch.matmul(xs[i], wt, out=ys[i])
        else:
            torch.addmm(bias, xs[i], wt, out=ys[i])

    lib_us, _ = _time_launches(library, n_sets, steps, warmup)
    flops = 2 * M * n_out * K
    tflops = flops / (us * 1e-6) / 1e12
    return dict(repeats_us=[round(x, 3) for x in kernel_repeats], kernel="proj_gemm_kernel",
                workload=f"proj_{kind}_bf16_M{M}_N{n_out}_K{K}", us=us, flops=flops,
                warmup_launches=n_warm, steps=steps, sets=n_sets, tflops=tflops,
                roofline_frac=tflops / BF16_PEAK_TFLOPS, library_us=lib_us,
                library_tflops=flops / (lib_us * 1e-6) / 1e12)


def bench_litela(B: int, N: int, H: int, steps: int, warmup: int) -> dict:
    """LiteLA attention with the QKV projection fused in (kf_litela_fused_attn:
    x[B, N, 32H] -> the attention output before the output projection, q, k
    and v never written to HBM), head dim 32, bf16.  The unfused pair -- the
    projection GEMM (kf_proj_gemm) into a packed qkv, then kf_linattn_fwd --
    is timed beside it as "unfused_us".  Flops: the projection's 2 M 3C C plus
    the attention's 4 B H N D (D + 1); the projection dominates, so the
    roofline is the dense bf16 MFMA peak."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    D, C = 32, 32 * H
    M = B * N
    g = _gen(13)
    w = (torch.randn(3 * C, C, generator=g) / C ** 0.5).to(torch.bfloat16).to("cuda")
    n_sets = _sets_for(M * C * 2 * 5)
    xs = [torch.randn(B, N, C, generator=g).to(torch.bfloat16).to("cuda") for _ in range(n_sets)]
    outs = [torch.empty(B, N, C, device="cuda", dtype=torch.bfloat16) for _ in range(n_sets)]
    stream = _lib.stream_of(xs[0])
    wsb = lib.kf_litela_fused_workspace_bytes(B, N, H)
    ws = torch.empty(max(wsb, 256), device="cuda", dtype=torch.uint8)

    def fused(i):
        rc = lib.kf_litela_fused_attn(_lib.ptr(xs[i]), _lib.ptr(w), None, _lib.ptr(outs[i]), _lib.ptr(ws), wsb,
                                      B, N, H, D, 1e-15, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_litela_fused_attn")

    us, n_warm = _time_launches(fused, n_sets, steps, warmup)
    repeats = list(LAST_REPEATS)
    qkv = torch.empty(B, N, 3 * C, device="cuda", dtype=torch.bfloat16)
    splits = lib.kf_linattn_default_splits(B, H, D, N)
    lwsb = lib.kf_linattn_workspace_bytes(B, H, D, splits)
    lws = torch.zeros(max(lwsb, 256), device="cuda", dtype=torch.uint8)

    def unfused(i):
        rc = lib.kf_proj_gemm(_lib.ptr(xs[i]), _lib.ptr(w), None, _lib.ptr(qkv), M, 3 * C, C, C, 3 * C,
                              _lib.KF_WEIGHT_NK, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_proj_gemm")
        rc = lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(outs[i]), _lib.ptr(lws), lwsb, B, N, H, D, splits, 1e-15,
                                _lib.KF_BF16, _lib.KF_BF16, stream)
        if rc:
            _lib.check(rc, "kf_linattn_fwd")

    unfused_us, _ = _time_launches(unfused, n_sets, steps, warmup)
    flops = 2 * M * 3 * C * C + 4 * B * H * N * D * (D + 1)
    tflops = flops / (us * 1e-6) / 1e12
    return dict(repeats_us=[round(x, 3) for x in repeats], kernel="litela_fused",
                workload=f"litela_fused_bf16_B{B}_H{H}_N{N}", us=us, flops=flops, warmup_launches=n_warm,
                steps=steps, sets=n_sets, tflops=tflops, roofline_frac=tflops / BF16_PEAK_TFLOPS,
                unfused_us=unfused_us, speedup_vs_unfused=unfused_us / us)


def bench_copy(nbytes: int, steps: int, warmup: int) -> dict:
    """HBM stream ceiling: the library's 16-byte-per-lane copy kernel (kfm_copy,
    kernelforge_amd/csrc/measure.hip) reading and writing `nbytes` each, the
    traffic of one RMSNorm launch; the best of one-wavefront blocks with one
    vector per lane and 256-thread blocks with 1, 2 and 4."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    n_sets = _sets_for(2 * nbytes)
    src = [torch.empty(nbytes // 2, device="cuda", dtype=torch.bfloat16).normal_() for _ in range(n_sets)]
    dst = [torch.empty_like(x) for x in src]
    stream = _lib.stream_of(src[0])
    ptrs = [(_lib.ptr(src[i]), _lib.ptr(dst[i])) for i in range(n_sets)]
    best = None
    for vpt, threads in ((1, 64), (1, 256), (2, 256), (4, 256)):
        def launch(i, vpt=vpt, threads=threads):
            rc = lib.kfm_copy(ptrs[i][0], ptrs[i][1], nbytes, vpt, threads, stream)
            if rc:
                _lib.check(rc, "kfm_copy")

        us, n_warm = _time_launches(launch, n_sets, steps, warmup)
        if best is None or us < best["us"]:
            best = dict(repeats_us=[round(x, 3) for x in LAST_REPEATS], kernel="copy_kernel",
                        workload=f"copy_{nbytes >> 20}MiB", vectors_per_lane=vpt, threads_per_block=threads,
                        bytes=2 * nbytes, us=us, warmup_launches=n_warm, steps=steps)
    best["gbs"] = best["bytes"] / (best["us"] * 1e-6) / 1e9
    best["frac_of_peak"] = best["gbs"] / HBM_PEAK_GBS
    return best


def bench_copy_sweep(steps: int, warmup: int) -> dict:
    """Stream-ceiling sweep behind the copy ceiling (kfm_copy_ex): at the
    three RMSNorm traffic sizes (64, 128 and 256 MiB read and written), every
    block size (64, 256, 1024 threads) x vectors per lane (1, 2, 4, 8) x cache
    policy (nontemporal or plain loads and stores), then the fastest shape of
    each size with dynamic LDS capping the blocks per CU.  Microseconds per
    launch and the fraction of 8 TB/s; the best entry per size."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    policies = {0: "nt/nt", 1: "plain/nt", 2: "nt/plain", 3: "plain/plain"}
    out = {}
    for nbytes in (16384 * 2048 * 2, 16384 * 4096 * 2, 16384 * 8192 * 2):
        n_sets = _sets_for(2 * nbytes)
        src = [torch.empty(nbytes // 2, device="cuda", dtype=torch.bfloat16).normal_() for _ in range(n_sets)]
        dst = [torch.empty_like(x) for x in src]
        stream = _lib.stream_of(src[0])
        ptrs = [(_lib.ptr(src[i]), _lib.ptr(dst[i])) for i in range(n_sets)]

        def run(vpt, threads, pol, lds):
            # A one-block copy first: it separates consecutive configurations
            # of the same kernel and grid in a kernel trace.
            _lib.check(lib.kfm_copy_ex(ptrs[0][0], ptrs[0][1], 16, 1, 64, 0, 0, stream), "kfm_copy_ex")

            def launch(i):
                rc = lib.kfm_copy_ex(ptrs[i][0], ptrs[i][1], nbytes, vpt, threads, pol, lds, stream)
                if rc:
                    _lib.check(rc, "kfm_copy_ex")

            us, _ = _time_launches(launch, n_sets, steps, warmup)
            return dict(threads=threads, vectors_per_lane=vpt, policy=policies[pol], lds_bytes=lds,
                        us=round(us, 3), frac_of_peak=round(2 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))

        rows = [run(vpt, threads, pol, 0) for threads in (64, 256, 1024) for vpt in (1, 2, 4, 8)
                for pol in (0, 1, 2, 3)]
        best = min(rows, key=lambda r: r["us"])
        # Occupancy caps for the fastest shape: blocks per CU limited to about
        # 160 KiB / lds_bytes.
        for lds in (5 * 1024, 10 * 1024, 20 * 1024, 40 * 1024):
            rows.append(run(best["vectors_per_lane"], best["threads"],
                            {v: k for k, v in policies.items()}[best["policy"]], lds))
        best = min(rows, key=lambda r: r["us"])
        out[f"copy_{nbytes >> 20}MiB"] = dict(bytes=2 * nbytes, best=best, rows=rows)
        print(f"# copy sweep {nbytes >> 20} MiB: best {best}", file=sys.stderr, flush=True)
        del src, dst
    return dict(kernel="copy_kernel", workload="copy_sweep", us=0.0, sizes=out)


def bench_mfma(warmup: int) -> dict:
    """Dense bf16 MFMA ceiling: kfm_mfma_bf16 (two independent
    v_mfma_f32_32x32x16_bf16 chains per wavefront) at 1, 2 and 4 wavefronts
    per SIMD, each run ~1-2 ms; the best rate."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 8192
    best = None
    for waves_per_simd in (1, 2, 4):
        blocks = cus * waves_per_simd  # 4 wavefronts (one per SIMD) per block
        out = torch.empty(blocks * 256, device="cuda", dtype=torch.float32)
        stream = _lib.stream_of(out)

        def launch(_):
            rc = lib.kfm_mfma_bf16(_lib.ptr(out), blocks, iters, stream)
            if rc:
                _lib.check(rc, "kfm_mfma_bf16")

        us, _ = _time_launches(launch, 1, 5, warmup)
        flops = blocks * 4 * iters * 2 * 32768
        tflops = flops / (us * 1e-6) / 1e12
        if best is None or tflops > best["tflops"]:
            best = dict(repeats_us=[round(x, 3) for x in LAST_REPEATS], kernel="mfma_kernel",
                        workload="mfma_bf16_32x32x16_dense", waves_per_simd=waves_per_simd,
                        us=us, flops=flops, tflops=tflops, frac_of_peak=tflops / BF16_PEAK_TFLOPS)
    return best


def bench_coissue(warmup: int) -> dict:
    """How much of a wavefront's own VALU work issues under its MFMAs:
    kfm_coissue at one wavefront per SIMD (one 256-thread block per CU), two
    independent v_mfma_f32_32x32x16_bf16 chains with K = 0..8 independent
    v_fma_f32 or v_exp_f32 after each MFMA, and one dependent chain with no
    VALU work ("one_chain").  Cycles come from the shader clock inside the
    kernel (median over wavefronts); extra_cycles_per_valu =
    (cycles_K - cycles_0) / K per MFMA."""
    from kernelforge_amd import _lib

    lib = _lib.load_probes()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 4096  # x 8 MFMAs per wavefront
    out = torch.empty(cus * 256, device="cuda", dtype=torch.float32)
    cyc = torch.zeros(cus * 4, device="cuda", dtype=torch.int64)
    stream = _lib.stream_of(out)
    res = dict(kernel="coissue_kernel", workload="mfma32x32x16_plus_valu", waves_per_simd=1,
               mfma_per_wave=8 * iters)

    def run(k, exp, chains):
        def launch(_):
            rc = lib.kfm_coissue(_lib.ptr(out), _lib.ptr(cyc), cus, iters, k, exp, chains, stream)
            if rc:
                _lib.check(rc, "kfm_coissue")

        us, _ = _time_launches(launch, 1, 5, warmup)
        c = cyc.double().median().item() / (8 * iters)
        return dict(cycles_per_mfma=round(c, 2), ns_per_mfma=round(us * 1e3 / (8 * iters), 3),
                    clock_ghz=round(c / (us * 1e3 / (8 * iters)), 3))

    res["one_chain"] = run(0, 0, 1)
    for kind, exp in (("fma", 0), ("exp", 1)):
        rows = {k: run(k, exp, 2) for k in (0, 1, 2, 3, 4, 6, 8)}
        for k in rows:
            rows[k]["extra_cycles_per_valu"] = (round((rows[k]["cycles_per_mfma"] - rows[0]["cycles_per_mfma"]) / k, 2)
                                                if k else None)
        res[kind] = {str(k): v for k, v in rows.items()}
    res["us"] = res["fma"]["0"]["ns_per_mfma"] * 8 * iters / 1e3
    return res


def bench_lds_rate(warmup: int) -> dict:
    """LDS read issue rate per CU: kfm_lds_rate with 4, 8 and 16 wavefronts per
    CU (one block per CU), conflict-free ds_read_b128 against
    ds_read_b64_tr_b16.  cycles_per_instr_per_cu = the slowest wavefront's
    shader-clock cycles (median over blocks) / the block's read instructions."""
    from kernelforge_amd import _lib

    lib = _lib.load_probes()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 2048
    res = dict(kernel="lds_rate_kernel", workload="lds_reads_conflict_free")
    for waves in (4, 8, 16):
        out = torch.empty(cus * 64 * waves, device="cuda", dtype=torch.int32)
        cyc = torch.zeros(cus * waves, device="cuda", dtype=torch.int64)
        stream = _lib.stream_of(out)
        for name, tr, nbytes in (("b128", 0, 16), ("tr_b64", 1, 8)):
            def launch(_, tr=tr):
                rc = lib.kfm_lds_rate(_lib.ptr(out), _lib.ptr(cyc), cus, waves, iters, tr, stream)
                if rc:
                    _lib.check(rc, "kfm_lds_rate")

            us, _ = _time_launches(launch, 1, 5, warmup)
            c = cyc.view(cus, waves).max(dim=1).values.double().median().item()
            instrs = waves * iters * 8
            res[f"{name}_w{waves}"] = dict(us=round(us, 2), cycles_per_instr_per_cu=round(c / instrs, 3),
                                           bytes_per_cycle_per_cu=round(instrs * 64 * nbytes / c, 1))
    res["tr_over_b128_cycles_w16"] = round(res["tr_b64_w16"]["cycles_per_instr_per_cu"] /
                                           res["b128_w16"]["cycles_per_instr_per_cu"], 3)
    res["us"] = res["b128_w16"]["us"]
    return res


# ---------------------------------------------------------------------------
# CPU baseline (oracle on the host cores, bounded sample).
# ---------------------------------------------------------------------------
def cpu_baselines(rows=16384, hidden=4096) -> dict:
    from oracle import fa as ofa
    from oracle import rmsnorm as orms
    from oracle import sana as osana

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def med(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2]

    out = {}
    g = _gen(1)
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    t = med(lambda: orms.rmsnorm(x, w, 1e-6), 5)
    out["rmsnorm"] = dict(value=(2 * rows * hidden * 2 + hidden * 2) / t / 1e9, unit="GB/s", cores=cores,
                          kind="port", seconds_per_pass=t,
                          sample=f"oracle.rmsnorm on the full bf16 [{rows},{hidden}] input, median of 5")
    qkv = torch.randn(2, 4096, 3, 70 * 32, generator=g).to(torch.bfloat16)
    sana_flops = 4 * 2 * 70 * 4096 * 32 * 33
    t = med(lambda: osana.linear_attention(qkv, 70, 32), 3)
    out["sana"] = dict(value=sana_flops / t / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                       seconds_per_pass=t,
                       sample="oracle.sana.linear_attention (fp32_attention=True) on the full B=2,H=70,N=4096 "
                              "input, median of 3")
    t = med(lambda: osana.linear_attention(qkv, 70, 32, fp32_attention=False), 3)
    out["sana_eager_bf16"] = dict(value=sana_flops / t / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                                  seconds_per_pass=t,
                                  sample="oracle.sana.linear_attention as written with bf16 matmuls "
                                         "(fp32_attention=False) on the full B=2,H=70,N=4096 input, median of 3")
    # FA: one (batch, head) slice of B=2, H=16, N=4096, D=128 (1/32 of the work).
    q, k, v, tq, tk, tv = (torch.randn(1, 4096, 1, 128, generator=g).to(torch.bfloat16) for _ in range(6))
    t = med(lambda: ofa.attention_jvp(q, k, v, tq, tk, tv), 1)
    flops = 12 * 4096 * 4096 * 128
    out["fa"] = dict(value=flops / t / 1e12, unit="TFLOP/s", cores=cores, kind="port", seconds_per_pass=t,
                     seconds_full_config_est=32 * t,
                     sample="oracle.fa.attention_jvp (dense fp32 torch.func.jvp) on 1 of the 32 (b,h) "
                            "slices of B=2,H=16,N=4096,D=128, median of 1 after 1 warm-up")
    out["cpu_model"] = cpu_model()
    return out


def cpu_model() -> str:
    """The host CPU's model name (as lscpu prints it), from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic() -> dict:
    """HBM bytes per launch, "kernel:workload" -> bytes, from rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE scaled by the same counters on a 256 MiB copy (profiles/traffic.json,
    summarised in profiles/hbm_traffic.md).  Keys starting with "_" are metadata."""
    path = ROOT / "profiles" / "traffic.json"
    if path.exists():
        try:
            return json.loads(path.read_text())
        except ValueError:
            return {}
    return {}


def main() -> int:
    global SETTLE_MS
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default=None,
                    help="run one workload only (rmsnorm2048|rmsnorm4096|rmsnorm8192|sanaA|sanaB|"
                         "fa_fwd_jvp|fa_jvp|fa_fwd|fa_bwd|proj_qkvA|proj_outA|litela_fusedA|copy2048|copy4096|copy8192|mfma), "
                         "e.g. under "
                         "rocprofv3, or a probe that the default run skips (coissue|lds_rate: issue rates; "
                         "copy_sweep: the stream-ceiling sweep)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="GPU time of untimed launches after the warm-up steps (clock settling)")
    args = ap.parse_args()
    SETTLE_MS = args.settle_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; run with --gpus 1 (the hot paths are "
              "single-GPU kernels; no run here uses a second GPU)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 2
    torch.cuda.init()
    steps, warmup = args.steps, args.warmup

    runners = {
        "rmsnorm2048": lambda: bench_rmsnorm(2048, steps, warmup),
        "rmsnorm4096": lambda: bench_rmsnorm(4096, steps, warmup, repeats=1),
        "rmsnorm8192": lambda: bench_rmsnorm(8192, steps, warmup),
        "sanaA": lambda: bench_sana(2, 70, 4096, steps, warmup),
        "sanaB": lambda: bench_sana(1, 70, 16384, steps, warmup),
        "fa_fwd_jvp": lambda: bench_fa("fwd_jvp", max(10, steps // 5), max(3, warmup // 2)),
        "fa_jvp": lambda: bench_fa("jvp", max(10, steps // 5), max(3, warmup // 2)),
        "fa_fwd": lambda: bench_fa("fwd", max(10, steps // 5), max(3, warmup // 2)),
        "fa_bwd": lambda: bench_fa("bwd", max(10, steps // 5), max(3, warmup // 2)),
        "proj_qkvA": lambda: bench_proj("qkv", 2, 4096, 2240, steps, warmup),
        "proj_outA": lambda: bench_proj("out", 2, 4096, 2240, steps, warmup),
        "litela_fusedA": lambda: bench_litela(2, 4096, 70, steps, warmup),
        "copy2048": lambda: bench_copy(16384 * 2048 * 2, steps, warmup),
        "copy4096": lambda: bench_copy(16384 * 4096 * 2, steps, warmup),
        "copy8192": lambda: bench_copy(16384 * 8192 * 2, steps, warmup),
        "mfma": lambda: bench_mfma(warmup),
    }
    # Hardware probes behind claims about issue rates; --only runs them, the
    # default run does not.
    probes = {
        "coissue": lambda: bench_coissue(warmup),
        "copy_sweep": lambda: bench_copy_sweep(min(steps, 50), warmup),
        "lds_rate": lambda: bench_lds_rate(warmup),
    }
    if args.only:
        r = {**runners, **probes}[args.only]()
        print(json.dumps(r), flush=True)
        return 0

    results = {}
    for name, fn in runners.items():
        results[name] = fn()
        results[name].setdefault("repeats_us", [round(x, 3) for x in LAST_REPEATS])
        print(f"# {name}: {results[name]['us']:.2f} us", file=sys.stderr, flush=True)
    head = results["rmsnorm4096"]
    traffic = load_traffic()
    tr = traffic.get(head["kernel"] + ":" + head["workload"])
    cpu = None if args.no_cpu else cpu_baselines()
    for name in results:
        if cpu and name == "rmsnorm4096":
            results[name]["speedup_vs_cpu"] = head["gbs"] / cpu["rmsnorm"]["value"]
        if cpu and name == "sanaA":
            results[name]["speedup_vs_cpu_oracle_fp32"] = results[name]["tflops"] / cpu["sana"]["value"]
            results[name]["speedup_vs_cpu_eager_bf16"] = (results[name]["tflops"]
                                                          / cpu["sana_eager_bf16"]["value"])
        if cpu and name == "fa_fwd_jvp":
            results[name]["speedup_vs_cpu"] = results[name]["tflops"] / cpu["fa"]["value"]
        t = traffic.get(results[name]["kernel"] + ":" + results[name]["workload"])
        if t is not None:
            results[name]["traffic_bytes"] = t
        if name.startswith("rmsnorm"):
            ceil = results["copy" + name[len("rmsnorm"):]]["gbs"]
            results[name]["frac_of_copy_ceiling"] = results[name]["gbs"] / ceil
        if name.startswith("fa_"):
            results[name]["frac_of_mfma_ceiling"] = results[name]["tflops"] / results["mfma"]["tflops"]
    line = {
        "metric": BASELINE_METRIC,
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": warmup,
        "warmup_launches": head["warmup_launches"],
        "settle_ms": SETTLE_MS,
        "ms_per_step": head["us"] / 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": head["workload"], "rows": 16384, "hidden": 4096, "eps": 1e-6,
                   "input_sets_rotated": head["sets"]},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": tr,
                     "algorithmic_bytes": head["bytes"], "kernel": head["kernel"],
                     "frac_of_copy_ceiling": round(head["frac_of_copy_ceiling"], 4)},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["rmsnorm"]["value"], 3), "unit": "GB/s", "cores": cpu["rmsnorm"]["cores"],
            "kind": "port", "sample": cpu["rmsnorm"]["sample"]},
        "results": results,
        "cpu_baselines": cpu,
        "copy_ceiling_gbs": round(results["copy4096"]["gbs"], 1),
        "mfma_ceiling_tflops": round(results["mfma"]["tflops"], 1),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
