#!/usr/bin/env python3
"""Benchmark of the hot path: batched C2C FFT, N=1024, batch 65536 (the headline workload).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--cpu-seconds S]
                    [--prewarm-ms M] [--settle-ms S] [--sweep]

One step = one ThunderFFT_global launch (the C ABI's asynchronous entry,
thff_global_async) over the whole batch of 65536 signals of N=1024, inputs
resident in HBM (generated on the device by thff_fill_uniform).  Before the
first leg, M ms (default 250) of untimed launches bring the device to the
clocks later legs see (prewarm_s in the output).  Per leg: W untimed steps,
then untimed steps filling about S ms (default 60; settle_ms in the output,
so that a heavy kernel is timed at its steady clocks rather than the
transient after a pause), then K steps back to back between two HIP events
recorded on the launch stream, bracketed by device synchronisation;
ms_per_step is the event time / K.  value = GFLOP/s (5 N log2 N per
transform) of the float forward transform; the inverse and the half
transforms are measured the same way and reported under "also".  Each leg
allocates its output right after its input; also.placement_*_n1024 repeats
the forward transform with the output at 8 offsets inside one allocation,
since the time of the fp16 kernels that walk many tiles per workgroup (the
convolutions and the N = 2048, 4096 C2C) depends on where the output lies.

roofline.achieved = algorithmic bytes per launch (read + write of every
complex value once: 2 * batch * N * sizeof(T)) / the mean launch duration
above; roofline.traffic = HBM bytes per launch from the rocprofv3 FETCH_SIZE /
WRITE_SIZE runs summarised in profiles/ (each scaled by what the counter reads
for a plain copy of known size); also.*.mfma_util_pct = rocprofiler's MfmaUtil
for the MFMA kernels, from the rocprofv3 run summarised there too.  cpu_baseline = the oracle's threaded fp32
radix-4 FFT, vectorised across signals (the reference has no CPU FFT), timed on this host's cores on a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

HBM_PEAK_GBPS = 8000.0
N_FFT = 1024
BATCH = 65536
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "pmc_c2c_n1024_b65536.md")
MFMA_PROFILE = os.path.join(ROOT, "profiles", "pmc_mfma_c2c_n1024_b65536.md")


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-fp64-check", action="store_true",
                    help="skip the timed host fp64 check of the GPU output")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target wall time of the CPU baseline sample")
    ap.add_argument("--prewarm-ms", type=float, default=250.0,
                    help="untimed device warm-up before the first timed leg (ms of back-to-back "
                         "launches of that leg's kernel)")
    ap.add_argument("--settle-ms", type=float, default=60.0,
                    help="per leg, after its W warm-up launches: further untimed launches of "
                         "that leg's kernel filling about this many ms before the timed ones")
    ap.add_argument("--compute", action="store_true",
                    help="only the differential-compute legs (every kernel of "
                         "COMPUTE_MODES); prints one JSON line")
    ap.add_argument("--sweep", action="store_true",
                    help="the size sweep instead: every N at batch 2^26/N, both types and "
                         "directions; prints one line per case and a JSON summary")
    return ap.parse_args()


SETTLE_MS = 60.0  # set from --settle-ms in main()


PER_LAUNCH = 25  # individually timed launches per leg (their median is reported)
LAST_MEDIAN_MS = None  # median of the last leg's per-launch timings, set by timed()


def timed(launch, steps: int, warmup: int, stream) -> float:
    """Mean ms per launch of `launch` over `steps` back-to-back launches on
    `stream`, timed with HIP events bracketed by device synchronisation.
    Afterwards PER_LAUNCH more launches are timed one by one (an event pair
    around each, on the same stream) and their median is left in
    LAST_MEDIAN_MS.
    Before them: `warmup` untimed launches, then as many more as fill about
    SETTLE_MS (counted from the warm-up's own mean).  A heavy kernel started
    after a pause first runs at transient clocks on MI355X: the fp32 conv1d
    of 16384 x 2048 reads 165 us for ~12 launches, 220-230 us for the next
    ~20, then climbs back over ~200 launches (~35 ms) to a steady 163-167 us.
    Settling times that steady state."""
    import torch

    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0.record(stream)
    for _ in range(warmup):
        launch()
    w1.record(stream)
    torch.cuda.synchronize()
    if SETTLE_MS > 0 and warmup > 0:
        per_ms = max(w0.elapsed_time(w1) / warmup, 1e-3)
        for _ in range(int(math.ceil(SETTLE_MS / per_ms))):
            launch()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        launch()
    end.record(stream)
    torch.cuda.synchronize()
    mean_ms = start.elapsed_time(end) / steps
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(PER_LAUNCH)]
    for a, b in pairs:
        a.record(stream)
        launch()
        b.record(stream)
    torch.cuda.synchronize()
    global LAST_MEDIAN_MS
    LAST_MEDIAN_MS = statistics.median(a.elapsed_time(b) for a, b in pairs)
    return mean_ms


def time_gpu(T: str, forward: bool, steps: int, warmup: int, n: int = N_FFT,
             batch: int = BATCH) -> dict:
    import torch

    import thunderfft_amd as thff

    dt = torch.float32 if T == "float" else torch.float16
    elem = 8 if T == "float" else 4
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    thff.fill_uniform(T, x, n * batch, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize(T, n)
    t0 = time.perf_counter()
    ms = timed(lambda: thff.ThunderFFT_global_async(T, n, forward, x, y, batch, stream),
               steps, warmup, stream)
    wall = time.perf_counter() - t0
    nbytes = 2 * n * batch * elem
    flops = 5.0 * n * math.log2(n) * batch
    del x, y
    return {
        "precision": T, "direction": "forward" if forward else "inverse", "n": n, "batch": batch,
        "us_per_call": ms * 1e3, "median_us_per_call": LAST_MEDIAN_MS * 1e3,
        "ns_per_transform": ms * 1e6 / batch,
        "gflops": flops / (ms * 1e-3) / 1e9,
        "gbps": nbytes / (ms * 1e-3) / 1e9,
        "pct_hbm_peak": 100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "bytes_per_call": nbytes, "wall_s": wall,
    }


def time_conv(kind: str, T: str, steps: int, warmup: int, size: int = 64,
              images: int = 8192) -> dict:
    """One of the fused convolution workloads: conv1d (16384 signals of 2048,
    per-signal complex filters with N(0, 1/sqrt(2048)) taps) or conv2d (`images`
    size x size images, one shared real filter with a N(0, 1/7) 7 x 7 corner
    block: 8192 of 64 x 64 is config 5; 2048 of 128 x 128 and 32 of 1024 x 1024
    move the same 2^25 values; 1 of 1024 x 1024 is the reference sample's
    shape, sample/conv2d/thunder.cu:556-565)."""
    import numpy as np
    import torch

    import thunderfft_amd as thff

    dt = torch.float32 if T == "float" else torch.float16
    elem = 8 if T == "float" else 4
    gen = torch.Generator(device="cuda").manual_seed(2048)
    if kind == "conv1d":
        n, batch = 2048, 16384
        count = n * batch
        h = (torch.randn(2 * count, device="cuda", generator=gen) / math.sqrt(n)).to(dt)
        nbytes = 3 * count * elem
        flops = 3 * 5.0 * n * math.log2(n) * batch + 6.0 * count
        init_n = n
    else:
        n, batch = size * size, images
        count = n * batch
        hh = np.zeros((size, size, 2), dtype=np.float32)
        hh[:7, :7, 0] = np.random.default_rng(7).normal(0.0, 1.0 / 7.0, (7, 7))
        h = torch.from_numpy(hh.reshape(-1)).to(device="cuda", dtype=dt)
        nbytes = 2 * count * elem
        flops = 2 * 2 * size * 5.0 * size * math.log2(size) * batch + 6.0 * count
        if size == 1024:  # the filter's spectrum is computed in every call
            flops += 2 * size * 5.0 * size * math.log2(size)
        init_n = size
    x = torch.empty(2 * count, dtype=dt, device="cuda")
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    thff.fill_uniform(T, x, count, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize(T, init_n)

    def launch():
        if kind == "conv1d":
            thff.ThunderFFT_conv1d_async(T, n, x, h, y, batch, True, stream)
        else:
            thff.ThunderFFT_conv2d_async(T, size, size, x, h, y, batch, stream)

    ms = timed(launch, steps, warmup, stream)
    thff.ThunderFFTFinalize(T)
    del x, y, h
    shape = "2048" if kind == "conv1d" else f"{size}x{size}"
    how = ("row pass, fused column FFT * H * IFFT, inverse row pass (filter spectrum in the call)"
           if kind == "conv2d" and size == 1024 else "fused FFT * H * IFFT")
    return {"workload": f"{kind} {batch} x {shape} {T}2, {how}",
            "precision": T, "us_per_call": ms * 1e3, "median_us_per_call": LAST_MEDIAN_MS * 1e3,
            "gflops": flops / (ms * 1e-3) / 1e9,
            "gbps": nbytes / (ms * 1e-3) / 1e9,
            "pct_hbm_peak": 100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "bytes_per_call": nbytes}


def time_conv_real(T: str, n: int, steps: int, warmup: int, with_filter: bool = False) -> dict:
    """The reference's real-input fused convolution
    (sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331) at 2^26 real samples:
    16384 signals [B=16384*4096/(n*64)][D=64][n], one real 9-tap filter per
    channel (the sample's default K).  By default the spectra are prepared
    once outside the timed region (its include_filter_fft=0 mode); with
    with_filter every timed step prepares them first (the sample's default,
    include_filter_fft=1, :481,582)."""
    import torch

    import thunderfft_amd as thff

    channels = 64
    count = 1 << 26
    batch = count // (n * channels)
    dt = torch.float32 if T == "float" else torch.float16
    elem = 4 if T == "float" else 2
    gen = torch.Generator(device="cuda").manual_seed(n)
    x = torch.rand(count, device="cuda", generator=gen).to(dt)
    y = torch.empty_like(x)
    h = torch.zeros(channels, n, device="cuda")
    h[:, :9] = torch.rand(channels, 9, device="cuda", generator=gen) / n
    spectrum = torch.empty(channels * n * 2, device="cuda")
    stream = torch.cuda.current_stream()
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_conv1d_real_filter(T, n, h, spectrum, channels, 1.0, stream)

    def launch():
        if with_filter:
            thff.ThunderFFT_conv1d_real_filter_async(T, n, h, spectrum, channels, 1.0, stream)
        thff.ThunderFFT_conv1d_real_async(T, n, x, spectrum, y, batch, channels, stream)

    ms = timed(launch, steps, warmup, stream)
    thff.ThunderFFTFinalize(T)
    nbytes = 2 * count * elem  # x and y; the spectra (2 MiB) stay in L2
    transforms = count // (2 * n)  # two real signals per complex transform
    flops = transforms * (2 * 5.0 * n * math.log2(n) + 6.0 * n)
    if with_filter:
        flops += channels * 5.0 * n * math.log2(n)
    del x, y, h, spectrum
    prep = ("spectra prepared in every step (include_filter_fft=1)" if with_filter
            else "spectra prepared once")
    return {"workload": (f"conv1d_real [{batch}][{channels}][{n}] {T}, 9-tap real filters, "
                         f"fused FFT * H * IFFT (two signals per complex transform), {prep}"),
            "precision": T, "us_per_call": ms * 1e3, "median_us_per_call": LAST_MEDIAN_MS * 1e3,
            "gflops": flops / (ms * 1e-3) / 1e9,
            "gbps": nbytes / (ms * 1e-3) / 1e9,
            "pct_hbm_peak": 100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "bytes_per_call": nbytes}


def time_conv_valid(T: str, ntaps: int, steps: int, warmup: int) -> dict:
    """The reference's tiled valid conv1d (sample/conv1d/main.cu:38-174) on one
    complex signal of 2^26 samples with `ntaps` complex taps (its default is
    9): float in 64-point FFT windows with 65 - ntaps valid outputs each (the
    reference's tiling), half in 256-point windows (257 - ntaps outputs) on
    MFMA.  GFLOP/s counts the windows' transforms at 5 N log2 N."""
    import torch

    import thunderfft_amd as thff

    length = 1 << 26
    out_len = length - ntaps + 1
    dt = torch.float32 if T == "float" else torch.float16
    elem = 8 if T == "float" else 4
    gen = torch.Generator(device="cuda").manual_seed(ntaps)
    x = torch.rand(2 * length, device="cuda", generator=gen).to(dt)
    y = torch.empty(2 * out_len, dtype=dt, device="cuda")
    taps = torch.rand(2 * ntaps, device="cuda", generator=gen)
    stream = torch.cuda.current_stream()
    thff.ThunderFFTInitialize(T, 64)

    def launch():
        thff.ThunderFFT_conv1d_valid_async(T, x, length, taps, ntaps, y, 1, stream)

    ms = timed(launch, steps, warmup, stream)
    thff.ThunderFFTFinalize(T)
    nbytes = (length + out_len) * elem
    win = 256 if T == "half" else 64  # half: 256-point windows on MFMA; float: 64-point on VALU
    windows = -(-out_len // (win + 1 - ntaps))
    flops = windows * (2 * 5.0 * win * math.log2(win) + 6.0 * win)
    del x, y, taps
    return {"workload": (f"conv1d_valid {length} x {ntaps} taps {T}2, {win}-point windows "
                         f"({win + 1 - ntaps} outputs each)"),
            "precision": T, "us_per_call": ms * 1e3, "median_us_per_call": LAST_MEDIAN_MS * 1e3,
            "gflops": flops / (ms * 1e-3) / 1e9,
            "gbps": nbytes / (ms * 1e-3) / 1e9,
            "pct_hbm_peak": 100.0 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "bytes_per_call": nbytes}


# Differential-compute kernels of libthff_bench_compute.so (thffx_compute_repeat's
# precision argument): the library's float and half transforms, and the float
# transform with both DFT16 stages on the matrix cores (exact fp32 MFMA, and a
# bf16x3 split), the measurement of the float path on MFMA.
COMPUTE_MODES = {"float": 0, "half": 1, "float_mfma_f32": 2, "float_mfma_bf16x3": 3}
COMPUTE_KERNELS = {
    "float": "fp32 VALU passes (the library's float kernel)",
    "half": "fp16 MFMA (v_mfma_f32_16x16x32_f16)",
    "float_mfma_f32": "fp32 data, both DFT16 stages on v_mfma_f32_16x16x4_f32",
    "float_mfma_bf16x3": "fp32 data, both DFT16 stages as bf16x3 on v_mfma_f32_16x16x32_bf16",
}


def placement_spread(T: str, steps: int, warmup: int,
                     offsets_mib=(0, 32, 64, 96, 128, 160, 192, 224)) -> dict:
    """The C2C of the main workload (N=1024 x 65536 forward) with its output
    placed at x + (buffer size) + d MiB inside one allocation, for each d in
    offsets_mib.  On MI355X the time of the fp16 MFMA kernels that walk many
    tiles per workgroup depends on where the output lies relative to the
    input (a pattern repeating every 128 MiB of d, and differing between
    processes for the same d: the physical pages differ); the fp32 kernel's
    does not, nor does the fp16 one-shot kernel's that this leg now runs at
    N = 1024.  The spread bounds what a single placement, such as the other
    legs', can read."""
    import torch

    import thunderfft_amd as thff

    n, batch = N_FFT, BATCH
    dt = torch.float32 if T == "float" else torch.float16
    esize = 4 if T == "float" else 2            # bytes per real component
    per_mib = (1 << 20) // esize                # components per MiB
    comps = 2 * n * batch                       # components per buffer
    big = torch.empty(2 * comps + max(offsets_mib) * per_mib, dtype=dt, device="cuda")
    x = big[:comps]
    stream = torch.cuda.current_stream()
    thff.fill_uniform(T, x, n * batch, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize(T, n)
    us = []
    for d in offsets_mib:
        y = big[comps + d * per_mib: 2 * comps + d * per_mib]
        ms = timed(lambda: thff.ThunderFFT_global_async(T, n, True, x, y, batch, stream),
                   steps, warmup, stream)
        us.append(round(ms * 1e3, 2))
    del big, x
    return {"workload": f"C2C {T}2 forward N={n} x {batch}, output at x + {comps * esize >> 20} "
                        f"MiB + d", "offsets_mib": list(offsets_mib), "us_per_call": us,
            "min_us": min(us), "median_us": statistics.median(us), "max_us": max(us)}


def compute_differential(T: str, repeats: int = 1000, trials: int = 3) -> dict:
    """Reference-style compute time of the N=1024, batch-65536 transform
    (sample/bench/paper_fft.cu:131-148): one launch loads every tile once,
    repeats the transform R times in registers/LDS and stores once;
    (t(2R) - t(R)) / R is one pass over the batch without HBM traffic.  The
    reference publishes 126.53 us for fp32 (TF32) on A100 (README.md:72-76)."""
    import ctypes

    import torch

    import thunderfft_amd as thff

    path = os.path.join(ROOT, "thunderfft_amd", "_build", "libthff_bench_compute.so")
    L = ctypes.CDLL(path)
    L.thffx_compute_repeat.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    n, batch = N_FFT, BATCH
    storage = "half" if T == "half" else "float"
    dt = torch.float32 if storage == "float" else torch.float16
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    thff.fill_uniform(storage, x, n * batch, 0x7F4A7C15 + n, 0, stream)
    x.mul_(1.0 / 32.0)  # keeps the repeated values finite a little longer
    thff.ThunderFFTInitialize(storage, n)
    prec = COMPUTE_MODES[T]

    def once(r):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        rc = L.thffx_compute_repeat(prec, x.data_ptr(), y.data_ptr(), batch, r, stream.cuda_stream)
        e.record(stream)
        torch.cuda.synchronize()
        if rc != 0:
            raise RuntimeError(f"thffx_compute_repeat failed ({rc})")
        return s.elapsed_time(e) * 1e3

    for _ in range(3):
        once(repeats)
    per = []
    for _ in range(trials):
        t_r, t_2r = once(repeats), once(2 * repeats)
        per.append((t_2r - t_r) / repeats)
    thff.ThunderFFTFinalize(storage)
    del x, y
    per.sort()
    return {"precision": T, "repeats": repeats, "trials": trials,
            "compute_us_per_pass": per[len(per) // 2], "kernel": COMPUTE_KERNELS[T],
            "reference_a100_us": 126.53 if storage == "float" else None}


def copy_bandwidth(steps: int, warmup: int) -> tuple[float, float]:
    """Read + write rates of a 512 MiB device-to-device copy, GB/s: the
    library's non-temporal 16-byte streaming copy (thff_copy_nt, the access
    pattern of the transforms, timed like a leg) and torch's copy_ (its
    copyBuffer kernel also calibrates the rocprofv3 traffic counters)."""
    import torch

    import thunderfft_amd as thff

    nbytes = 512 << 20
    a = torch.empty(nbytes // 8, dtype=torch.float64, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    stream = torch.cuda.current_stream()
    ms_nt = timed(lambda: thff.copy_nt(b, a, nbytes, stream), steps, warmup, stream)
    for _ in range(10):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    s.record()
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    del a, b
    return 2 * nbytes / (ms_nt * 1e-3) / 1e9, 2 * nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(target_s: float) -> dict:
    """The oracle's batched fp32 FFT (radix-4 passes, the reference's
    algorithm class, vectorised across 16 signals per AVX2 group and threaded
    over the groups) on this host's cores, on a bounded sample of the N=1024
    workload, writing into one reused output array."""
    import numpy as np

    import oracle

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = max(1, min(int(cores or 1), 64))
    n = N_FFT
    sample = 1024
    x = oracle.uniform(n, sample)
    out = np.empty_like(x)
    oracle.fft_f32_batched(x, True, cores, out)  # warm
    # grow the sample until one timed pass takes a meaningful share of target_s
    while True:
        x = oracle.uniform(n, sample)
        out = np.empty_like(x)
        oracle.fft_f32_batched(x, True, cores, out)  # touches the output's pages
        t0 = time.perf_counter()
        oracle.fft_f32_batched(x, True, cores, out)
        dt = time.perf_counter() - t0
        if dt >= target_s / 4 or sample >= BATCH:
            break
        sample = min(BATCH, sample * max(2, int(target_s / 4 / max(dt, 1e-3))))
    reps = max(1, min(1000, int(round(target_s / max(dt, 1e-3)))))  # about target_s of wall time
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.fft_f32_batched(x, True, cores, out)
    dt = (time.perf_counter() - t0) / reps
    flops = 5.0 * n * math.log2(n) * sample
    del x, out
    return {"value": flops / dt / 1e9, "unit": "GFLOP/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{sample} float forward transforms of N={n} (of the {BATCH}-signal "
                      f"workload), {reps} timed passes, {dt * 1e3:.1f} ms per pass, "
                      f"oracle fft_f32_batched (radix-4, 16 signals per AVX2 vector group) "
                      f"on {cores} threads",
            "us_per_transform": dt * 1e6 / sample}


def cpu_model() -> str:
    """The host CPU's model name with its family / model / stepping numbers
    (/proc/cpuinfo; a virtual machine may report only a generic name such as
    "AMD EPYC"), or the platform string."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, value = line.partition(":")
                fields[key.strip()] = value.strip()
    except OSError:
        pass
    name = fields.get("model name")
    if not name:
        import platform
        return platform.processor() or platform.machine()
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def sync_wrapper(T: str, calls: int = 25, warmup: int = 10) -> dict:
    """The synchronous ThunderFFT_global wrapper as a caller sees it: host wall
    time around each call (argument checks, the table lookup, the launch and
    hipStreamSynchronize, plus the ctypes binding), median of `calls` calls
    at N=1024, batch 65536."""
    import torch

    import thunderfft_amd as thff

    n, batch = N_FFT, BATCH
    dt = torch.float32 if T == "float" else torch.float16
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    thff.fill_uniform(T, x, n * batch, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize(T, n)
    for _ in range(warmup):
        thff.ThunderFFT_global(T, n, True, x, y, batch, stream)
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        thff.ThunderFFT_global(T, n, True, x, y, batch, stream)
        times.append(time.perf_counter() - t0)
    del x, y
    return {"precision": T, "calls": calls, "median_us_per_call": statistics.median(times) * 1e6,
            "min_us_per_call": min(times) * 1e6,
            "note": "host wall clock around the synchronous wrapper, through ctypes"}


def host_fp64_check(subset: int = 256) -> dict:
    """Part of the cpu_baseline leg (the oracle runs only there, as the
    checker).  The host fp64 check, timed on its own: the GPU's float forward transform
    of the bench input (N=1024, batch 65536) against the oracle's fp64 radix-2
    FFT of the same seeded input over the full batch (one thread), and that
    FFT against the fp64 direct DFT on a `subset`-signal subset."""
    import numpy as np
    import torch

    import oracle
    import thunderfft_amd as thff

    n, batch = N_FFT, BATCH
    x_d = torch.empty(2 * n * batch, dtype=torch.float32, device="cuda")
    y_d = torch.empty_like(x_d)
    stream = torch.cuda.current_stream()
    thff.fill_uniform("float", x_d, n * batch, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize("float", n)
    thff.ThunderFFT_global("float", n, True, x_d, y_d, batch, stream)
    got = y_d.cpu().numpy().view(np.complex64).reshape(batch, n)
    del x_d, y_d
    x = oracle.uniform(n, batch)  # the generator the device fill uses
    t0 = time.perf_counter()
    ref = oracle.fft(x, True)
    t_fft = time.perf_counter() - t0
    rows = np.unique(np.linspace(0, batch - 1, subset).astype(np.int64))
    t0 = time.perf_counter()
    direct = oracle.dft(x[rows], True)
    t_dft = time.perf_counter() - t0
    fft_vs_dft = float(np.linalg.norm(ref[rows] - direct) / np.linalg.norm(direct))
    err2 = ref2 = 0.0
    for lo in range(0, batch, 4096):
        r = ref[lo:lo + 4096]
        err2 += float(np.sum(np.abs(got[lo:lo + 4096].astype(np.complex128) - r) ** 2))
        ref2 += float(np.sum(np.abs(r) ** 2))
    del ref, direct, got, x
    return {"fp64_fft_s": t_fft, "fp64_fft_signals": batch, "direct_dft_s": t_dft,
            "direct_dft_signals": int(len(rows)), "threads": 1,
            "fp64_fft_vs_direct_dft_rel_l2": fft_vs_dft,
            "gpu_float_fwd_vs_fp64_rel_l2": math.sqrt(err2 / ref2), "gate": 5e-3}


def sig(v: float, digits: int = 6) -> float:
    """v to `digits` significant figures (no loss for small values)."""
    return float(f"{v:.{digits}g}")


def _profile_value(path: str, field: str, key: str):
    """The value of the machine-readable line `field key: value` of a profile
    summary, or None."""
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(rf"^{field} {re.escape(key)}: ([0-9.]+)\s*$", text, re.M)
    return m.group(1) if m else None


def kernel_sources_sha16() -> str:
    """First 16 hex digits of the sha256 of the kernel sources (every
    include/thunderfft/detail/*.hpp and thunderfft_amd/csrc/* file, sorted by
    path): the profile summaries record the value they were measured with."""
    import glob
    import hashlib

    files = sorted(glob.glob(os.path.join(ROOT, "include", "thunderfft", "detail", "*.hpp")) +
                   glob.glob(os.path.join(ROOT, "thunderfft_amd", "csrc", "*")))
    h = hashlib.sha256()
    for f in files:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def profile_sources(path: str):
    """The kernel_sources_sha16 a profile summary was measured with, or None."""
    try:
        with open(path) as f:
            m = re.search(r"^kernel_sources_sha16: ([0-9a-f]+)\s*$", f.read(), re.M)
    except OSError:
        return None
    return m.group(1) if m else None


def load_traffic(key: str):
    """HBM bytes per launch for `key` (e.g. float_fwd) from the PMC summary."""
    v = _profile_value(TRAFFIC_PROFILE, "hbm_bytes_per_launch", key)
    return int(v) if v is not None else None


def load_mfma_util(key: str):
    """rocprofiler's MfmaUtil (% of SIMD cycles with the matrix cores busy)
    for `key` (e.g. half_fwd) from the PMC summary."""
    v = _profile_value(MFMA_PROFILE, "mfma_util_pct", key)
    return float(v) if v is not None else None


def prewarm(ms: float) -> float:
    """Untimed back-to-back float N=1024 forward launches for about `ms` ms, so
    that the first timed leg starts from the clocks the later legs see (a fresh
    process's first ~15 ms of GPU work run up to 15% slower on MI355X).
    Returns the seconds spent."""
    import torch

    import thunderfft_amd as thff

    if ms <= 0:
        return 0.0
    n, batch = N_FFT, BATCH
    x = torch.empty(2 * n * batch, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream()
    thff.fill_uniform("float", x, n * batch, 0x7F4A7C15 + n, 0, stream)
    thff.ThunderFFTInitialize("float", n)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            thff.ThunderFFT_global_async("float", n, True, x, y, batch, stream)
        torch.cuda.synchronize()
    del x, y
    return time.perf_counter() - t0


def sweep(a) -> None:
    """The size sweep: N = 64 ... 4096 at batch 2^26 / N (1 GiB fp32, 512 MiB
    fp16 moved per launch), float and half, forward and inverse."""
    import thunderfft_amd as thff

    out = []
    for T in ("float", "half"):
        for n in (64, 128, 256, 512, 1024, 2048, 4096):
            for fwd in (True, False):
                r = time_gpu(T, fwd, a.steps, a.warmup, n, (1 << 26) // n)
                out.append({k: (sig(v) if isinstance(v, float) else v) for k, v in r.items()})
                print(f"[sweep] {T} N={n} batch={(1 << 26) // n} {'forward' if fwd else 'inverse'}: "
                      f"{r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
                      f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
                      file=sys.stderr, flush=True)
            thff.ThunderFFTFinalize(T)
    print(json.dumps({"sweep": out, "steps": a.steps, "warmup": a.warmup,
                      "settle_ms": a.settle_ms}), flush=True)


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only; the batched transform shards "
              "over GPUs by splitting the batch (each rank transforms its own signals, "
              "with no exchange). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import thunderfft_amd as thff

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    thff.lib()
    global SETTLE_MS
    SETTLE_MS = a.settle_ms
    prewarm_s = prewarm(a.prewarm_ms)
    if a.sweep:
        sweep(a)
        return
    if a.compute:
        out = {}
        for T in COMPUTE_MODES:
            r = compute_differential(T)
            out[T] = {k: (sig(v) if isinstance(v, float) else v) for k, v in r.items()}
            print(f"[compute] {T} ({r['kernel']}): {r['compute_us_per_pass']:.1f} us per pass",
                  file=sys.stderr, flush=True)
        print(json.dumps({"compute": out}), flush=True)
        return
    runs = {}
    for T in ("float", "half"):
        for fwd in (True, False):
            r = time_gpu(T, fwd, a.steps, a.warmup)
            runs[f"{T}_{'fwd' if fwd else 'inv'}"] = r
            print(f"[bench] {T} {'forward' if fwd else 'inverse'}: {r['us_per_call']:.1f} us, "
                  f"{r['gbps']:.0f} GB/s ({r['pct_hbm_peak']:.1f}% of HBM peak), "
                  f"{r['gflops']:.0f} GFLOP/s", file=sys.stderr, flush=True)
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")
    for kind, T in (("conv1d", "float"), ("conv1d", "half"), ("conv2d", "float"), ("conv2d", "half")):
        r = time_conv(kind, T, max(1, a.steps // 2), max(1, a.warmup // 2))
        runs[f"{kind}_{T}"] = r
        print(f"[bench] {r['workload']}: {r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
              f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
              file=sys.stderr, flush=True)
    for size, images, key in ((128, 2048, "conv2d128"), (1024, 32, "conv2d1024"),
                              (1024, 1, "conv2d1024_single")):
        for T in ("float", "half"):
            r = time_conv("conv2d", T, max(1, a.steps // 2), max(1, a.warmup // 2), size, images)
            runs[f"{key}_{T}"] = r
            print(f"[bench] {r['workload']}: {r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
                  f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
                  file=sys.stderr, flush=True)
    for T, n in (("half", 4096),):
        r = time_conv_real(T, n, max(1, a.steps // 2), max(1, a.warmup // 2), with_filter=True)
        runs[f"conv1d_real_{T}_n{n}_with_filter"] = r
        print(f"[bench] {r['workload']}: {r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
              f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
              file=sys.stderr, flush=True)
    for T, n in (("half", 4096), ("half", 1024), ("half", 256), ("float", 4096)):
        r = time_conv_real(T, n, max(1, a.steps // 2), max(1, a.warmup // 2))
        runs[f"conv1d_real_{T}_n{n}"] = r
        print(f"[bench] {r['workload']}: {r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
              f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
              file=sys.stderr, flush=True)
    for T, ntaps in (("half", 9), ("float", 9)):
        r = time_conv_valid(T, ntaps, max(1, a.steps // 2), max(1, a.warmup // 2))
        runs[f"conv1d_valid_{T}_f{ntaps}"] = r
        print(f"[bench] {r['workload']}: {r['us_per_call']:.1f} us, {r['gbps']:.0f} GB/s "
              f"({r['pct_hbm_peak']:.1f}% of HBM peak), {r['gflops']:.0f} GFLOP/s",
              file=sys.stderr, flush=True)
    for T in COMPUTE_MODES:
        r = compute_differential(T)
        runs[f"compute_{T}"] = r
        print(f"[bench] {T} N=1024 x 65536 differential compute (R={r['repeats']}, "
              f"{r['kernel']}): {r['compute_us_per_pass']:.1f} us per pass",
              file=sys.stderr, flush=True)
    for T in ("float", "half"):
        r = sync_wrapper(T)
        runs[f"sync_wrapper_{T}_fwd"] = r
        print(f"[bench] {T} N=1024 x 65536 synchronous ThunderFFT_global: "
              f"{r['median_us_per_call']:.1f} us per call (median of {r['calls']})",
              file=sys.stderr, flush=True)
    for T in ("float", "half"):
        r = placement_spread(T, max(5, a.steps // 4), max(1, a.warmup // 4))
        runs[f"placement_{T}_n1024"] = r
        print(f"[bench] {r['workload']}, d = {r['offsets_mib']} MiB: {r['us_per_call']} us",
              file=sys.stderr, flush=True)
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")
    copy_gbps, torch_copy_gbps = copy_bandwidth(a.steps, a.warmup)
    print(f"[bench] 512 MiB non-temporal copy: {copy_gbps:.0f} GB/s "
          f"({100.0 * copy_gbps / HBM_PEAK_GBPS:.1f}% of HBM peak); torch copy_ {torch_copy_gbps:.0f} GB/s",
          file=sys.stderr, flush=True)
    main_run = runs["float_fwd"]
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(a.cpu_seconds)
        if not a.no_fp64_check:
            fp64 = host_fp64_check()
            print(f"[bench] host fp64 check: fp64 FFT of {fp64['fp64_fft_signals']} signals "
                  f"{fp64['fp64_fft_s']:.1f} s, direct DFT of {fp64['direct_dft_signals']} "
                  f"{fp64['direct_dft_s']:.2f} s; GPU float forward vs fp64 rel L2 "
                  f"{fp64['gpu_float_fwd_vs_fp64_rel_l2']:.3e}", file=sys.stderr, flush=True)
            cpu["host_fp64_check"] = {k: (sig(v) if isinstance(v, float) else v)
                                      for k, v in fp64.items()}
    achieved = main_run["gbps"]
    out = {
        "metric": "C2C FFT µs, GFLOP/s and % HBM peak at N=1024 b=65536 (fp32/fp16)",
        "value": round(main_run["gflops"], 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "prewarm_s": round(prewarm_s, 3),
        "settle_ms": a.settle_ms,
        "ms_per_step": round(main_run["us_per_call"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded counter-based U[-1,1) complex inputs generated on device",
        "config": {"workload": "batched C2C FFT float2 forward, N=1024, batch=65536, "
                               "out-of-place", "n": N_FFT, "batch": BATCH,
                   "precision": "float2 storage, fp32 arithmetic"},
        "us_per_call": round(main_run["us_per_call"], 3),
        "pct_hbm_peak": round(main_run["pct_hbm_peak"], 2),
        "pct_copy_bw": round(100.0 * achieved / copy_gbps, 2),
        "copy_gbps": round(copy_gbps, 1),
        "copy_note": "copy_gbps: 512 MiB read + write by thff_copy_nt (one 16-byte non-temporal "
                     "vector per lane), the streaming ceiling; torch_copy_gbps: torch copy_ of the "
                     "same buffer",
        "torch_copy_gbps": round(torch_copy_gbps, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": load_traffic("float_fwd"),
                     "kernel": "thff::c2c_kernel<float2, 1024, true, false, false>",
                     "algorithmic_bytes": main_run["bytes_per_call"],
                     "traffic_profile": "profiles/pmc_c2c_n1024_b65536.md"},
        # traffic and mfma_util_pct are read from the rocprofv3 summaries in
        # profiles/; they describe the kernels being timed only when the
        # kernel sources are the ones the summaries were measured with.
        "profiles_match_kernel_sources": None,
        "cpu_baseline": cpu,
        "median_us_per_call": sig(main_run["median_us_per_call"]),
        "also": {k: {kk: (sig(vv) if isinstance(vv, float) else vv)
                     for kk, vv in v.items()} for k, v in runs.items()},
    }
    cur = kernel_sources_sha16()
    out["profiles_match_kernel_sources"] = {
        "match": profile_sources(TRAFFIC_PROFILE) == cur == profile_sources(MFMA_PROFILE),
        "kernel_sources_sha16": cur,
        "traffic_profile_sha16": profile_sources(TRAFFIC_PROFILE),
        "mfma_profile_sha16": profile_sources(MFMA_PROFILE),
    }
    for k in out["also"]:
        out["also"][k]["hbm_traffic_bytes"] = load_traffic(k)
        util = load_mfma_util(k)
        if util is not None:
            out["also"][k]["mfma_util_pct"] = util
    out["also"]["conv_note"] = ("conv1d bytes = x, h and y (3 * 2^25 complex); conv2d bytes = x "
                                "and y (2 * images * rows * cols complex: 2^25 per array except "
                                "the single 1024 x 1024 image; the filter is read per workgroup "
                                "from L2 at 64 and 128, and its spectrum is computed in every "
                                "1024 x 1024 call, whose intermediate passes are not counted); "
                                "conv1d_real bytes = x and y (2 * 2^26 "
                                "real samples); conv1d_valid bytes = x and y (2^26 + 2^26 - F + 1 "
                                "complex); GFLOP/s counts 5 N log2 N per transform")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
