"""GPU parity of the fused FFT convolution (thff_conv1d) against the fp64
direct circular convolution, through the C ABI.

The reference gates its fused convolution on the relative L2 of the output
against a direct circular convolution (sample/conv1d/
conv1d_fullfft_l4096_thunder.cu:499-554, gate 5e-3).  Here: every length x
{float, half} x {per-signal, shared filter}, batches that leave a partial last
tile; the benchmarked conv1d (16384 signals of 2048, per-signal filters) on a
subset of signals against the direct convolution, and over every signal
through an exact property: convolving with a shifted unit impulse rolls the
signal.
"""
import numpy as np
import pytest

import oracle
from thff_testlib import GATE, SIZES, from_device, to_device

pytestmark = pytest.mark.gpu

# fp32: three chained transforms; half: one output rounding to binary16.
TIGHT = {"float": 5e-6, "half": 1e-3}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch

    import thunderfft_amd as thff

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    thff.lib()
    yield
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")


def _filters(n, count, seed):
    """Complex taps with re, im ~ N(0, 1/sqrt(n)) (the benchmarked conv1d's filters)."""
    rng = np.random.default_rng(seed)
    h = rng.normal(0.0, 1.0 / np.sqrt(n), size=(count, n, 2)).astype(np.float32)
    return h.view(np.complex64).reshape(count, n)


def _run(T, n, x, h, per_signal):
    import thunderfft_amd as thff

    batch = x.shape[0]
    xr, hr = oracle.represent(x, T), oracle.represent(h, T)
    d_x, d_h = to_device(xr, T), to_device(hr, T)
    d_y = to_device(np.full((batch, n), np.nan, dtype=np.complex64), T)
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_conv1d(T, n, d_x, d_h, d_y, batch, per_signal)
    y = from_device(d_y, T).reshape(batch, n)
    ref = oracle.circconv1d(xr, hr, per_signal)
    return oracle.metrics(y, ref)


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_conv1d_matches_direct_convolution(T, n):
    import thunderfft_amd as thff

    fpb = thff.transforms_per_block(n)
    for per_signal in (True, False):
        for batch in sorted({1, fpb + 1, 2 * fpb + max(1, fpb // 2)} - {0}):
            if n >= 2048 and batch > 6:
                continue
            x = oracle.uniform(n, batch, seed=1000 + n + batch)
            h = _filters(n, batch if per_signal else 1, seed=n * 7 + batch)
            m = _run(T, n, x, h, per_signal)
            label = (f"{T} N={n} batch={batch} {'per-signal' if per_signal else 'shared'}: "
                     f"rel_l2={m['rel_l2']:.3e}")
            print(label, flush=True)
            assert m["nonfinite"] == 0, label
            assert m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
def test_config4_conv1d_2048(T):
    """16384 signals of 2048, per-signal filters (the benchmarked conv1d)."""
    import torch

    import thunderfft_amd as thff

    n, batch = 2048, 16384
    dt = torch.float32 if T == "float" else torch.float16
    seed = oracle.BENCH_SEED_BASE + n
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, n * batch, seed)
    y = torch.empty_like(x)
    thff.ThunderFFTInitialize(T, n)

    # (1) a subset of signals with normal taps against the direct convolution
    rows = np.unique(np.concatenate([np.linspace(0, batch - 1, 48).astype(np.int64),
                                     np.arange(batch - 3, batch)]))
    h_host = _filters(n, batch, seed=4).reshape(batch, n)
    h_host = oracle.represent(h_host, T)
    h = to_device(h_host, T)
    thff.ThunderFFT_conv1d(T, n, x, h, y, batch, True)
    rows_t = torch.from_numpy(rows).cuda()
    sub = from_device(y.view(batch, 2 * n).index_select(0, rows_t).contiguous(), T)
    sub = sub.reshape(len(rows), n)
    xin = np.concatenate([oracle.uniform(n, 1, seed, first_element=int(r) * n) for r in rows])
    ref = oracle.circconv1d(oracle.represent(xin, T), h_host[rows], True)
    m = oracle.metrics(sub, ref)
    print(f"{T} conv1d N={n} batch={batch} subset rel_l2={m['rel_l2']:.3e}", flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]

    # (2) every signal: a unit impulse at s_b = (7b) mod n rolls signal b by s_b
    shifts = (7 * np.arange(batch)) % n
    imp = torch.zeros(batch, n, 2, dtype=dt, device="cuda")
    imp[torch.arange(batch, device="cuda"), torch.from_numpy(shifts).cuda(), 0] = 1
    thff.ThunderFFT_conv1d(T, n, x, imp, y, batch, True)
    xs = x.view(batch, n, 2).float()
    idx = (torch.arange(n, device="cuda")[None, :] - torch.from_numpy(shifts).cuda()[:, None]) % n
    want = torch.gather(xs, 1, idx[:, :, None].expand(batch, n, 2))
    err = float(torch.linalg.vector_norm(y.view(batch, n, 2).float() - want) /
                torch.linalg.vector_norm(want))
    print(f"  impulse roll over all signals rel_l2={err:.3e}", flush=True)
    assert np.isfinite(err) and err <= TIGHT[T]
    del x, y, h, imp
    torch.cuda.empty_cache()


# Batches with several tiles per workgroup of the device-sized grids (up to
# 3 x 256 workgroups of 16, 4 or 1 signals at N = 256, 1024, 4096) and a
# partial last round: exercises the loads issued a tile ahead.
MANY = {256: 3 * 768 * 16 + 7, 1024: 3 * 768 * 4 + 3, 4096: 2112}


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("per_signal", [True, False])
@pytest.mark.parametrize("n", sorted(MANY))
def test_conv1d_many_signals_per_workgroup(T, per_signal, n):
    """More signals than workgroups, so every workgroup convolves several in
    turn (a shared filter is transformed once per workgroup or wave).  A
    subset against the direct convolution, then every signal through the
    impulse roll (per-signal shifts, or one shared shift)."""
    import torch

    import thunderfft_amd as thff

    batch = MANY[n]
    dt = torch.float32 if T == "float" else torch.float16
    seed = oracle.BENCH_SEED_BASE + n + 11
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, n * batch, seed)
    y = torch.full_like(x, float("nan"))
    thff.ThunderFFTInitialize(T, n)
    nh = batch if per_signal else 1
    mode = "per-signal" if per_signal else "shared"

    rows = np.unique(np.concatenate([np.linspace(0, batch - 1, 12).astype(np.int64),
                                     np.arange(batch - 2, batch)]))
    h_host = oracle.represent(_filters(n, nh, seed=41).reshape(nh, n), T)
    thff.ThunderFFT_conv1d(T, n, x, to_device(h_host, T), y, batch, per_signal)
    rows_t = torch.from_numpy(rows).cuda()
    sub = from_device(y.view(batch, 2 * n).index_select(0, rows_t).contiguous(), T)
    sub = sub.reshape(len(rows), n)
    xin = np.concatenate([oracle.uniform(n, 1, seed, first_element=int(r) * n) for r in rows])
    ref = oracle.circconv1d(oracle.represent(xin, T),
                            h_host[rows] if per_signal else h_host, per_signal)
    m = oracle.metrics(sub, ref)
    print(f"{T} conv1d N={n} batch={batch} {mode} subset rel_l2={m['rel_l2']:.3e}", flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]

    shifts = (13 * np.arange(nh) + 5) % n
    imp = torch.zeros(nh, n, 2, dtype=dt, device="cuda")
    imp[torch.arange(nh, device="cuda"), torch.from_numpy(shifts).cuda(), 0] = 1
    y.fill_(float("nan"))
    thff.ThunderFFT_conv1d(T, n, x, imp, y, batch, per_signal)
    xs = x.view(batch, n, 2).float()
    s = torch.from_numpy(np.broadcast_to(shifts, (batch,)).copy()).cuda()
    idx = (torch.arange(n, device="cuda")[None, :] - s[:, None]) % n
    want = torch.gather(xs, 1, idx[:, :, None].expand(batch, n, 2))
    got = y.view(batch, n, 2).float()
    assert bool(torch.isfinite(got).all())
    err = float(torch.linalg.vector_norm(got - want) / torch.linalg.vector_norm(want))
    worst = float((got - want).abs().max())
    print(f"  impulse roll over all signals rel_l2={err:.3e} max={worst:.3e}", flush=True)
    assert err <= TIGHT[T] and worst <= (5e-3 if T == "half" else 1e-5)
    del x, y, imp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("per_signal", [True, False])
def test_conv1d_grid_stride_walks(T, n, per_signal):
    """2^25 values plus a partial tile: 8192 tiles of 4096 values, more than
    twice any device-sized grid (at most 16 workgroups per CU), so every
    workgroup convolves several tiles in turn, prefetching the next one where
    the launch shape does.  Every signal through the impulse roll."""
    import torch

    import thunderfft_amd as thff

    fpb = thff.transforms_per_block(n)
    batch = (1 << 25) // n + fpb // 2 + 1
    dt = torch.float32 if T == "float" else torch.float16
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, n * batch, oracle.BENCH_SEED_BASE + 3 * n + per_signal)
    y = torch.full_like(x, float("nan"))
    thff.ThunderFFTInitialize(T, n)
    nh = batch if per_signal else 1
    shifts = (7 * np.arange(nh) + 3) % n
    imp = torch.zeros(nh, n, 2, dtype=dt, device="cuda")
    imp[torch.arange(nh, device="cuda"), torch.from_numpy(shifts).cuda(), 0] = 1
    print(f"{T} conv1d N={n} batch={batch} {'per-signal' if per_signal else 'shared'}", flush=True)
    thff.ThunderFFT_conv1d(T, n, x, imp, y, batch, per_signal)
    xs = x.view(batch, n, 2).float()
    s = torch.from_numpy(np.broadcast_to(shifts, (batch,)).copy()).cuda()
    idx = (torch.arange(n, device="cuda")[None, :] - s[:, None]) % n
    want = torch.gather(xs, 1, idx[:, :, None].expand(batch, n, 2))
    got = y.view(batch, n, 2).float()
    assert bool(torch.isfinite(got).all())
    err = float(torch.linalg.vector_norm(got - want) / torch.linalg.vector_norm(want))
    worst = float((got - want).abs().max())
    print(f"  impulse roll rel_l2={err:.3e} max={worst:.3e}", flush=True)
    assert err <= TIGHT[T] and worst <= (5e-3 if T == "half" else 1e-5)
    del x, y, imp, xs, want, got
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", ["half", "float"])
def test_conv1d_beyond_2e31_values(T):
    """The benchmarked conv1d's length (2048) over 2^31 + 3 * 2048 complex
    values per array (x, h and y: 8.6 GB each in fp16, 17 GB in fp32): signal
    b's filter is a unit impulse at (13 b + 5) mod N, so output row b is input
    row b rolled by that shift; checked on the first rows, a spread and every
    row past value 2^31."""
    import torch

    import thunderfft_amd as thff

    n = 2048
    batch = (1 << 31) // n + 3
    dt = torch.float32 if T == "float" else torch.float16
    x = torch.empty(2 * n * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, n * batch, oracle.BENCH_SEED_BASE + 77)
    shifts = (13 * torch.arange(batch, device="cuda") + 5) % n
    h = torch.zeros(batch, n, 2, dtype=dt, device="cuda")
    h[torch.arange(batch, device="cuda"), shifts, 0] = 1
    y = torch.full_like(x, float("nan"))
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_conv1d(T, n, x, h, y, batch, True)
    del h
    rows = torch.from_numpy(np.unique(np.concatenate([
        np.arange(3), np.linspace(0, batch - 1, 16).astype(np.int64),
        np.arange((1 << 31) // n - 2, batch)]))).cuda()
    xs = x.view(batch, n, 2).index_select(0, rows).float()
    ys = y.view(batch, n, 2).index_select(0, rows).float()
    idx = (torch.arange(n, device="cuda")[None, :] - shifts[rows][:, None]) % n
    want = torch.gather(xs, 1, idx[:, :, None].expand(len(rows), n, 2))
    assert bool(torch.isfinite(ys).all())
    err = float(torch.linalg.vector_norm(ys - want) / torch.linalg.vector_norm(want))
    print(f"{T} conv1d N={n} batch={batch}: sampled rows rel_l2={err:.3e}", flush=True)
    assert err <= TIGHT[T]
    del x, y
    torch.cuda.empty_cache()


def _filter2d(seed, full=False):
    """The benchmarked conv2d filter: real 64 x 64, nonzero 7 x 7 corner block with
    i.i.d. N(0, 1/7) taps (full=True: every tap nonzero, complex)."""
    rng = np.random.default_rng(seed)
    h = np.zeros((64, 64), dtype=np.complex64)
    if full:
        h[:] = (rng.normal(0, 1 / 64, (64, 64)) + 1j * rng.normal(0, 1 / 64, (64, 64)))
    else:
        h[:7, :7] = rng.normal(0.0, 1.0 / 7.0, (7, 7))
    return h


@pytest.mark.parametrize("T", ["float", "half"])
def test_conv2d_matches_direct_convolution(T):
    import thunderfft_amd as thff

    thff.ThunderFFTInitialize(T, 64)
    for batch, full in ((1, False), (3, True), (2, False)):
        x = oracle.uniform(4096, batch, seed=77 + batch).reshape(batch, 64, 64)
        h = _filter2d(batch, full)
        xr, hr = oracle.represent(x, T), oracle.represent(h, T)
        d_x, d_h = to_device(xr, T), to_device(hr, T)
        d_y = to_device(np.full((batch, 64, 64), np.nan, dtype=np.complex64), T)
        thff.ThunderFFT_conv2d(T, 64, 64, d_x, d_h, d_y, batch)
        y = from_device(d_y, T).reshape(batch, 64, 64)
        m = oracle.metrics(y, oracle.circconv2d(xr, hr))
        label = f"{T} conv2d 64x64 batch={batch} full_filter={full}: rel_l2={m['rel_l2']:.3e}"
        print(label, flush=True)
        assert m["nonfinite"] == 0, label
        assert m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
def test_config5_conv2d_64x64(T):
    """8192 images of 64 x 64, shared 7 x 7-corner filter (the benchmarked conv2d):
    every workgroup walks several images (the next one's loads in flight)."""
    import torch

    import thunderfft_amd as thff

    batch = 8192
    seed = oracle.BENCH_SEED_BASE + 4096
    x = torch.empty(2 * 4096 * batch, dtype=torch.float32 if T == "float" else torch.float16,
                    device="cuda")
    thff.fill_uniform(T, x, 4096 * batch, seed)
    y = torch.empty_like(x)
    thff.ThunderFFTInitialize(T, 64)

    # (1) the benchmark filter (7 x 7 corner block) on a subset of images against the direct convolution
    h = _filter2d(5)
    thff.ThunderFFT_conv2d(T, 64, 64, x, to_device(h, T), y, batch)
    rows = np.array([0, 1, 2047, 4096, 6000, batch - 2, batch - 1])
    sub = from_device(y.view(batch, 2 * 4096)[torch.from_numpy(rows).cuda()].contiguous(), T)
    xin = np.concatenate([oracle.uniform(4096, 1, seed, first_element=int(r) * 4096)
                          for r in rows]).reshape(len(rows), 64, 64)
    xin = oracle.represent(xin, T)
    m = oracle.metrics(sub.reshape(len(rows), 64, 64), oracle.circconv2d(xin, oracle.represent(h, T)))
    print(f"{T} conv2d 64x64 batch={batch} subset rel_l2={m['rel_l2']:.3e}", flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]

    # (2) every image: a unit impulse at (dr, dc) rolls every image by (dr, dc)
    dr, dc = 5, 61
    imp = np.zeros((64, 64), dtype=np.complex64)
    imp[dr, dc] = 1
    thff.ThunderFFT_conv2d(T, 64, 64, x, to_device(imp, T), y, batch)
    want = torch.roll(x.view(batch, 64, 64, 2).float(), shifts=(dr, dc), dims=(1, 2))
    err = float(torch.linalg.vector_norm(y.view(batch, 64, 64, 2).float() - want) /
                torch.linalg.vector_norm(want))
    print(f"  impulse roll over all images rel_l2={err:.3e}", flush=True)
    assert np.isfinite(err) and err <= TIGHT[T]
    del x, y
    torch.cuda.empty_cache()


def _corner_filter(size, seed, k=7, full=False):
    """size x size filter: a k x k corner block of i.i.d. N(0, 1/k) real taps
    (the benchmarked filter's shape), or every tap complex N(0, 1/size^2)."""
    rng = np.random.default_rng(seed)
    h = np.zeros((size, size), dtype=np.complex64)
    if full:
        s = 1.0 / size
        h[:] = rng.normal(0, s, (size, size)) + 1j * rng.normal(0, s, (size, size))
    else:
        h[:k, :k] = rng.normal(0.0, 1.0 / k, (k, k))
    return h


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("size", [128, 1024])
def test_conv2d_large_images_match_direct_convolution(T, size):
    """128 x 128 (one fused kernel per image) and 1024 x 1024 (the reference
    sample's shape, sample/conv2d/thunder.cu:556-565: row pass, fused column
    pass, inverse row pass) against the fp64 direct circular convolution:
    the 7 x 7 corner filter on 1 and 3 images, a filter with one tap at
    (dr, dc) (every image rolls by it) and, at 128, a dense complex filter."""
    import thunderfft_amd as thff

    thff.ThunderFFTInitialize(T, size)
    cases = [(1, _corner_filter(size, 3)), (3, _corner_filter(size, 4))]
    imp = np.zeros((size, size), dtype=np.complex64)
    imp[size // 2 + 3, size - 5] = 1
    cases.append((2, imp))
    if size == 128:
        cases.append((2, _corner_filter(size, 5, full=True)))
    for batch, h in cases:
        x = oracle.uniform(size * size, batch, seed=91 + batch + size).reshape(batch, size, size)
        xr, hr = oracle.represent(x, T), oracle.represent(h, T)
        d_x, d_h = to_device(xr, T), to_device(hr, T)
        d_y = to_device(np.full((batch, size, size), np.nan, dtype=np.complex64), T)
        thff.ThunderFFT_conv2d(T, size, size, d_x, d_h, d_y, batch)
        y = from_device(d_y, T).reshape(batch, size, size)
        m = oracle.metrics(y, oracle.circconv2d(xr, hr))
        nnz = int(np.count_nonzero(h))
        label = f"{T} conv2d {size}x{size} batch={batch} taps={nnz}: rel_l2={m['rel_l2']:.3e}"
        print(label, flush=True)
        assert m["nonfinite"] == 0, label
        assert m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("size,batch", [(128, 2048 + 3), (1024, 32), (1024, 9)])
def test_conv2d_large_image_batches(T, size, batch):
    """Benchmark-sized batches (2^25 values, plus a few images so the walk is
    uneven at 128), and 9 images at 1024 (the half2 column pass on MFMA with
    an uneven grid-stride walk): a subset of images against the direct
    convolution with the 7 x 7 corner filter, then a one-tap filter rolls
    every image."""
    import torch

    import thunderfft_amd as thff

    img = size * size
    seed = oracle.BENCH_SEED_BASE + img
    dt = torch.float32 if T == "float" else torch.float16
    x = torch.empty(2 * img * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, img * batch, seed)
    y = torch.empty_like(x)
    thff.ThunderFFTInitialize(T, size)
    h = _corner_filter(size, 6)
    thff.ThunderFFT_conv2d(T, size, size, x, to_device(h, T), y, batch)
    rows = np.unique(np.array([0, 1, batch // 2, batch - 2, batch - 1]))
    sub = from_device(y.view(batch, 2 * img)[torch.from_numpy(rows).cuda()].contiguous(), T)
    xin = np.concatenate([oracle.uniform(img, 1, seed, first_element=int(r) * img)
                          for r in rows]).reshape(len(rows), size, size)
    xin = oracle.represent(xin, T)
    m = oracle.metrics(sub.reshape(len(rows), size, size),
                       oracle.circconv2d(xin, oracle.represent(h, T)))
    print(f"{T} conv2d {size}x{size} batch={batch} subset rel_l2={m['rel_l2']:.3e}", flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]
    dr, dc = 7, size - 3
    imp = np.zeros((size, size), dtype=np.complex64)
    imp[dr, dc] = 1
    thff.ThunderFFT_conv2d(T, size, size, x, to_device(imp, T), y, batch)
    want = torch.roll(x.view(batch, size, size, 2).float(), shifts=(dr, dc), dims=(1, 2))
    err = float(torch.linalg.vector_norm(y.view(batch, size, size, 2).float() - want) /
                torch.linalg.vector_norm(want))
    print(f"  impulse roll over all images rel_l2={err:.3e}", flush=True)
    assert np.isfinite(err) and err <= TIGHT[T]
    del x, y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", ["float", "half"])
def test_conv2d_beyond_2e31_values(T):
    """2^19 + 3 images of 64 x 64 (2^31 + 12288 complex values: 17 GB fp32,
    8.6 GB fp16 per array) with a unit-impulse filter at (dr, dc): every image
    rolls by (dr, dc); checked on the first images, a spread and every image
    past value 2^31."""
    import torch

    import thunderfft_amd as thff

    batch = (1 << 19) + 3
    dt = torch.float32 if T == "float" else torch.float16
    x = torch.empty(2 * 4096 * batch, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, 4096 * batch, oracle.BENCH_SEED_BASE + 4099)
    y = torch.full_like(x, float("nan"))
    thff.ThunderFFTInitialize(T, 64)
    dr, dc = 17, 3
    imp = np.zeros((64, 64), dtype=np.complex64)
    imp[dr, dc] = 1
    thff.ThunderFFT_conv2d(T, 64, 64, x, to_device(imp, T), y, batch)
    rows = torch.from_numpy(np.unique(np.concatenate([
        np.arange(3), np.linspace(0, batch - 1, 16).astype(np.int64),
        np.arange((1 << 31) // 4096 - 2, batch)]))).cuda()
    xs = x.view(batch, 64, 64, 2).index_select(0, rows).float()
    ys = y.view(batch, 64, 64, 2).index_select(0, rows).float()
    want = torch.roll(xs, shifts=(dr, dc), dims=(1, 2))
    assert bool(torch.isfinite(ys).all())
    err = float(torch.linalg.vector_norm(ys - want) / torch.linalg.vector_norm(want))
    print(f"{T} conv2d batch={batch}: sampled images rel_l2={err:.3e}", flush=True)
    assert err <= TIGHT[T]
    del x, y
    torch.cuda.empty_cache()
