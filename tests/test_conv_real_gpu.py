"""GPU parity of the real-input fused convolution (thff_conv1d_real) and its
filter-spectrum preparation (thff_conv1d_real_filter), through the C ABI.

The reference's thunder_convN_block_kernel_realin_realout
(sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331) convolves real half
signals [B][D][N] with one real filter per channel and writes the
unnormalized result; its driver (:354-570) draws the inputs with
srand(42)/rand(), prepares the spectra once, and gates rel L2 of output/N
against the direct circular convolution at 5e-3 (:499-554).  Here:

* the reference's own cases (N = 256, 1024, 4096; its default K = 9, B = D = 1
  and wider K, B, D) on its own seeded inputs, half and float;
* every length x {float, half} with channel counts and odd batches that leave
  partial tiles and an unpaired last signal, against the fp64 direct
  convolution, with output sentinels;
* the spectra against numpy's FFT;
* at full size (65535 signals of 1024; 2112 of 4096) the exact property that a
  unit impulse at tap s rolls each signal by s.
"""
import numpy as np
import pytest

import oracle
from thff_testlib import GATE, SIZES

pytestmark = pytest.mark.gpu

# float: two fp32 transforms and a product; half: plus one output rounding.
TIGHT = {"float": 5e-6, "half": 1e-3}
GUARD = 16
GUARD_VALUE = -37.0


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


def represent(x, T):
    """The real values storage type T holds (float32, or binary16 round trip)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if T == "float":
        return x.copy()
    return oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(x.reshape(-1))).reshape(x.shape)


def to_device(x, T):
    import torch

    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if T == "float":
        return torch.from_numpy(x.copy()).cuda()
    bits = oracle.f32_to_f16_bits(x)
    return torch.from_numpy(bits.view(np.int16).copy()).cuda().view(torch.float16)


def from_device(t, T):
    import torch

    if T == "float":
        return t.detach().cpu().numpy().astype(np.float32)
    bits = t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    return oracle.f16_bits_to_f32(bits)


def spectra(T, n, h, scale):
    """Device spectra of the real fp32 filters h (channels, n)."""
    import torch

    import thunderfft_amd as thff

    channels = h.shape[0]
    d_h = torch.from_numpy(np.ascontiguousarray(h, dtype=np.float32).reshape(-1)).cuda()
    d_s = torch.full((channels * n * 2,), float("nan"), dtype=torch.float32, device="cuda")
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_conv1d_real_filter(T, n, d_h, d_s, channels, scale)
    return d_s


def convolve(T, n, x, d_spec, channels, sync=True):
    """Run the fused real convolution on x (batch, channels, n); returns the
    output (batch, channels, n) and the number of changed output sentinels."""
    import thunderfft_amd as thff

    batch = x.shape[0]
    count = batch * channels * n
    d_x = to_device(x, T)
    host = np.full(count + GUARD, np.nan, dtype=np.float32)
    host[count:] = GUARD_VALUE
    d_y = to_device(host, T)
    if sync:
        thff.ThunderFFT_conv1d_real(T, n, d_x, d_spec, d_y, batch, channels)
    else:
        import torch

        thff.ThunderFFT_conv1d_real_async(T, n, d_x, d_spec, d_y, batch, channels)
        torch.cuda.synchronize()
    y = from_device(d_y, T)
    guards = int(np.sum(y[count:] != GUARD_VALUE))
    return y[:count].reshape(batch, channels, n), guards


def rel_l2(y, ref):
    m = oracle.metrics(np.asarray(y, np.float32).astype(np.complex64),
                       np.asarray(ref, np.float64).astype(np.complex128))
    return m["rel_l2"], m["nonfinite"]


# The reference's cases: its default (K = 9, B = D = 1, :575-585) and wider
# K / B / D, including K = N and an odd B*D.
REFERENCE_CASES = [(9, 1, 1), (1, 2, 3), (53, 3, 5), (None, 4, 16)]


@pytest.mark.parametrize("T", ["half", "float"])
@pytest.mark.parametrize("n", [256, 1024, 4096])
def test_reference_cases_on_reference_inputs(T, n):
    for taps, batch, channels in REFERENCE_CASES:
        taps = n if taps is None else taps
        x, h = oracle.conv_real_inputs(n, taps, batch, channels, seed=42)
        xr = represent(x, T)
        d_spec = spectra(T, n, h, 1.0)  # the reference's unscaled spectra
        y, guards = convolve(T, n, xr, d_spec, channels)
        ref = oracle.circconv1d_channels(xr, h, taps)
        err, bad = rel_l2(y / n, ref)  # the reference's gate: output / N
        label = f"{T} N={n} K={taps} B={batch} D={channels}: rel_l2(out/N)={err:.3e}"
        print(label, flush=True)
        assert bad == 0 and guards == 0, label
        assert err <= GATE and err <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_all_lengths_partial_tiles(T, n):
    import thunderfft_amd as thff

    fpb = thff.transforms_per_block(n)
    rng = np.random.default_rng(n)
    for channels, batch in ((1, 1), (3, 5), (fpb + 1, 2)):
        if n >= 2048 and channels * batch > 12:
            continue
        x = rng.uniform(-1, 1, size=(batch, channels, n)).astype(np.float32)
        h = rng.normal(0, 1 / np.sqrt(n), size=(channels, n)).astype(np.float32)
        xr = represent(x, T)
        d_spec = spectra(T, n, h, 1.0 / n)  # normalised: y = x (*) h
        y, guards = convolve(T, n, xr, d_spec, channels)
        ref = oracle.circconv1d_channels(xr, h)
        err, bad = rel_l2(y, ref)
        label = f"{T} N={n} D={channels} B={batch}: rel_l2={err:.3e}"
        print(label, flush=True)
        assert bad == 0 and guards == 0, label
        assert err <= GATE and err <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_filter_spectra_match_numpy(T, n):
    rng = np.random.default_rng(3 * n)
    channels = 5
    h = rng.normal(size=(channels, n)).astype(np.float32)
    scale = 1.0 / n if n % 128 else 1.0
    d_s = spectra(T, n, h, scale)
    got = d_s.cpu().numpy().view(np.complex64).reshape(channels, n)
    ref = np.fft.fft(h.astype(np.float64), axis=-1) * scale
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    print(f"{T} N={n} spectra: rel_l2={err:.3e}", flush=True)
    assert np.all(np.isfinite(got)) and err <= 2e-6


@pytest.mark.parametrize("T", ["float", "half"])
def test_async_equals_sync_and_scale(T):
    n, batch, channels = 1024, 7, 6
    rng = np.random.default_rng(17)
    x = represent(rng.uniform(0, 1, size=(batch, channels, n)), T)
    h = rng.uniform(0, 1.0 / n, size=(channels, n)).astype(np.float32)
    raw, _ = convolve(T, n, x, spectra(T, n, h, 1.0), channels)
    raw_async, _ = convolve(T, n, x, spectra(T, n, h, 1.0), channels, sync=False)
    assert np.array_equal(raw, raw_async)
    normed, _ = convolve(T, n, x, spectra(T, n, h, 1.0 / n), channels)
    # scale = 1 writes N * (x (*) h), scale = 1/N writes x (*) h
    err, _ = rel_l2(raw / n, normed)
    assert err <= TIGHT[T], err


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n,batch,channels", [(1024, 255, 257), (4096, 33, 64), (4096, 401, 3),
                                               (1024, 2801, 5), (512, 2601, 5), (256, 2401, 7),
                                               (64, 2403, 61), (128, 2403, 31), (2048, 803, 11)])
def test_full_size_impulse_rolls(T, n, batch, channels):
    """Filter d is a unit impulse at tap s_d = (17 d + 1) mod N, so every output
    row is its input row rolled by s_d (checked over all signals).  All but the
    first two cases have more tiles than a 256-CU device's grid (512 to 1024
    workgroups), so workgroups walk several tiles (prefetching the next one
    where the launch shape does), with channel counts that do not divide the
    grid's stride in transforms: a workgroup's tiles change channel and pair,
    and a kept spectrum must be reloaded."""
    import torch

    import thunderfft_amd as thff

    shifts = (17 * np.arange(channels) + 1) % n
    h = np.zeros((channels, n), dtype=np.float32)
    h[np.arange(channels), shifts] = 1.0
    count = batch * channels * n
    thff.ThunderFFTInitialize(T, n)
    d_x = torch.empty(count, dtype=torch.float32 if T == "float" else torch.float16, device="cuda")
    d_x.uniform_(-1, 1)
    x = from_device(d_x, T).reshape(batch, channels, n)
    d_spec = spectra(T, n, h, 1.0 / n)
    d_y = torch.full_like(d_x, float("nan"))
    thff.ThunderFFT_conv1d_real(T, n, d_x, d_spec, d_y, batch, channels)
    y = from_device(d_y, T).reshape(batch, channels, n)
    idx = (np.arange(n)[None, :] - shifts[:, None]) % n  # y[k] = x[(k - s) mod N]
    expect = np.take_along_axis(x, np.broadcast_to(idx, x.shape), axis=-1)
    err = np.abs(y - expect)
    rel = float(np.linalg.norm((y - expect).ravel()) / np.linalg.norm(expect.ravel()))
    label = f"{T} N={n} B={batch} D={channels}: max_err={err.max():.3e} rel_l2={rel:.3e}"
    print(label, flush=True)
    assert np.all(np.isfinite(y)), label
    if T == "float":
        # fp32 between the transforms: every element within fp32 rounding
        assert np.all(err <= 1e-5 * np.abs(expect) + 2e-6), label
    else:
        # fp16 N >= 256 run on MFMA with f16 data between the stages:
        # errors are spread evenly over a signal, so bound them against the
        # signal scale (|x| <= 1 here); a wrong shift or channel is O(1)
        assert rel <= 1e-3 and err.max() <= 5e-3, label


@pytest.mark.parametrize("T", ["half", "float"])
def test_beyond_2e31_samples(T):
    """[8194][64][4096] real samples, 2^31 + 2^19 per array (4.3 GB fp16,
    8.6 GB fp32), channel d's filter a unit impulse at (17 d + 1) mod N, so
    every output row is its input row rolled; checked on the first rows, a
    spread and every row past sample 2^31."""
    import torch

    import thunderfft_amd as thff

    n, channels = 4096, 64
    batch = (1 << 31) // (channels * n) + 2
    rows_total = batch * channels
    shifts = (17 * np.arange(channels) + 1) % n
    h = np.zeros((channels, n), dtype=np.float32)
    h[np.arange(channels), shifts] = 1.0
    thff.ThunderFFTInitialize(T, n)
    d_x = torch.empty(rows_total * n, dtype=torch.float32 if T == "float" else torch.float16,
                      device="cuda")
    d_x.uniform_(-1, 1)
    d_spec = spectra(T, n, h, 1.0 / n)
    d_y = torch.full_like(d_x, float("nan"))
    thff.ThunderFFT_conv1d_real(T, n, d_x, d_spec, d_y, batch, channels)
    rows = torch.from_numpy(np.unique(np.concatenate([
        np.arange(3), np.linspace(0, rows_total - 1, 16).astype(np.int64),
        np.arange((1 << 31) // n - 2, rows_total)]))).cuda()
    xs = d_x.view(rows_total, n).index_select(0, rows).float()
    ys = d_y.view(rows_total, n).index_select(0, rows).float()
    s = torch.from_numpy(shifts).cuda()[rows % channels]
    idx = (torch.arange(n, device="cuda")[None, :] - s[:, None]) % n
    want = torch.gather(xs, 1, idx)
    assert bool(torch.isfinite(ys).all())
    rel = float(torch.linalg.vector_norm(ys - want) / torch.linalg.vector_norm(want))
    worst = float((ys - want).abs().max())
    print(f"{T} real conv N={n} rows={rows_total}: sampled rows rel_l2={rel:.3e} "
          f"max={worst:.3e}", flush=True)
    if T == "float":
        assert bool(((ys - want).abs() <= 1e-5 * want.abs() + 2e-6).all())
    else:
        assert rel <= 1e-3 and worst <= 5e-3
    del d_x, d_y
    torch.cuda.empty_cache()


def test_n4096_many_channels_odd_batch():
    """fp16 N = 4096 with 262145 channels: row 1 of a pair lies D N = 2^30 + 4096
    values past row 0, so the row offsets pass 2^31 bytes within one pair.
    Odd batch (3): the second pair has no row 1.  Channel d's filter is a
    unit impulse at (17 d + 1) mod N, so each output row is its input row
    rolled; checked on rows of every batch index at spread channels, the
    first and the last."""
    import torch

    import thunderfft_amd as thff

    n, channels, batch = 4096, 262145, 3
    assert 2 * (channels + 1) * n > 2**31 - 1
    thff.ThunderFFTInitialize("half", n)
    shifts = (17 * torch.arange(channels, device="cuda") + 1) % n
    d_h = torch.zeros(channels, n, dtype=torch.float32, device="cuda")
    d_h[torch.arange(channels, device="cuda"), shifts] = 1.0
    d_spec = torch.empty(channels, n, 2, dtype=torch.float32, device="cuda")
    thff.ThunderFFT_conv1d_real_filter("half", n, d_h, d_spec, channels, 1.0 / n)
    del d_h
    rows_total = batch * channels
    d_x = torch.empty(rows_total * n, dtype=torch.float16, device="cuda")
    d_x.uniform_(-1, 1)
    d_y = torch.full_like(d_x, float("nan"))
    thff.ThunderFFT_conv1d_real("half", n, d_x, d_spec, d_y, batch, channels)
    chans = torch.tensor([0, 1, 2, 131072, 262143, 262144], device="cuda")
    rows = (torch.arange(batch, device="cuda")[:, None] * channels + chans[None, :]).reshape(-1)
    xs = d_x.view(rows_total, n).index_select(0, rows).float()
    ys = d_y.view(rows_total, n).index_select(0, rows).float()
    s = shifts[rows % channels]
    idx = (torch.arange(n, device="cuda")[None, :] - s[:, None]) % n
    want = torch.gather(xs, 1, idx)
    assert bool(torch.isfinite(ys).all())
    rel = float(torch.linalg.vector_norm(ys - want) / torch.linalg.vector_norm(want))
    worst = float((ys - want).abs().max())
    print(f"half real conv N={n} channels={channels} batch={batch}: rel_l2={rel:.3e} "
          f"max={worst:.3e}", flush=True)
    assert rel <= 1e-3 and worst <= 5e-3
    del d_x, d_y, d_spec
    torch.cuda.empty_cache()
