"""GPU parity of the tiled valid 1-D correlation (thff_conv1d_valid) through
the C ABI.

The reference's conv1d_direct_fft_kernel (sample/conv1d/main.cu:38-128)
slides 64-point FFT windows (valid part 65 - F) over one complex half2
signal; its driver (:207-336) draws inputs with srand(42)/rand() and reports
the relative L2 and Linf errors against the direct definition
y[i] = sum_k x[i + k] f[k] (:156-174).  Here:

* the sample's own cases (its default 65536 x 9 and the README's 1024 x 9)
  and the filter-length extremes on its own seeded inputs, half and float,
  gated at 5e-3 against both the direct result of the stored inputs and the
  sample's own comparison against the unrounded fp32 inputs;
* batches of odd-length signals, input_len == filter_len, every filter
  length 1..64 on a short signal, with output sentinels;
* at 2^24 samples the property that a unit impulse at tap k0 shifts the
  signal, y[i] = x[i + k0]: per output for float (fp32 arithmetic), against
  the signal scale for half (its 256-point windows run on MFMA with f16
  data at each DFT16 stage).
"""
import numpy as np
import pytest

import oracle
from thff_testlib import GATE, from_device, to_device

pytestmark = pytest.mark.gpu

TIGHT = {"float": 2e-6, "half": 1e-3}
# The half path runs its 256-point windows on MFMA with f16 data at each
# DFT16 stage: per-output errors are bounded against the signal scale.
HALF_MAX_ABS = 5e-3
GUARD = 16
GUARD_VALUE = -271.0 + 137.0j


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch

    import thunderfft_amd as thff

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    thff.lib()
    thff.ThunderFFTInitialize("float", 64)
    thff.ThunderFFTInitialize("half", 64)
    yield
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")


def run(T, x, f, batch=1, sync=True):
    """x: complex (batch, L) host values T can hold; f: complex taps.  Returns
    the device output (batch, L - F + 1) and the count of changed sentinels."""
    import torch

    import thunderfft_amd as thff

    length, ntaps = x.shape[-1], f.size
    out = length - ntaps + 1
    count = batch * out
    d_x = to_device(x.reshape(-1), T)
    d_f = torch.from_numpy(np.ascontiguousarray(f, dtype=np.complex64).view(np.float32)).cuda()
    host = np.full(count + GUARD, np.nan + 0j, dtype=np.complex64)
    host[count:] = GUARD_VALUE
    d_y = to_device(host, T)
    if sync:
        thff.ThunderFFT_conv1d_valid(T, d_x, length, d_f, ntaps, d_y, batch)
    else:
        thff.ThunderFFT_conv1d_valid_async(T, d_x, length, d_f, ntaps, d_y, batch)
        torch.cuda.synchronize()
    y = from_device(d_y, T)
    guards = int(np.sum(y[count:] != np.complex64(GUARD_VALUE)))
    return y[:count].reshape(batch, out), guards


@pytest.mark.parametrize("T", ["half", "float"])
@pytest.mark.parametrize("length,ntaps", [(65536, 9), (1024, 9), (4096, 1), (4096, 64),
                                          (1000, 33), (64, 64)])
def test_sample_cases_on_sample_inputs(T, length, ntaps):
    x32, f = oracle.conv1d_valid_inputs(length, ntaps, seed=42)
    xr = oracle.represent(x32, T)
    y, guards = run(T, xr[None, :], f)
    m = oracle.metrics(y[0], oracle.conv1d_valid(xr, f))
    # the sample's own comparison: against the unrounded fp32 inputs (main.cu:314-322)
    m_sample = oracle.metrics(y[0], oracle.conv1d_valid(x32, f))
    label = (f"{T} L={length} F={ntaps}: rel_l2={m['rel_l2']:.3e} "
             f"(vs fp32 inputs {m_sample['rel_l2']:.3e}, linf {m_sample['rel_linf']:.3e})")
    print(label, flush=True)
    assert m["nonfinite"] == 0 and guards == 0, label
    assert m["rel_l2"] <= TIGHT[T] and m_sample["rel_l2"] <= GATE, label


@pytest.mark.parametrize("T", ["float", "half"])
def test_every_filter_length_and_batches(T):
    rng = np.random.default_rng(64)
    for ntaps in range(1, 65):
        for length, batch in ((ntaps, 3), (ntaps + 200 + 7 * ntaps, 2), (3001, 1)):
            if length < ntaps:
                continue
            x = (rng.uniform(-1, 1, (batch, length)) + 1j * rng.uniform(-1, 1, (batch, length)))
            f = (rng.normal(size=ntaps) + 1j * rng.normal(size=ntaps)) / np.sqrt(ntaps)
            xr = oracle.represent(x.astype(np.complex64), T)
            y, guards = run(T, xr, f.astype(np.complex64), batch)
            m = oracle.metrics(y, oracle.conv1d_valid(xr, f.astype(np.complex64)))
            label = f"{T} F={ntaps} L={length} B={batch}: rel_l2={m['rel_l2']:.3e}"
            assert m["nonfinite"] == 0 and guards == 0, label
            assert m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label
    print(f"{T}: 64 filter lengths x 3 shapes pass", flush=True)


@pytest.mark.parametrize("T", ["float", "half"])
def test_async_equals_sync(T):
    x, f = oracle.conv1d_valid_inputs(5000, 17, seed=5)
    xr = oracle.represent(x, T)[None, :]
    a, _ = run(T, xr, f)
    b, _ = run(T, xr, f, sync=False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("ntaps,k0", [(9, 5), (64, 63), (1, 0)])
def test_large_impulse_shifts(T, ntaps, k0):
    """2 signals of 2^23 + 13 samples; f = unit impulse at tap k0."""
    import torch

    import thunderfft_amd as thff

    length, batch = (1 << 23) + 13, 2
    out = length - ntaps + 1
    dt = torch.float32 if T == "float" else torch.float16
    d_x = torch.empty(2 * batch * length, dtype=dt, device="cuda").uniform_(-1, 1)
    f = np.zeros(ntaps, dtype=np.complex64)
    f[k0] = 1.0
    d_f = torch.from_numpy(f.view(np.float32)).cuda()
    d_y = torch.full((2 * batch * out,), float("nan"), dtype=dt, device="cuda")
    thff.ThunderFFT_conv1d_valid(T, d_x, length, d_f, ntaps, d_y, batch)
    x = from_device(d_x, T).reshape(batch, length)
    y = from_device(d_y, T).reshape(batch, out)
    expect = x[:, k0:k0 + out]
    err = np.abs(y - expect)
    rel_l2 = float(np.linalg.norm(err) / np.linalg.norm(expect))
    label = f"{T} F={ntaps} k0={k0}: max_err={err.max():.3e} rel_l2={rel_l2:.3e}"
    print(label, flush=True)
    assert np.all(np.isfinite(y)), label
    if T == "float":
        # fp32 arithmetic: per-element
        assert np.all(err <= 1e-6 * np.abs(expect) + 1e-6), label
    else:
        # MFMA: f16 data at each DFT16 stage spreads rounding over a window,
        # so errors are bounded against the signal scale (|x| <= 1)
        assert err.max() <= HALF_MAX_ABS and rel_l2 <= TIGHT["half"], label


@pytest.mark.parametrize("T", ["half", "float"])
def test_signal_beyond_2e31_values(T):
    """One signal of 2^31 + 777 complex values (8.6 GB fp16, 17 GB fp32) with a
    unit impulse at tap 5 of 9: y[i] = x[i + 5].  Checked on the first 2^20
    outputs and on every output from 2^31 - 2^20 to the end."""
    import torch

    import thunderfft_amd as thff

    ntaps, k0 = 9, 5
    length = (1 << 31) + 777
    out = length - ntaps + 1
    dt = torch.float32 if T == "float" else torch.float16
    d_x = torch.empty(2 * length, dtype=dt, device="cuda")
    thff.fill_uniform(T, d_x, length, oracle.BENCH_SEED_BASE + 91)
    f = np.zeros(ntaps, dtype=np.complex64)
    f[k0] = 1.0
    d_f = torch.from_numpy(f.view(np.float32)).cuda()
    d_y = torch.full((2 * out,), float("nan"), dtype=dt, device="cuda")
    thff.ThunderFFT_conv1d_valid(T, d_x, length, d_f, ntaps, d_y)
    for lo, hi in ((0, 1 << 20), ((1 << 31) - (1 << 20), out)):
        y = d_y[2 * lo:2 * hi].float()
        want = d_x[2 * (lo + k0):2 * (hi + k0)].float()
        err = (y - want).abs()
        if T == "float":
            ok = bool((err <= 1e-6 * want.abs() + 1e-6).all())
        else:  # MFMA: bounded against the signal scale (|x| <= 1)
            rel_l2 = float(torch.linalg.vector_norm(err) / torch.linalg.vector_norm(want))
            ok = float(err.max()) <= HALF_MAX_ABS and rel_l2 <= TIGHT["half"]
        ok = ok and bool(torch.isfinite(y).all())
        print(f"{T} outputs [{lo}, {hi}): max_err={float(err.max()):.3e}", flush=True)
        assert ok, (T, lo, hi)
    del d_x, d_y
    torch.cuda.empty_cache()
