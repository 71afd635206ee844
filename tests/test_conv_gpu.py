"""GPU parity of the fused FFT convolution (thff_conv1d) against the fp64
direct circular convolution, through the C ABI.

The reference gates its fused convolution on the relative L2 of the output
against a direct circular convolution (sample/conv1d/
conv1d_fullfft_l4096_thunder.cu:499-554, gate 5e-3).  Here: every length x
{float, half} x {per-signal, shared filter}, batches that leave a partial last
tile; BASELINE config 4 (16384 signals of 2048, per-signal filters) on a
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
    """Complex taps with re, im ~ N(0, 1/sqrt(n))."""
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
    """16384 signals of 2048, per-signal filters."""
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
