"""Pin the CPU oracle (oracle/) before trusting it (CPU only).

Each oracle function is checked against something it does not compute
itself: the golden fixtures written by numpy.fft from a pure-Python input
generator, closed-form spectra of the reference's input kinds
(sample/validation/fft_validation.cu:130-163), Parseval / linearity /
round-trip invariants, brute force on tiny N, and numpy.float16 rounding.
The last group plants plausible mistakes in oracle-side data to show that the
5e-3 relative-L2 gate (fft_validation.cu:26) catches each of them.
"""
import os

import numpy as np
import pytest

import oracle
from thff_testlib import GATE, SIZES

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c2c_numpy.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def rel(a, b):
    return float(np.linalg.norm((np.asarray(a) - np.asarray(b)).ravel()) /
                 np.linalg.norm(np.asarray(b).ravel()))


# ---------------------------------------------------------------- generators
def test_uniform_matches_python_restatement(golden):
    for key in golden.files:
        if key.endswith("_x"):
            x = golden[key]
            n = x.shape[-1]
            got = oracle.uniform(n, x.shape[0])
            assert got.dtype == np.complex64 and got.shape == x.shape
            assert np.array_equal(got.view(np.uint32), x.view(np.uint32)), key


def test_uniform_range_and_offset():
    x = oracle.uniform(1024, 64).view(np.float32)
    assert x.min() >= -1.0 and x.max() < 1.0
    assert abs(float(x.mean())) < 0.01 and abs(float(x.var()) - 1 / 3) < 0.01
    # first_element offsets the counter: a slice equals the tail of the whole
    whole = oracle.uniform(64, 8)
    tail = oracle.uniform(64, 3, first_element=5 * 64)
    assert np.array_equal(whole[5:], tail)


def test_input_kinds_closed_form():
    n, batch = 64, 9
    g = oracle.make_input(n, batch, 0)
    rms = np.sqrt(np.mean(np.abs(g.astype(np.complex128)) ** 2, axis=1))
    assert np.allclose(rms, 1.0, atol=1e-6)
    imp = oracle.make_input(n, batch, 1)
    for b in range(batch):
        nz = np.flatnonzero(imp[b])
        assert list(nz) == [(13 * b + 7) % n] and imp[b, nz[0]] == np.complex64(0.75 + 0.25j)
    tone = oracle.make_input(n, batch, 2)
    k = np.arange(n)
    for b in range(batch):
        f = 1 + (7 * b) % (n - 1)
        expect = 0.5 * np.exp(1j * (2 * np.pi * f * k / n + 0.13 * b))
        assert np.abs(tone[b] - expect).max() < 1e-6
    const = oracle.make_input(n, batch, 3)
    assert np.all(const == np.complex64(0.25 - 0.125j))


# ---------------------------------------------------------------- DFT / FFT
@pytest.mark.parametrize("forward", [True, False])
def test_dft_and_fft_match_numpy_golden(golden, forward):
    tag = "fwd" if forward else "inv"
    for key in golden.files:
        if not key.endswith("_x"):
            continue
        x = golden[key]
        expect = golden[key[:-2] + "_" + tag]
        assert rel(oracle.fft(x, forward), expect) < 1e-13, key
        if x.shape[-1] <= 1024:  # O(N^2)
            assert rel(oracle.dft(x, forward), expect) < 1e-12, key


@pytest.mark.parametrize("n", [2, 4, 8])
def test_brute_force_tiny(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n)) + 1j * rng.standard_normal((3, n))
    for forward in (True, False):
        s = -1 if forward else 1
        expect = np.zeros_like(x)
        for b in range(3):
            for k in range(n):
                expect[b, k] = sum(x[b, j] * complex(np.cos(2 * np.pi * j * k / n),
                                                     s * np.sin(2 * np.pi * j * k / n))
                                   for j in range(n))
        assert rel(oracle.dft(x, forward), expect) < 1e-14
        assert rel(oracle.fft(x, forward), expect) < 1e-14


@pytest.mark.parametrize("n", SIZES)
def test_fft_equals_dft_all_sizes(n):
    x = oracle.uniform(n, 2)
    for forward in (True, False):
        if n <= 1024:
            assert rel(oracle.fft(x, forward), oracle.dft(x, forward)) < 1e-13
        assert rel(oracle.fft(x, forward), np.fft.fft(x.astype(np.complex128)) if forward
                   else np.fft.ifft(x.astype(np.complex128)) * n) < 1e-13


@pytest.mark.parametrize("n", SIZES)
def test_kat_spectra(n):
    """Closed-form spectra of the reference's impulse / constant / tone inputs."""
    batch = 5
    k = np.arange(n)
    for forward in (True, False):
        s = -1.0 if forward else 1.0
        imp = oracle.make_input(n, batch, 1).astype(np.complex128)
        Y = oracle.fft(imp, forward)
        for b in range(batch):
            n0 = (13 * b + 7) % n
            expect = (0.75 + 0.25j) * np.exp(s * 2j * np.pi * k * n0 / n)
            assert np.abs(Y[b] - expect).max() < 1e-12
        const = oracle.make_input(n, batch, 3).astype(np.complex128)
        Y = oracle.fft(const, forward)
        assert np.abs(Y[:, 0] - n * (0.25 - 0.125j)).max() < 1e-12
        assert np.abs(Y[:, 1:]).max() < 1e-12
        tone = oracle.make_input(n, batch, 2).astype(np.complex128)
        Y = oracle.fft(tone, forward)
        for b in range(batch):
            f = 1 + (7 * b) % (n - 1)
            peak = f if forward else (n - f) % n
            expect = np.zeros(n, dtype=np.complex128)
            expect[peak] = n * 0.5 * np.exp(0.13j * b)
            # the tone was rounded to fp32, so leakage is fp32-sized, not zero
            assert np.abs(Y[b] - expect).max() < 1e-4 * n


@pytest.mark.parametrize("n", [64, 1024, 4096])
def test_invariants(n):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, n)) + 1j * rng.standard_normal((4, n))
    y = rng.standard_normal((4, n)) + 1j * rng.standard_normal((4, n))
    X = oracle.fft(x)
    # Parseval
    assert np.allclose(np.sum(np.abs(X) ** 2, axis=1), n * np.sum(np.abs(x) ** 2, axis=1),
                       rtol=1e-12)
    # linearity
    a, b = 0.3 - 1.1j, -2.0 + 0.5j
    assert rel(oracle.fft(a * x + b * y), a * X + b * oracle.fft(y)) < 1e-13
    # round trip, unnormalized
    assert rel(oracle.fft(X, forward=False), n * x) < 1e-13
    # conj(FFT(conj x)) = unnormalized inverse
    assert rel(np.conj(oracle.fft(np.conj(x))), oracle.fft(x, forward=False)) < 1e-13


# ---------------------------------------------------------------- fp32 baseline port
@pytest.mark.parametrize("n", SIZES)
def test_fourstep_f32_accuracy(n):
    x = oracle.uniform(n, 8)
    for forward in (True, False):
        got = oracle.fft_f32_fourstep(x, forward)
        m = oracle.metrics(got, oracle.fft(x, forward))
        assert m["rel_l2"] < 1e-6 and m["nonfinite"] == 0


def test_fourstep_threads_bitwise_identical():
    x = oracle.uniform(1024, 37)
    a = oracle.fft_f32_fourstep(x, True, threads=1)
    b = oracle.fft_f32_fourstep(x, True, threads=5)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------- fp32 batched baseline
@pytest.mark.parametrize("n", SIZES)
def test_batched_f32_accuracy(n):
    """The CPU baseline's 16-signal vector groups, on a batch that is not a
    multiple of 16 (the last group padded), against the fp64 FFT."""
    x = oracle.uniform(n, 37)
    for forward in (True, False):
        got = oracle.fft_f32_batched(x, forward, threads=3)
        m = oracle.metrics(got, oracle.fft(x, forward))
        assert m["rel_l2"] < 1e-6 and m["nonfinite"] == 0


def test_batched_f32_kats_and_threads():
    """Closed forms (an offset impulse's phasor, a tone's single bin) and a
    result independent of the thread count; a reused output is overwritten."""
    n, b = 256, 20
    x = np.zeros((b, n), np.complex64)
    x[:, 5] = 0.75 + 0.25j
    got = oracle.fft_f32_batched(x, True)
    k = np.arange(n)
    want = (0.75 + 0.25j) * np.exp(-2j * np.pi * k * 5 / n)
    assert np.max(np.abs(got - want)) < 1e-6
    t = np.exp(2j * np.pi * 7 * k / n).astype(np.complex64)
    got = oracle.fft_f32_batched(np.tile(t, (b, 1)), True)
    assert abs(got[3, 7] - n) < 1e-3 and np.max(np.abs(np.delete(got[3], 7))) < 1e-3
    y = oracle.uniform(1024, 53)
    out = np.full(y.shape, np.nan, np.complex64)
    a = oracle.fft_f32_batched(y, True, threads=1)
    c = oracle.fft_f32_batched(y, True, threads=7, out=out)
    assert c is out and np.array_equal(a.view(np.uint32), c.view(np.uint32))


# ---------------------------------------------------------------- half rounding
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(3)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf,
                        -np.inf, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10, 0.1, 1 / 3,
                        1 + 2 ** -11, 1 + 3 * 2 ** -11, 2049.0, 2051.0], dtype=np.float32)
    vals = np.concatenate([special, rng.standard_normal(200000).astype(np.float32) * 100,
                           rng.standard_normal(20000).astype(np.float32) * 1e-5,
                           (rng.integers(0, 2**32, 200000, dtype=np.uint64)
                            .astype(np.uint32).view(np.float32))])
    vals = vals[~np.isnan(vals)]
    bits = oracle.f32_to_f16_bits(vals)
    assert np.array_equal(bits, vals.astype(np.float16).view(np.uint16))
    all_bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.f16_bits_to_f32(all_bits)
    ref = all_bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(f[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(f[~finite]))


# ---------------------------------------------------------------- convolution
def test_circconv_matches_fft_product():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 32)) + 1j * rng.standard_normal((3, 32))
    h = rng.standard_normal((3, 32)) + 1j * rng.standard_normal((3, 32))
    expect = np.fft.ifft(np.fft.fft(x) * np.fft.fft(h))
    assert rel(oracle.circconv1d(x, h, True), expect) < 1e-13
    shared = oracle.circconv1d(x, h[:1], False)
    assert rel(shared, np.fft.ifft(np.fft.fft(x) * np.fft.fft(h[:1]))) < 1e-13
    x2 = rng.standard_normal((2, 8, 16)) + 1j * rng.standard_normal((2, 8, 16))
    h2 = rng.standard_normal((8, 16)) + 0j
    expect2 = np.fft.ifft2(np.fft.fft2(x2) * np.fft.fft2(h2))
    assert rel(oracle.circconv2d(x2, h2), expect2) < 1e-13


def test_circconv2d_sparse_filters_pinned():
    """The 2-D oracle skips zero taps: a single complex tap at (dr, dc) gives
    w * roll(x, (dr, dc)) (a transposed or correlated form fails), a sparse
    corner block on non-square images matches numpy's FFT product, and an
    all-zero filter gives zeros."""
    rng = np.random.default_rng(29)
    x = rng.standard_normal((2, 48, 40)) + 1j * rng.standard_normal((2, 48, 40))
    h = np.zeros((48, 40), dtype=np.complex128)
    h[5, 37] = 0.75 - 0.5j
    assert rel(oracle.circconv2d(x, h), (0.75 - 0.5j) * np.roll(x, (5, 37), axis=(1, 2))) < 1e-15
    h = np.zeros((48, 40), dtype=np.complex128)
    h[:7, :3] = rng.standard_normal((7, 3)) + 1j * rng.standard_normal((7, 3))
    expect = np.fft.ifft2(np.fft.fft2(x) * np.fft.fft2(h))
    assert rel(oracle.circconv2d(x, h), expect) < 1e-13
    assert np.array_equal(oracle.circconv2d(x, np.zeros_like(h)), np.zeros_like(x))


def test_circconv_channels_pinned():
    """Real per-channel convolution: numpy's FFT product, a shifted impulse
    (y = c * roll(x, k0): a correlation or a wrong channel would fail), the
    tap truncation, and the complex per-signal oracle with expanded filters."""
    rng = np.random.default_rng(5)
    batch, channels, n = 2, 3, 32
    x = rng.standard_normal((batch, channels, n))
    h = rng.standard_normal((channels, n))
    expect = np.fft.ifft(np.fft.fft(x) * np.fft.fft(h)[None]).real
    y = oracle.circconv1d_channels(x, h)
    assert rel(y, expect) < 1e-13
    per_signal = oracle.circconv1d(x.reshape(-1, n), np.tile(h, (batch, 1)), True)
    assert rel(y.reshape(-1, n), per_signal.real) < 1e-13
    # impulse taps: channel d delays by d + 1 and scales by d + 2
    imp = np.zeros((channels, n))
    for d in range(channels):
        imp[d, d + 1] = d + 2
    yi = oracle.circconv1d_channels(x, imp)
    for d in range(channels):
        assert np.array_equal(yi[:, d], (d + 2) * np.roll(x[:, d], d + 1, axis=-1))
    # only the first `taps` taps count
    taps = 5
    cut = h.copy()
    cut[:, taps:] = 0
    assert rel(oracle.circconv1d_channels(x, h, taps), oracle.circconv1d_channels(x, cut)) < 1e-15


def test_conv_real_inputs_are_the_c_library_sequence():
    """The sample's inputs: srand(42) then rand()/RAND_MAX per signal value and
    (rand()/RAND_MAX)/n per tap, drawn through this process's C library (a
    separate route into the same generator) and glibc's known first values."""
    import ctypes

    libc = ctypes.CDLL("libc.so.6")
    rand_max = np.float32(2147483647)
    n, taps, batch, channels = 64, 7, 3, 2
    x, h = oracle.conv_real_inputs(n, taps, batch, channels, seed=42)
    libc.srand(42)
    draws = np.array([libc.rand() for _ in range(batch * channels * n + channels * taps)])
    assert draws[0] == 71876166 and draws[1] == 708592740  # glibc, seed 42
    ex = draws[: x.size].astype(np.float32) / rand_max
    assert np.array_equal(x.reshape(-1), ex)
    eh = np.zeros((channels, n), dtype=np.float32)
    eh[:, :taps] = (draws[x.size:].astype(np.float32) / rand_max).reshape(channels, taps) / np.float32(n)
    assert np.array_equal(h, eh)


# ---------------------------------------------------------------- the gate has teeth
def test_metrics_definition():
    ref = np.array([3 + 4j, 0, 1], dtype=np.complex128)
    y = np.array([3 + 4j, 1e-3j, 1], dtype=np.complex64)
    m = oracle.metrics(y, ref)
    assert abs(m["rel_l2"] - 1e-3 / np.sqrt(26)) < 1e-9
    assert abs(m["max_abs"] - 1e-3) < 1e-9 and abs(m["rel_linf"] - 1e-3 / 5) < 1e-9
    y[1] = np.nan
    assert oracle.metrics(y, ref)["nonfinite"] == 1


@pytest.mark.parametrize("n", [64, 1024])
def test_gate_rejects_planted_mistakes(n):
    """Wrong sign, dropped twiddle, swapped digit order, dropped input term and
    missing scaling each push a correct-looking FFT far past the 5e-3 gate."""
    x = oracle.uniform(n, 4).astype(np.complex128)
    ref = oracle.fft(x, True)
    wrong_sign = oracle.fft(x, False)
    assert oracle.metrics(wrong_sign.astype(np.complex64), ref)["rel_l2"] > 100 * GATE
    # four-step with the inter-stage twiddle dropped
    n1 = 16
    n2 = n // n1
    cols = np.fft.fft(x.reshape(4, n1, n2), axis=1)  # length-n1 over stride-n2
    no_tw = np.fft.fft(cols, axis=2).transpose(0, 2, 1).reshape(4, n)
    assert oracle.metrics(no_tw.astype(np.complex64), ref)["rel_l2"] > 100 * GATE
    # transposed (digit-swapped) output order
    swapped = ref.reshape(4, n1, n2).transpose(0, 2, 1).reshape(4, n)
    assert oracle.metrics(swapped.astype(np.complex64), ref)["rel_l2"] > 100 * GATE
    # one input element dropped per signal
    x_drop = x.copy()
    x_drop[:, 5] = 0
    assert oracle.metrics(oracle.fft(x_drop).astype(np.complex64), ref)["rel_l2"] > 2 * GATE
    # inverse with a 1/N normalization the reference does not apply
    scaled = oracle.fft(ref, False) / n
    assert oracle.metrics(scaled.astype(np.complex64), n * x)["rel_l2"] > 100 * GATE


def test_conv1d_valid_pinned():
    """Valid correlation: numpy.convolve with the reversed filter (a library
    routine), a shifted impulse (y[i] = c * x[i + k0]; conjugating the taps or
    flipping the direction fails it), F = 1 and F = L, and batched rows."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal((3, 50)) + 1j * rng.standard_normal((3, 50))
    f = rng.standard_normal(9) + 1j * rng.standard_normal(9)
    y = oracle.conv1d_valid(x, f)
    assert y.shape == (3, 42)
    for b in range(3):
        assert rel(y[b], np.convolve(x[b], f[::-1], mode="valid")) < 1e-13
    imp = np.zeros(9, dtype=complex)
    imp[4] = 2 - 1j
    assert np.array_equal(oracle.conv1d_valid(x, imp), (2 - 1j) * x[:, 4:46])
    assert rel(oracle.conv1d_valid(x, f[:1]), x * f[0]) < 1e-15
    assert rel(oracle.conv1d_valid(x[:, :9], f)[:, 0], x[:, :9] @ f) < 1e-13


def test_conv1d_valid_inputs_are_the_c_library_sequence():
    import ctypes

    libc = ctypes.CDLL("libc.so.6")
    rand_max = np.float32(2147483647)
    length, ntaps = 40, 5
    x, f = oracle.conv1d_valid_inputs(length, ntaps, seed=42)
    libc.srand(42)
    draws = np.array([libc.rand() for _ in range(2 * (length + ntaps))]).astype(np.float32) / rand_max
    assert np.array_equal(x.view(np.float32), draws[: 2 * length])
    assert np.array_equal(f.view(np.float32), draws[2 * length:])
