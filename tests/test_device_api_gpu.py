"""GPU tests of the device-side fusion API (<thunderfft/thunderfft_device.hpp>).

Kernels written against the public API the way a caller would
(thunderfft_amd/apps/device_example.hip, built into
thunderfft_amd/_build/libthff_device_example.so) are run through ctypes:

* the reference's validate_core pattern (sample/validation/
  fft_validation.cu:84-123): gmem -> smem (layout_t) -> fragment ->
  ThunderFFT_kernel_reg -> smem -> gmem, with 64 workspace sentinels that must
  survive;
* the same through ThunderFFT_gmem2reg / reg2gmem only;
* a fused forward FFT x per-bin filter x inverse FFT / N;
* both again through ThunderFFT_kernel_reg(reg, W, workspace) in the
  reference's argument types, W for half from
  unit_fp16::make_reg_b_precompute<N, fwd> (the reference's fused-sample
  pattern, sample/README.md:406-409), for float the table.

Every length x {float, half} x {forward, inverse} against the fp64 oracle;
the float results must also agree with ThunderFFT_global's to rel L2 1e-6
(both run the same passes; the compiler may contract them differently).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle
from thff_testlib import GATE, SIZES, TIGHT, from_device, to_device

pytestmark = pytest.mark.gpu

EXAMPLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "thunderfft_amd", "_build", "libthff_device_example.so")
PREC = {"float": 0, "half": 1}


@pytest.fixture(scope="module")
def ex():
    import torch

    import thunderfft_amd as thff

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    thff.lib()
    if not os.path.exists(EXAMPLE):
        raise FileNotFoundError(f"{EXAMPLE} missing: run __graft_entry__.build()")
    L = ctypes.CDLL(EXAMPLE)
    vp, ci = ctypes.c_void_p, ctypes.c_int
    L.thffx_device_fft.argtypes = [ci, ci, ci, vp, vp, ci, vp, vp]
    L.thffx_device_fft_reg.argtypes = [ci, ci, ci, vp, vp, ci, vp]
    L.thffx_fused_filter.argtypes = [ci, ci, vp, vp, vp, ci, vp]
    L.thffx_fragment_map.argtypes = [ci, ci, vp, vp]
    L.thffx_device_fft_w.argtypes = [ci, ci, ci, vp, vp, ci, vp]
    L.thffx_device_fft_reversed_in.argtypes = [ci, ci, ci, vp, vp, ci, vp, vp]
    L.thffx_fused_filter_w.argtypes = [ci, ci, vp, vp, vp, ci, vp]
    yield L
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_device_api_fft(ex, T, n):
    import torch

    import thunderfft_amd as thff

    bpb = thff.transforms_per_block(n)
    batch = 2 * bpb
    thff.ThunderFFTInitialize(T, n)
    x = oracle.represent(oracle.uniform(n, batch, seed=31 + n), T)
    d_x = to_device(x, T)
    guard = torch.zeros(1, dtype=torch.int32, device="cuda")
    for forward in (True, False):
        ref = oracle.fft(x, forward)
        d_lib = torch.empty_like(d_x)
        thff.ThunderFFT_global(T, n, forward, d_x, d_lib, batch)
        for kind in ("smem", "reg", "smem_reversed_in"):
            d_y = torch.full_like(d_x, float("nan"))
            if kind == "smem":
                rc = ex.thffx_device_fft(PREC[T], n, int(forward), d_x.data_ptr(), d_y.data_ptr(),
                                         batch, guard.data_ptr(), None)
            elif kind == "smem_reversed_in":
                # a reversed input layout: the permutation the transforms expect (identity)
                rc = ex.thffx_device_fft_reversed_in(PREC[T], n, int(forward), d_x.data_ptr(),
                                                     d_y.data_ptr(), batch, guard.data_ptr(), None)
            else:
                rc = ex.thffx_device_fft_reg(PREC[T], n, int(forward), d_x.data_ptr(),
                                             d_y.data_ptr(), batch, None)
            assert rc == 0, (kind, rc)
            y = from_device(d_y, T).reshape(batch, n)
            m = oracle.metrics(y, ref)
            label = f"device API ({kind}) {T} N={n} {'fwd' if forward else 'inv'}: rel_l2={m['rel_l2']:.3e}"
            print(label, flush=True)
            assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label
            if T == "float":
                # Same passes as the library kernel; the compiler may fuse the other
                # multiply of a complex product into an FMA, so rounding may differ.
                lib = from_device(d_lib, T).reshape(batch, n)
                assert oracle.metrics(y, lib)["rel_l2"] <= 1e-6, label
    assert int(guard.item()) == 0, "workspace sentinels changed"


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", [64, 1024, 2048, 4096])
def test_device_api_fused_filter(ex, T, n):
    import thunderfft_amd as thff

    bpb = thff.transforms_per_block(n)
    batch = 3 * bpb
    thff.ThunderFFTInitialize(T, n)
    x = oracle.represent(oracle.uniform(n, batch, seed=7 * n), T)
    rng = np.random.default_rng(n)
    H = (rng.normal(size=n) + 1j * rng.normal(size=n)).astype(np.complex64)
    d_x = to_device(x, T)
    d_h = to_device(H, "float")
    d_y = to_device(np.full((batch, n), np.nan, dtype=np.complex64), T)
    assert ex.thffx_fused_filter(PREC[T], n, d_x.data_ptr(), d_y.data_ptr(), d_h.data_ptr(),
                                 batch, None) == 0
    y = from_device(d_y, T).reshape(batch, n)
    ref = oracle.fft(oracle.fft(x, True) * H.astype(np.complex128)[None, :], False) / n
    m = oracle.metrics(y, ref)
    label = f"device API fused filter {T} N={n}: rel_l2={m['rel_l2']:.3e}"
    print(label, flush=True)
    # half: the spectrum is also rounded to binary16 between the transforms
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE
    assert m["rel_l2"] <= (5e-6 if T == "float" else 2e-3), label


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_device_api_precomputed_coefficients(ex, T, n):
    """ThunderFFT_kernel_reg(reg, W, ws): half with per-lane coefficients
    built by make_reg_b_precompute (no table), float with the table; every
    length and direction against the oracle, and the fused filter."""
    import thunderfft_amd as thff

    bpb = thff.transforms_per_block(n)
    batch = 2 * bpb
    thff.ThunderFFTInitialize(T, n)
    x = oracle.represent(oracle.uniform(n, batch, seed=53 + n), T)
    d_x = to_device(x, T)
    for forward in (True, False):
        d_y = to_device(np.full((batch, n), np.nan, dtype=np.complex64), T)
        assert ex.thffx_device_fft_w(PREC[T], n, int(forward), d_x.data_ptr(), d_y.data_ptr(),
                                     batch, None) == 0
        m = oracle.metrics(from_device(d_y, T).reshape(batch, n), oracle.fft(x, forward))
        label = f"device API (W) {T} N={n} {'fwd' if forward else 'inv'}: rel_l2={m['rel_l2']:.3e}"
        print(label, flush=True)
        assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label
    rng = np.random.default_rng(n + 1)
    H = (rng.normal(size=n) + 1j * rng.normal(size=n)).astype(np.complex64)
    d_h = to_device(H, "float")
    d_y = to_device(np.full((batch, n), np.nan, dtype=np.complex64), T)
    assert ex.thffx_fused_filter_w(PREC[T], n, d_x.data_ptr(), d_y.data_ptr(), d_h.data_ptr(),
                                   batch, None) == 0
    ref = oracle.fft(oracle.fft(x, True) * H.astype(np.complex128)[None, :], False) / n
    m = oracle.metrics(from_device(d_y, T).reshape(batch, n), ref)
    label = f"device API fused filter (W) {T} N={n}: rel_l2={m['rel_l2']:.3e}"
    print(label, flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= (5e-6 if T == "float" else 2e-3), label


@pytest.mark.parametrize("T", ["float", "half"])
def test_fragment_order_is_a_bijection(ex, T):
    """fragment_transform / fragment_element map the block's 256 lanes x 16
    registers one-to-one onto its batch_per_block<N> transforms x N elements, for
    every length (half at N = 256 ... 4096 uses the MFMA layouts)."""
    import torch

    import thunderfft_amd as thff

    for n in SIZES:
        d_map = torch.full((2 * 256 * 16,), -1, dtype=torch.int32, device="cuda")
        assert ex.thffx_fragment_map(PREC[T], n, d_map.data_ptr(), None) == 0
        m = d_map.cpu().numpy().reshape(256 * 16, 2)
        bpb = thff.transforms_per_block(n)
        assert m[:, 0].min() >= 0 and m[:, 0].max() < bpb, (T, n)
        assert m[:, 1].min() >= 0 and m[:, 1].max() < n, (T, n)
        flat = m[:, 0].astype(np.int64) * n + m[:, 1]
        assert np.unique(flat).size == bpb * n == 4096, (T, n)


def documented_order(T, n, tid, j):
    """The fragment order the device header's contract states: (transform,
    element) of register j of lane tid."""
    w, lane = tid // 64, tid % 64
    nn, q, b, r = lane % 16, lane // 16, j // 4, j % 4
    if T == "float" or n <= 128:
        return tid // (n // 16), tid % (n // 16) + (n // 16) * j
    if n == 2048:
        return w // 2, 4 * (w % 2) + b + 8 * nn + 128 * (q + 4 * r)
    if n == 4096:
        return 0, 4 * w + b + 16 * nn + 256 * (q + 4 * r)
    c = n // 256
    return w * (4 // c) + b // c, nn + 16 * (b % c) + 16 * c * (q + 4 * r)


@pytest.mark.parametrize("T", ["float", "half"])
def test_fragment_order_matches_contract(ex, T):
    """The order the kernels use is the one the header documents, so a caller
    can index per-bin data (a filter spectrum) without calling the device
    helpers."""
    import torch

    for n in SIZES:
        d_map = torch.full((2 * 256 * 16,), -1, dtype=torch.int32, device="cuda")
        assert ex.thffx_fragment_map(PREC[T], n, d_map.data_ptr(), None) == 0
        m = d_map.cpu().numpy().reshape(256, 16, 2)
        want = np.array([[documented_order(T, n, tid, j) for j in range(16)] for tid in range(256)])
        assert np.array_equal(m, want), (T, n)
