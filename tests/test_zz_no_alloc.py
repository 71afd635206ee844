"""The allocation-free 2-D convolution entry point, thff_conv2d_noalloc (no
counterpart in the reference: for callers that cannot allocate device
memory), called through the C ABI and checked bit for bit against the
allocating entry point, thff_conv2d_async, on the same inputs: two calls in a
row for each image size and precision, the second with fewer images, so that
the per-GPU workspace array is reused with a smaller input after a larger
one.  The 1024 x 1024 form is the one that uses the workspace; 64 and 128
take the fused kernels and are checked the same way."""
import ctypes

import numpy as np
import pytest

import oracle
from thff_testlib import from_device, to_device

pytestmark = pytest.mark.gpu


def _call(L, fn, T, size, d_x, d_h, d_y, batch):
    rc = getattr(L, fn)(0 if T == "float" else 1, size, size, ctypes.c_void_p(d_x.data_ptr()),
                        ctypes.c_void_p(d_h.data_ptr()), ctypes.c_void_p(d_y.data_ptr()), batch,
                        None)
    assert rc == 0, (fn, rc, L.thff_last_error())


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("size", [1024, 128, 64])
def test_conv2d_noalloc_matches_allocating_entry(T, size):
    import torch

    import thunderfft_amd as thff

    L = thff.lib()
    thff.ThunderFFTInitialize(T, size)
    rng = np.random.default_rng(size + (T == "half"))
    h = np.zeros((size, size), dtype=np.complex64)
    h[:7, :7] = rng.normal(0.0, 1.0 / 7.0, (7, 7)) + 1j * rng.normal(0.0, 1.0 / 7.0, (7, 7))
    d_h = to_device(oracle.represent(h, T), T)
    for batch in (3, 1):  # the second call is smaller than the first
        x = oracle.uniform(size * size, batch, seed=1000 * batch + size).reshape(batch, size, size)
        d_x = to_device(oracle.represent(x, T), T)
        d_ref = to_device(np.full((batch, size, size), np.nan, dtype=np.complex64), T)
        d_y = to_device(np.full((batch, size, size), np.nan, dtype=np.complex64), T)
        _call(L, "thff_conv2d_async", T, size, d_x, d_h, d_ref, batch)
        torch.cuda.synchronize()
        _call(L, "thff_conv2d_noalloc", T, size, d_x, d_h, d_y, batch)
        torch.cuda.synchronize()
        ref = from_device(d_ref, T)
        y = from_device(d_y, T)
        print(f"{T} {size}x{size} batch={batch}: noalloc == allocating "
              f"{np.array_equal(y.view(np.uint32), ref.view(np.uint32))}", flush=True)
        assert np.isfinite(y).all()
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (T, size, batch)


def test_conv2d_noalloc_rejects_before_any_hip_call():
    """Argument checks as thff_conv2d's, before any HIP call; shapes the
    allocation-free workspace cannot hold are rejected."""
    import thunderfft_amd as thff

    L = thff.lib()
    for rows, cols in ((2048, 2048), (256, 256), (1024, 512)):
        assert L.thff_conv2d_noalloc(0, rows, cols, 16, 32, 48, 1, None) == -22
    assert L.thff_conv2d_noalloc(0, 1024, 1024, 16, 32, 48, 0, None) == 0  # zero batch: no-op
    assert L.thff_conv2d_noalloc(0, 1024, 1024, 16, 32, 16, 1, None) == -22  # y aliases x
    assert L.thff_conv2d_noalloc(0, 1024, 1024, 16, 32, 40, 1, None) == -22  # misaligned y
