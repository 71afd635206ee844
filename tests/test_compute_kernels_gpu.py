"""One pass of the differential-compute kernels (libthff_bench_compute.so,
thffx_compute_repeat with repeats = 1 is one forward N = 1024 transform)
against the fp64 oracle: the library's fp32 VALU transform, and the float
transform with both DFT16 stages on the matrix cores -- exact fp32 MFMA
(v_mfma_f32_16x16x4_f32) and the bf16x3 split on v_mfma_f32_16x16x32_bf16 --
whose speed bench.py measures.  Prints each relative L2 (the accuracy the
bf16x3 split reaches is part of that measurement)."""
import ctypes
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "thunderfft_amd", "_build", "libthff_bench_compute.so")
# mode -> (kernel, relative L2 bound against the fp64 transform)
MODES = {0: ("fp32 VALU", 2e-6), 2: ("fp32 MFMA 16x16x4", 2e-6), 3: ("bf16x3 MFMA", 1e-4)}


@pytest.mark.parametrize("mode", sorted(MODES))
def test_compute_kernel_single_pass(mode):
    import torch

    import thunderfft_amd as thff

    L = ctypes.CDLL(LIB)
    L.thffx_compute_repeat.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    n, batch = 1024, 12
    x = oracle.uniform(n, batch)
    d_in = torch.from_numpy(x.view(np.float32).copy()).cuda()
    d_out = torch.full_like(d_in, float("nan"))
    thff.ThunderFFTInitialize("float", n)
    rc = L.thffx_compute_repeat(mode, d_in.data_ptr(), d_out.data_ptr(), batch, 1, None)
    torch.cuda.synchronize()
    assert rc == 0
    got = d_out.cpu().numpy().view(np.complex64)
    m = oracle.metrics(got, oracle.fft(x, True).reshape(-1))
    name, bound = MODES[mode]
    print(f"{name}: one forward N=1024 pass, rel_l2={m['rel_l2']:.3e} "
          f"rel_linf={m['rel_linf']:.3e}", flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= bound
    thff.ThunderFFTFinalize("float")
