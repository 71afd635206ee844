"""CPU oracle for the batched C2C FFT hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker.  The product
(``thunderfft_amd``) never imports it and has no CPU fallback.

The numerical work is in ``thff_oracle.c`` / ``thff_oracle_mt.cpp`` (built by
``oracle/Makefile`` into ``libthff_oracle.so``); this module is a thin numpy
wrapper.  Each C function cites the reference file:line it restates.  Every
function is pinned in ``tests/test_oracle.py`` (closed-form spectra,
Parseval, linearity, round trip, brute force, numpy.fft, numpy.float16).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libthff_oracle.so")
_lib = None

BENCH_SEED_BASE = 0x7F4A7C15  # seed = BENCH_SEED_BASE + N for the benchmark workloads


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc/g++ only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "libthff_oracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        fp = ctypes.POINTER(ctypes.c_float)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        L.thff_dft_f64.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, dp, dp]
        L.thff_fft_f64.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, dp, dp]
        L.thff_fft_f32_fourstep.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, fp, fp,
                                            ctypes.c_int]
        L.thff_fft_f32_batched.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, fp, fp,
                                           ctypes.c_int]
        L.thff_metrics.argtypes = [ctypes.c_long, fp, dp, dp]
        L.thff_metrics.restype = None
        L.thff_f32_to_f16_array.argtypes = [ctypes.c_long, fp, u16p]
        L.thff_f32_to_f16_array.restype = None
        L.thff_f16_to_f32_array.argtypes = [ctypes.c_long, u16p, fp]
        L.thff_f16_to_f32_array.restype = None
        L.thff_uniform_fill.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_long, fp]
        L.thff_uniform_fill.restype = None
        L.thff_make_input_kind.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, fp]
        L.thff_make_input_gaussian.argtypes = [ctypes.c_int, ctypes.c_long, fp]
        L.thff_circconv1d_f64.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int, dp, dp, dp]
        L.thff_circconv2d_f64.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_long, dp, dp, dp]
        L.thff_circconv1d_channels_f64.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int,
                                                   ctypes.c_int, dp, dp, dp]
        L.thff_conv_real_inputs.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_long,
                                            ctypes.c_int, ctypes.c_uint, fp, fp]
        L.thff_conv1d_valid_f64.argtypes = [ctypes.c_long, ctypes.c_int, ctypes.c_long, dp, dp,
                                            dp]
        L.thff_conv1d_valid_inputs.argtypes = [ctypes.c_long, ctypes.c_int, ctypes.c_uint, fp,
                                               fp]
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _as_c128(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.complex128)


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


def dft(x, forward: bool = True) -> np.ndarray:
    """Closed-form fp64 DFT along the last axis (unnormalized both ways)."""
    x = _as_c128(x)
    n = x.shape[-1]
    out = np.empty_like(x)
    _check(lib().thff_dft_f64(n, x.size // n, -1 if forward else 1,
                              _p(x.view(np.float64), ctypes.c_double),
                              _p(out.view(np.float64), ctypes.c_double)), "dft")
    return out


def fft(x, forward: bool = True) -> np.ndarray:
    """Iterative radix-2 fp64 FFT along the last axis (power-of-two N)."""
    x = _as_c128(x)
    n = x.shape[-1]
    out = np.empty_like(x)
    _check(lib().thff_fft_f64(n, x.size // n, -1 if forward else 1,
                              _p(x.view(np.float64), ctypes.c_double),
                              _p(out.view(np.float64), ctypes.c_double)), "fft")
    return out


def fft_f32_fourstep(x, forward: bool = True, threads: int = 1) -> np.ndarray:
    """fp32 restatement of the reference's radix-4 four-step (CPU baseline)."""
    x = np.ascontiguousarray(x, dtype=np.complex64)
    n = x.shape[-1]
    out = np.empty_like(x)
    _check(lib().thff_fft_f32_fourstep(n, x.size // n, -1 if forward else 1,
                                       _p(x.view(np.float32), ctypes.c_float),
                                       _p(out.view(np.float32), ctypes.c_float), threads),
           "fft_f32_fourstep")
    return out


def fft_f32_batched(x, forward: bool = True, threads: int = 1, out=None) -> np.ndarray:
    """fp32 radix-4 FFT vectorised across 16 signals at a time (the CPU
    baseline; thff_oracle_simd.c).  `out`: a complex64 array of x's shape to
    write into (reused by a timing loop, so no pass pays for new pages)."""
    x = np.ascontiguousarray(x, dtype=np.complex64)
    n = x.shape[-1]
    if out is None:
        out = np.empty_like(x)
    if out.shape != x.shape or out.dtype != np.complex64 or not out.flags.c_contiguous:
        raise ValueError("out must be a C-contiguous complex64 array of x's shape")
    _check(lib().thff_fft_f32_batched(n, x.size // n, -1 if forward else 1,
                                      _p(x.view(np.float32), ctypes.c_float),
                                      _p(out.view(np.float32), ctypes.c_float), threads),
           "fft_f32_batched")
    return out


def metrics(y, ref) -> dict:
    """rel_l2, max_abs, rel_linf, nonfinite -- fft_validation.cu:247-272."""
    y = np.ascontiguousarray(y, dtype=np.complex64)
    ref = _as_c128(ref)
    assert y.size == ref.size
    out = np.zeros(4, dtype=np.float64)
    lib().thff_metrics(y.size, _p(y.view(np.float32), ctypes.c_float),
                       _p(ref.view(np.float64), ctypes.c_double), _p(out, ctypes.c_double))
    return {"rel_l2": float(out[0]), "max_abs": float(out[1]), "rel_linf": float(out[2]),
            "nonfinite": int(out[3])}


def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().thff_f32_to_f16_array(x.size, _p(x, ctypes.c_float), _p(out, ctypes.c_uint16))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().thff_f16_to_f32_array(h.size, _p(h, ctypes.c_uint16), _p(out, ctypes.c_float))
    return out


def represent(x, dtype: str) -> np.ndarray:
    """Values the storage type actually holds (encode -> decode), as complex64."""
    x = np.ascontiguousarray(x, dtype=np.complex64)
    if dtype == "float":
        return x
    flat = x.view(np.float32)
    return f16_bits_to_f32(f32_to_f16_bits(flat)).view(np.complex64).reshape(x.shape)


def uniform(n: int, batch: int, seed: int | None = None, first_element: int = 0) -> np.ndarray:
    """Counter-based U[-1,1) complex signals, shape (batch, n), complex64."""
    if seed is None:
        seed = BENCH_SEED_BASE + n
    out = np.empty(2 * n * batch, dtype=np.float32)
    lib().thff_uniform_fill(seed & (2**64 - 1), 2 * first_element, out.size,
                            _p(out, ctypes.c_float))
    return out.view(np.complex64).reshape(batch, n)


INPUT_KINDS = ("gaussian_rms1", "offset_impulse", "complex_tone", "constant")


def make_input(n: int, batch: int, kind: int) -> np.ndarray:
    """fft_validation.cu:130-163 input kinds, shape (batch, n), complex64."""
    out = np.empty(2 * n * batch, dtype=np.float32)
    if kind == 0:
        rc = lib().thff_make_input_gaussian(n, batch, _p(out, ctypes.c_float))
    else:
        rc = lib().thff_make_input_kind(n, batch, kind, _p(out, ctypes.c_float))
    _check(rc, "make_input")
    return out.view(np.complex64).reshape(batch, n)


def circconv1d(x, h, per_signal_filter: bool = True) -> np.ndarray:
    x = _as_c128(x)
    h = _as_c128(h)
    n = x.shape[-1]
    out = np.empty_like(x)
    _check(lib().thff_circconv1d_f64(n, x.size // n, int(per_signal_filter),
                                     _p(x.view(np.float64), ctypes.c_double),
                                     _p(h.view(np.float64), ctypes.c_double),
                                     _p(out.view(np.float64), ctypes.c_double)), "circconv1d")
    return out


def circconv2d(x, h) -> np.ndarray:
    x = _as_c128(x)
    h = _as_c128(h)
    rows, cols = x.shape[-2], x.shape[-1]
    out = np.empty_like(x)
    _check(lib().thff_circconv2d_f64(rows, cols, x.size // (rows * cols),
                                     _p(x.view(np.float64), ctypes.c_double),
                                     _p(h.view(np.float64), ctypes.c_double),
                                     _p(out.view(np.float64), ctypes.c_double)), "circconv2d")
    return out


def circconv1d_channels(x, h, taps: int | None = None) -> np.ndarray:
    """Real direct circular convolution, one filter per channel (fp64).

    x: real (..., channels, n) signals; h: real (channels, n) filters of which
    the first ``taps`` (default n) are used.  conv1d_fullfft_l4096_thunder.cu:499-520.
    """
    x = np.ascontiguousarray(x, dtype=np.float64)
    h = np.ascontiguousarray(h, dtype=np.float64)
    channels, n = h.shape
    assert x.shape[-1] == n and x.shape[-2] == channels
    taps = n if taps is None else taps
    out = np.empty_like(x)
    _check(lib().thff_circconv1d_channels_f64(n, x.size // n, channels, taps,
                                              _p(x, ctypes.c_double), _p(h, ctypes.c_double),
                                              _p(out, ctypes.c_double)), "circconv1d_channels")
    return out


def conv_real_inputs(n: int, taps: int, batch: int, channels: int, seed: int = 42):
    """The real convolution sample's seeded inputs (srand(seed), rand()).

    Returns x float32 (batch, channels, n) and h float32 (channels, n), taps
    k >= ``taps`` zero.  conv1d_fullfft_l4096_thunder.cu:389-401, seed 42 at :617.
    """
    x = np.empty((batch, channels, n), dtype=np.float32)
    h = np.empty((channels, n), dtype=np.float32)
    _check(lib().thff_conv_real_inputs(n, taps, batch * channels, channels, seed,
                                       _p(x, ctypes.c_float), _p(h, ctypes.c_float)),
           "conv_real_inputs")
    return x, h


def conv1d_valid(x, f) -> np.ndarray:
    """Valid complex correlation y[..., i] = sum_k x[..., i + k] * f[k] (fp64, no
    conjugation), sample/conv1d/main.cu:156-174.  x: (..., L), f: (F,)."""
    x = _as_c128(x)
    f = _as_c128(f).reshape(-1)
    length, ntaps = x.shape[-1], f.size
    out = np.empty(x.shape[:-1] + (length - ntaps + 1,), dtype=np.complex128)
    _check(lib().thff_conv1d_valid_f64(length, ntaps, x.size // length,
                                       _p(x.view(np.float64), ctypes.c_double),
                                       _p(f.view(np.float64), ctypes.c_double),
                                       _p(out.view(np.float64), ctypes.c_double)), "conv1d_valid")
    return out


def conv1d_valid_inputs(length: int, ntaps: int, seed: int = 42):
    """The tiled-conv sample's inputs after srand(seed): complex64 x (length,) then
    taps (ntaps,), each component rand()/RAND_MAX.  sample/conv1d/main.cu:130-135,233,260-262."""
    x = np.empty(length, dtype=np.complex64)
    f = np.empty(ntaps, dtype=np.complex64)
    _check(lib().thff_conv1d_valid_inputs(length, ntaps, seed, _p(x.view(np.float32), ctypes.c_float),
                                          _p(f.view(np.float32), ctypes.c_float)),
           "conv1d_valid_inputs")
    return x, f
