"""thunderfft_amd -- MI355X (gfx950) ThunderFFT: batched C2C FFTs, N = 64..4096.

Python mirror of the reference's host API (mcrl/thunderfft,
include/thunderfft/thunderfft.cuh:55-63,150-154) over the C ABI of
``libthunderfft_amd.so`` (declared in include/thunderfft/thunderfft.h):

    ThunderFFTInitialize(T, N)                       # T in {"float", "half"}
    ThunderFFT_global(T, N, forward, d_in, d_out, batch, stream=0)
    ThunderFFTFinalize(T)

Errors keep the reference's two kinds: ``ValueError`` where the reference
throws ``std::invalid_argument`` (raised before any HIP call) and
``RuntimeError("[ThunderFFT] ...")`` where it throws ``std::runtime_error``.

Pointers are plain integers (device addresses); torch tensors are accepted
and their ``data_ptr()`` is used.  There is no CPU path: importing this module
fails loudly if the HIP library has not been built.
"""
from __future__ import annotations

import ctypes
import os

__all__ = [
    "SUPPORTED_N", "PRECISIONS", "lib", "ThunderFFTInitialize", "ThunderFFTFinalize",
    "ThunderFFT_global", "ThunderFFT_global_async", "twiddle_info", "fill_uniform",
    "fft", "transforms_per_block", "LIB_PATH", "ThunderFFT_conv1d", "ThunderFFT_conv1d_async",
    "ThunderFFT_conv2d", "ThunderFFT_conv2d_async", "ThunderFFT_conv2d_noalloc", "copy_nt",
]

SUPPORTED_N = (64, 128, 256, 512, 1024, 2048, 4096)
PRECISIONS = {"float": 0, "half": 1}
THFF_OK, THFF_EINVAL, THFF_EIO = 0, -22, -5

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libthunderfft_amd.so")

_lib = None


def lib() -> ctypes.CDLL:
    """Load libthunderfft_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m thunderfft_amd.build` "
                "(there is no CPU fallback)")
        # torch ships its own HIP runtime.  Loaded after this library, it would
        # be a second runtime in the process, and this library's would find no
        # device; loaded first, this library binds to torch's (same soname).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        vp = ctypes.c_void_p
        L.thff_version.restype = ctypes.c_int
        L.thff_last_error.restype = ctypes.c_char_p
        L.thff_initialize.argtypes = [ctypes.c_int, ctypes.c_int]
        L.thff_finalize.argtypes = [ctypes.c_int]
        sig = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int, vp]
        L.thff_global.argtypes = sig
        L.thff_global_async.argtypes = sig
        csig = [ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp]
        L.thff_conv1d.argtypes = csig
        L.thff_conv1d_async.argtypes = csig
        c2sig = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int, vp]
        L.thff_conv2d.argtypes = c2sig
        L.thff_conv2d_async.argtypes = c2sig
        L.thff_conv2d_noalloc.argtypes = c2sig
        rfsig = [ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.c_float, vp]
        L.thff_conv1d_real_filter.argtypes = rfsig
        L.thff_conv1d_real_filter_async.argtypes = rfsig
        rsig = [ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp]
        L.thff_conv1d_real.argtypes = rsig
        L.thff_conv1d_real_async.argtypes = rsig
        vsig = [ctypes.c_int, vp, ctypes.c_longlong, vp, ctypes.c_int, vp, ctypes.c_int, vp]
        L.thff_conv1d_valid.argtypes = vsig
        L.thff_conv1d_valid_async.argtypes = vsig
        L.thff_twiddle_info.argtypes = [ctypes.c_int, ctypes.POINTER(vp),
                                        ctypes.POINTER(ctypes.c_int)]
        L.thff_fill_uniform.argtypes = [ctypes.c_int, vp, ctypes.c_longlong, ctypes.c_ulonglong,
                                        ctypes.c_longlong, vp]
        L.thff_copy_nt.argtypes = [vp, vp, ctypes.c_longlong, vp]
        _lib = L
    return _lib


def _precision(T) -> int:
    if isinstance(T, str) and T in PRECISIONS:
        return PRECISIONS[T]
    name = getattr(T, "__name__", None) or str(T)
    for key, code in (("float16", 1), ("half", 1), ("complex32", 1), ("float32", 0),
                      ("float", 0), ("complex64", 0)):
        if key in name:
            return code
    raise ValueError(f"ThunderFFT supports float and half only (got {T!r})")


def _ptr(x) -> int:
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return int(x.data_ptr())
    raise TypeError(f"expected a device pointer or tensor, got {type(x).__name__}")


def _stream(s) -> int:
    if s is None or s == 0:
        return 0
    if isinstance(s, int):
        return s
    handle = getattr(s, "cuda_stream", None)
    if handle is None:
        raise TypeError("stream must be an integer hipStream_t or a torch.cuda.Stream")
    return int(handle)


def _raise(rc: int) -> None:
    if rc == THFF_OK:
        return
    msg = lib().thff_last_error().decode()
    if rc == THFF_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def ThunderFFTInitialize(T, N: int) -> None:
    """ThunderFFTInitialize<T>(N): build this device's twiddle table for (T, N)."""
    _raise(lib().thff_initialize(_precision(T), int(N)))


def ThunderFFTFinalize(T) -> None:
    """ThunderFFTFinalize<T>(): release this device's twiddle table for T."""
    _raise(lib().thff_finalize(_precision(T)))


def ThunderFFT_global(T, N: int, forward: bool, d_input, d_output, batch: int, stream=0) -> None:
    """ThunderFFT_global<T,N,forward>(d_input, d_output, batch, stream); synchronous."""
    _raise(lib().thff_global(_precision(T), int(N), int(bool(forward)), _ptr(d_input),
                             _ptr(d_output), int(batch), _stream(stream)))


def ThunderFFT_global_async(T, N: int, forward: bool, d_input, d_output, batch: int,
                            stream=0) -> None:
    """As ThunderFFT_global, but returns once the launch is enqueued on ``stream``."""
    _raise(lib().thff_global_async(_precision(T), int(N), int(bool(forward)), _ptr(d_input),
                                   _ptr(d_output), int(batch), _stream(stream)))


def ThunderFFT_conv1d(T, N: int, d_x, d_h, d_y, batch: int, per_signal_filter: bool = True,
                      stream=0) -> None:
    """Fused circular convolution y[b] = IFFT(FFT(x[b]) * FFT(h[b or 0])) / N; synchronous."""
    _raise(lib().thff_conv1d(_precision(T), int(N), _ptr(d_x), _ptr(d_h), _ptr(d_y), int(batch),
                             int(bool(per_signal_filter)), _stream(stream)))


def ThunderFFT_conv1d_async(T, N: int, d_x, d_h, d_y, batch: int, per_signal_filter: bool = True,
                            stream=0) -> None:
    """As ThunderFFT_conv1d, but returns once the launch is enqueued on ``stream``."""
    _raise(lib().thff_conv1d_async(_precision(T), int(N), _ptr(d_x), _ptr(d_h), _ptr(d_y),
                                   int(batch), int(bool(per_signal_filter)), _stream(stream)))


def ThunderFFT_conv1d_real_filter(T, N: int, d_h, d_spectrum, channels: int, scale: float = 1.0,
                                  stream=0) -> None:
    """spectrum[d] = scale * FFT(h[d]) for real fp32 filters h (channels, N) -> complex64
    spectra (channels, N), for ThunderFFT_conv1d_real of type T; synchronous."""
    _raise(lib().thff_conv1d_real_filter(_precision(T), int(N), _ptr(d_h), _ptr(d_spectrum),
                                         int(channels), float(scale), _stream(stream)))


def ThunderFFT_conv1d_real_filter_async(T, N: int, d_h, d_spectrum, channels: int,
                                        scale: float = 1.0, stream=0) -> None:
    """As ThunderFFT_conv1d_real_filter, but returns once the launch is enqueued."""
    _raise(lib().thff_conv1d_real_filter_async(_precision(T), int(N), _ptr(d_h), _ptr(d_spectrum),
                                               int(channels), float(scale), _stream(stream)))


def ThunderFFT_conv1d_real(T, N: int, d_x, d_spectrum, d_y, batch: int, channels: int,
                           stream=0) -> None:
    """Real fused convolution y[b][d] = Re IFFT(FFT(x[b][d]) * spectrum[d]) of real
    (batch, channels, N) signals of type T; synchronous."""
    _raise(lib().thff_conv1d_real(_precision(T), int(N), _ptr(d_x), _ptr(d_spectrum), _ptr(d_y),
                                  int(batch), int(channels), _stream(stream)))


def ThunderFFT_conv1d_real_async(T, N: int, d_x, d_spectrum, d_y, batch: int, channels: int,
                                 stream=0) -> None:
    """As ThunderFFT_conv1d_real, but returns once the launch is enqueued on ``stream``."""
    _raise(lib().thff_conv1d_real_async(_precision(T), int(N), _ptr(d_x), _ptr(d_spectrum),
                                        _ptr(d_y), int(batch), int(channels), _stream(stream)))


def ThunderFFT_conv1d_valid(T, d_x, input_len: int, d_taps, filter_len: int, d_y, batch: int = 1,
                            stream=0) -> None:
    """Tiled valid correlation y[b][i] = sum_k x[b][i + k] * taps[k] (complex, type T;
    taps complex64, 1 <= filter_len <= 64) through 64-point FFT windows; synchronous."""
    _raise(lib().thff_conv1d_valid(_precision(T), _ptr(d_x), int(input_len), _ptr(d_taps),
                                   int(filter_len), _ptr(d_y), int(batch), _stream(stream)))


def ThunderFFT_conv1d_valid_async(T, d_x, input_len: int, d_taps, filter_len: int, d_y,
                                  batch: int = 1, stream=0) -> None:
    """As ThunderFFT_conv1d_valid, but returns once the launch is enqueued on ``stream``."""
    _raise(lib().thff_conv1d_valid_async(_precision(T), _ptr(d_x), int(input_len), _ptr(d_taps),
                                         int(filter_len), _ptr(d_y), int(batch), _stream(stream)))


def ThunderFFT_conv2d(T, rows: int, cols: int, d_x, d_h, d_y, batch: int, stream=0) -> None:
    """2-D circular convolution y[b] = IFFT2(FFT2(x[b]) * FFT2(h)) / (rows*cols) with
    one shared filter: 64 x 64 and 128 x 128 images in one fused kernel per image,
    1024 x 1024 as row pass, fused column pass, inverse row pass; synchronous."""
    _raise(lib().thff_conv2d(_precision(T), int(rows), int(cols), _ptr(d_x), _ptr(d_h), _ptr(d_y),
                             int(batch), _stream(stream)))


def ThunderFFT_conv2d_async(T, rows: int, cols: int, d_x, d_h, d_y, batch: int, stream=0) -> None:
    """As ThunderFFT_conv2d, but returns once the launch is enqueued on ``stream``."""
    _raise(lib().thff_conv2d_async(_precision(T), int(rows), int(cols), _ptr(d_x), _ptr(d_h),
                                   _ptr(d_y), int(batch), _stream(stream)))


def ThunderFFT_conv2d_noalloc(T, rows: int, cols: int, d_x, d_h, d_y, batch: int,
                              stream=0) -> None:
    """As ThunderFFT_conv2d_async, but allocates no device memory (the 1024 x 1024
    form keeps its filter spectrum in the library's per-GPU device array; calls
    that overlap on one GPU race)."""
    _raise(lib().thff_conv2d_noalloc(_precision(T), int(rows), int(cols), _ptr(d_x), _ptr(d_h),
                                     _ptr(d_y), int(batch), _stream(stream)))


def twiddle_info(T) -> tuple[int, int]:
    """(device pointer, N) of this device's twiddle table for T; (0, 0) when released."""
    p = ctypes.c_void_p()
    n = ctypes.c_int()
    _raise(lib().thff_twiddle_info(_precision(T), ctypes.byref(p), ctypes.byref(n)))
    return int(p.value or 0), int(n.value)


def fill_uniform(T, d_out, count: int, seed: int, first_element: int = 0, stream=0) -> None:
    """Seeded U[-1,1) complex values (same formula as the test oracle's generator)."""
    _raise(lib().thff_fill_uniform(_precision(T), _ptr(d_out), int(count),
                                   int(seed) & (2**64 - 1), int(first_element), _stream(stream)))


def copy_nt(d_dst, d_src, nbytes: int, stream=0) -> None:
    """Non-temporal 16-byte streaming copy (the bandwidth ceiling bench.py reports)."""
    _raise(lib().thff_copy_nt(_ptr(d_dst), _ptr(d_src), int(nbytes), _stream(stream)))


def transforms_per_block(N: int) -> int:
    """Transforms per 256-lane workgroup of the global kernel."""
    return 256 * 16 // int(N)


def fft(x, forward: bool = True, out=None):
    """Transform the last axis of a CUDA tensor (complex64 or float16[..., N, 2]).

    A convenience over ThunderFFT_global.  ``out``, when given, must match
    ``x`` in dtype, shape and device, be contiguous and not overlap ``x``;
    every argument is checked (ValueError) before any HIP call.  The table for
    (T, N) is initialised on the tensor's device if needed, and the length
    that was current for T before the call is made current again afterwards
    (its table is kept, so that costs no allocation).
    """
    import torch

    if x.dtype == torch.complex64:
        T, n = "float", x.shape[-1]
    elif x.dtype == torch.float16 and x.dim() >= 2 and x.shape[-1] == 2:
        T, n = "half", x.shape[-2]
    else:
        raise ValueError("fft expects complex64 or float16[..., N, 2] tensors")
    if n not in SUPPORTED_N:
        raise ValueError(f"fft: unsupported FFT size {n} (supported: {SUPPORTED_N})")
    if out is not None:
        if out.dtype != x.dtype or tuple(out.shape) != tuple(x.shape) or out.device != x.device:
            raise ValueError("fft: out must match x in dtype, shape and device")
        if not out.is_contiguous():
            raise ValueError("fft: out must be contiguous")
        nbytes = x.numel() * x.element_size()
        if nbytes and (x.data_ptr() < out.data_ptr() + nbytes and
                       out.data_ptr() < x.data_ptr() + nbytes):
            raise ValueError("fft: out must not overlap x")
    if not x.is_cuda:
        raise ValueError("fft expects a device tensor (there is no CPU path)")
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    batch = x.numel() // (n * (2 if T == "half" else 1))
    if batch == 0:
        return out
    with torch.cuda.device(x.device):
        previous = twiddle_info(T)[1]
        if previous != n:
            ThunderFFTInitialize(T, n)
        try:
            ThunderFFT_global(T, n, forward, x, out, batch, torch.cuda.current_stream(x.device))
        finally:
            if previous not in (0, n):
                ThunderFFTInitialize(T, previous)
    return out
