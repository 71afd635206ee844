"""Shared helpers for the parity tests: device buffers, guarded outputs and the
oracle comparison of fft_validation.cu:194-276 (reference tree)."""
from __future__ import annotations

import numpy as np

import oracle

SIZES = (64, 128, 256, 512, 1024, 2048, 4096)
GATE = 5e-3  # relative L2 limit, sample/validation/fft_validation.cu:26
# Tighter bars this build is held to (fp32 arithmetic throughout): float
# results carry only fp32 rounding; half results add one output rounding to
# binary16 (relative 2^-11 per component at worst).
TIGHT = {"float": 2e-6, "half": 1e-3}
OUTPUT_GUARD = 16          # fft_validation.cu:25
GUARD_VALUE = (-271.0, 137.0)


def to_device(x: np.ndarray, T: str):
    """complex64 host array -> device tensor holding T storage (float2 / half2)."""
    import torch

    x = np.ascontiguousarray(x, dtype=np.complex64)
    if T == "float":
        return torch.from_numpy(x.view(np.float32).copy()).cuda()
    bits = oracle.f32_to_f16_bits(x.view(np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).cuda().view(torch.float16)


def from_device(t, T: str) -> np.ndarray:
    """device tensor of T storage -> complex64 host array."""
    import torch

    if T == "float":
        return t.detach().cpu().numpy().view(np.complex64)
    bits = t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    return oracle.f16_bits_to_f32(bits).view(np.complex64)


def guarded_output(count: int, T: str):
    """NaN-filled output of `count` complex values followed by OUTPUT_GUARD sentinels."""
    host = np.full(count + OUTPUT_GUARD, np.nan + 0j, dtype=np.complex64)
    host[count:] = GUARD_VALUE[0] + 1j * GUARD_VALUE[1]
    return to_device(host, T)


def guards_changed(out_host: np.ndarray, count: int) -> int:
    g = out_host[count:]
    return int(np.sum((g.real != GUARD_VALUE[0]) | (g.imag != GUARD_VALUE[1])))


def run_case(T: str, n: int, forward: bool, x: np.ndarray, sync_api: bool = True) -> dict:
    """One validation case: device FFT of x (shape (batch, n)) vs the fp64 oracle
    of the values T actually represents."""
    import thunderfft_amd as thff

    batch = x.shape[0]
    count = batch * n
    xr = oracle.represent(x, T)
    d_in = to_device(xr, T)
    d_out = guarded_output(count, T)
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_global(T, n, forward, d_in, d_out, batch)
    out = from_device(d_out, T)
    ref = oracle.fft(xr, forward=forward)
    m = oracle.metrics(out[:count], ref.reshape(-1))
    m["guards_changed"] = guards_changed(out, count)
    m["out"] = out[:count].reshape(batch, n)
    m["ref"] = ref
    return m
