"""The drop-in boundary on the CPU: library exports, the reference's 18 host API
checks (sample/validation/fft_validation.cu:320-352) through both the Python
mirror and the C++ template API, all decided before any HIP call."""
import os
import re
import subprocess

import pytest

import thunderfft_amd as thff

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "thunderfft", "thunderfft.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(thff_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 8
    L = thff.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert L.thff_version() >= 100


@pytest.mark.parametrize("T", ["float", "half"])
def test_host_checks_python(T):
    checks = 0
    for args, what in [((0, 0, -1), "negative batch"), ((0, 8, 1), "null input"),
                       ((8, 0, 1), "null output"), ((8, 8, 1), "aliased input/output")]:
        with pytest.raises(ValueError):
            thff.ThunderFFT_global(T, 64, True, *args)
        checks += 1
    thff.ThunderFFT_global(T, 64, True, 0, 0, 0)  # zero batch: no-op before pointers/HIP
    checks += 1
    for n in (-1, 0, 32, 8192):
        with pytest.raises(ValueError, match="unsupported FFT size"):
            thff.ThunderFFTInitialize(T, n)
        checks += 1
    assert checks == 9


def test_check_order_and_messages():
    # the reference checks batch sign before the pointers (thunderfft_impl_kernel.cuh:18-21)
    with pytest.raises(ValueError, match="nonnegative"):
        thff.ThunderFFT_global("float", 64, True, 8, 8, -1)
    with pytest.raises(ValueError, match="Unsupported ThunderFFT length"):
        thff.ThunderFFT_global("float", 100, True, 8, 16, 1)
    with pytest.raises(ValueError):
        thff.ThunderFFT_global("double", 64, True, 8, 16, 1)
    with pytest.raises(ValueError):
        thff.ThunderFFTInitialize("bf16", 64)
    assert thff.transforms_per_block(1024) == 4 and thff.transforms_per_block(64) == 64


def test_cpp_template_api_host_only():
    """Compile the C++ validation program against <thunderfft/thunderfft.cuh> and
    run its --host-only mode (the reference's GPU-free test, README.md:53)."""
    exe = os.path.join(ROOT, "thunderfft_amd", "_build", "thff_validate")
    if not os.path.exists(exe):
        from thunderfft_amd import build
        build.build_apps()
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    res = subprocess.run([exe, "--host-only"], capture_output=True, text=True, env=env,
                         timeout=120)
    assert res.returncode == 0, res.stderr
    assert "18 checks passed before any HIP calls" in res.stderr
    bad = subprocess.run([exe, "--bogus"], capture_output=True, text=True, env=env, timeout=60)
    assert bad.returncode == 2


def test_conv1d_argument_checks():
    """thff_conv1d rejects bad arguments before any HIP call (same rules as
    ThunderFFT_global, plus: the output may alias neither input)."""
    with pytest.raises(ValueError, match="nonnegative"):
        thff.ThunderFFT_conv1d("float", 64, 8, 16, 24, -1)
    thff.ThunderFFT_conv1d("float", 64, 0, 0, 0, 0)  # zero batch: no-op
    for args in ((0, 16, 24), (8, 0, 24), (8, 16, 0), (8, 16, 8), (8, 16, 16)):
        with pytest.raises(ValueError):
            thff.ThunderFFT_conv1d("float", 64, *args, 1)
    with pytest.raises(ValueError, match="Unsupported"):
        thff.ThunderFFT_conv1d("float", 96, 8, 16, 24, 1)
    with pytest.raises(ValueError):
        thff.ThunderFFT_conv1d("double", 64, 8, 16, 24, 1)


def test_conv2d_argument_checks():
    """thff_conv2d: square 64, 128 or 1024 images only; the rest as
    thff_conv1d, before any HIP call (the 1024 x 1024 form allocates its
    workspace only after every check)."""
    for rows, cols in ((32, 64), (64, 128), (128, 64), (256, 256), (2048, 2048), (1024, 512)):
        with pytest.raises(ValueError, match="64 x 64, 128 x 128 and 1024 x 1024"):
            thff.ThunderFFT_conv2d("float", rows, cols, 16, 32, 48, 1)
    for size in (64, 128, 1024):
        with pytest.raises(ValueError, match="nonnegative"):
            thff.ThunderFFT_conv2d("float", size, size, 16, 32, 48, -1)
        thff.ThunderFFT_conv2d("half", size, size, 0, 0, 0, 0)  # zero batch: no-op
        for args in ((0, 16, 32), (16, 0, 32), (16, 32, 0), (16, 32, 16), (16, 32, 32),
                     (24, 32, 48), (16, 40, 48), (16, 32, 56)):
            with pytest.raises(ValueError):
                thff.ThunderFFT_conv2d("float", size, size, *args, 1)
    with pytest.raises(ValueError, match="exceeds one launch"):
        thff.ThunderFFT_conv2d("float", 1024, 1024, 16, 32, 48, (1 << 16) + 1)


def test_conv1d_real_argument_checks():
    """thff_conv1d_real and its filter preparation reject bad arguments before
    any HIP call; the signal and output must be 16-byte aligned."""
    conv, filt = thff.ThunderFFT_conv1d_real, thff.ThunderFFT_conv1d_real_filter
    with pytest.raises(ValueError, match="nonnegative"):
        conv("half", 256, 16, 32, 48, -1, 1)
    conv("half", 256, 0, 0, 0, 0, 1)  # zero batch: no-op
    with pytest.raises(ValueError, match="channels must be positive"):
        conv("half", 256, 16, 32, 48, 1, 0)
    for args in ((0, 32, 48), (16, 0, 48), (16, 32, 0), (16, 32, 16), (16, 32, 32)):
        with pytest.raises(ValueError):
            conv("half", 256, *args, 1, 1)
    with pytest.raises(ValueError, match="16-byte aligned"):
        conv("half", 256, 24, 32, 48, 1, 1)
    with pytest.raises(ValueError, match="16-byte aligned"):
        conv("float", 256, 16, 32, 56, 1, 1)
    with pytest.raises(ValueError, match="Unsupported"):
        conv("half", 200, 16, 32, 48, 1, 1)
    with pytest.raises(ValueError):
        conv("double", 256, 16, 32, 48, 1, 1)
    # filter spectra
    with pytest.raises(ValueError, match="nonnegative"):
        filt("half", 256, 16, 32, -1)
    filt("half", 256, 0, 0, 0)  # zero channels: no-op
    for args in ((0, 32), (16, 0), (16, 16)):
        with pytest.raises(ValueError):
            filt("half", 256, *args, 1)
    with pytest.raises(ValueError, match="Unsupported"):
        filt("float", 8192, 16, 32, 1)


def test_conv1d_valid_argument_checks():
    """thff_conv1d_valid: the sample's two checks (1 <= filter_len <= 64,
    input_len >= filter_len), then batch, pointers, aliasing and alignment,
    all before any HIP call."""
    v = thff.ThunderFFT_conv1d_valid
    for ntaps in (0, 65, -1):
        with pytest.raises(ValueError, match="filter_len"):
            v("half", 16, 100, 32, ntaps, 48, 1)
    with pytest.raises(ValueError, match="input_len"):
        v("half", 16, 8, 32, 9, 48, 1)
    with pytest.raises(ValueError, match="nonnegative"):
        v("half", 16, 100, 32, 9, 48, -1)
    v("half", 0, 100, 0, 9, 0, 0)  # zero batch: no-op
    for args in ((0, 32, 48), (16, 0, 48), (16, 32, 0), (16, 32, 16), (16, 32, 32)):
        x, f, y = args
        with pytest.raises(ValueError):
            v("half", x, 100, f, 9, y, 1)
    with pytest.raises(ValueError, match="misaligned"):
        v("float", 20, 100, 32, 9, 48, 1)   # float2 input not 8-byte aligned
    with pytest.raises(ValueError, match="misaligned"):
        v("half", 16, 100, 36, 9, 48, 1)    # fp32 complex taps not 8-byte aligned
    with pytest.raises(ValueError):
        v("double", 16, 100, 32, 9, 48, 1)


def test_misaligned_buffers_rejected():
    """The convolutions move 16-byte vectors, so they reject buffers that do
    not start on a 16-byte boundary (THFF_EINVAL, before any HIP call).
    ThunderFFT_global takes any vec2_t<T> buffer, as the reference does: it
    rejects only buffers below the element's alignment (8 bytes for float2, 4
    for half2); element-aligned ones pass the argument checks."""
    for T, bad, elem_aligned in (("float", 20, 24), ("half", 18, 20)):
        for x, y in ((bad, 48), (16, bad + 32)):
            with pytest.raises(ValueError, match="aligned"):
                thff.ThunderFFT_global(T, 64, True, x, y, 1)
        # Past the argument checks: no table is live (none can be without a GPU),
        # so the call fails with the runtime error, not ValueError.
        try:
            thff.ThunderFFTFinalize(T)
        except RuntimeError:
            pass
        with pytest.raises(RuntimeError):
            thff.ThunderFFT_global(T, 64, True, elem_aligned, 48, 1)
        with pytest.raises(ValueError, match="16-byte aligned"):
            thff.ThunderFFT_conv1d(T, 64, 16, 24, 48, 1)
        with pytest.raises(ValueError, match="16-byte aligned"):
            thff.ThunderFFT_conv1d(T, 64, 16, 32, 56, 1, False)
        with pytest.raises(ValueError, match="16-byte aligned"):
            thff.ThunderFFT_conv2d(T, 64, 64, 24, 32, 48, 1)


def test_fft_convenience_argument_checks():
    """fft() checks its arguments before any HIP call: dtype and shape, the
    length, and a caller's `out` (dtype, shape, device, contiguity, overlap);
    host tensors are refused last (there is no CPU path)."""
    torch = pytest.importorskip("torch")
    x = torch.zeros(4, 64, dtype=torch.complex64)
    with pytest.raises(ValueError, match="complex64 or float16"):
        thff.fft(torch.zeros(4, 64, dtype=torch.float32))
    with pytest.raises(ValueError, match="unsupported FFT size"):
        thff.fft(torch.zeros(4, 100, dtype=torch.complex64))
    with pytest.raises(ValueError, match="unsupported FFT size"):
        thff.fft(torch.zeros(4, 96, 2, dtype=torch.float16))
    bad_outs = [torch.zeros(4, 64, dtype=torch.complex128), torch.zeros(2, 64, dtype=torch.complex64),
                torch.zeros(64, 4, dtype=torch.complex64).t()]
    for out in bad_outs:
        with pytest.raises(ValueError, match="out must"):
            thff.fft(x, out=out)
    with pytest.raises(ValueError, match="overlap"):
        thff.fft(x, out=x)
    big = torch.zeros(8, 64, dtype=torch.complex64)
    with pytest.raises(ValueError, match="overlap"):
        thff.fft(big[:4], out=big[2:6])
    with pytest.raises(ValueError, match="device tensor"):
        thff.fft(x, out=torch.zeros_like(x))


def test_copy_nt_argument_checks():
    """The benchmark's streaming copy rejects bad sizes and null, misaligned or
    overlapping buffers (THFF_EINVAL, before any HIP call); zero bytes is a no-op."""
    thff.copy_nt(0, 0, 0)
    for dst, src, n in ((4096, 0, 16), (0, 4096, 16), (4104, 8192, 16), (4096, 8200, 32),
                        (4096, 8192, 24), (4096, 8192, -16), (4096, 4096 + 16, 64),
                        (4096 + 16, 4096, 64)):
        with pytest.raises(ValueError):
            thff.copy_nt(dst, src, n)
