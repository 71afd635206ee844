"""Every public and internal header compiles on its own for gfx950 (the
reference ships a header-only library; its callers include any one header
first), with hipcc -fsyntax-only, no GPU needed."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["thunderfft/thunderfft.h", "thunderfft/thunderfft.hpp", "thunderfft/thunderfft.cuh",
           "thunderfft/thunderfft_device.hpp"] + [
    f"thunderfft/detail/{h}" for h in ("fft_core.hpp", "fft_tile.hpp", "fft_c2c.hpp",
                                      "fft_conv.hpp", "fft_mfma.hpp", "fft_conv_mfma.hpp")]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    pytest.skip("hipcc not found")


@pytest.mark.parametrize("header", HEADERS)
def test_header_is_self_contained(header, tmp_path):
    src = tmp_path / "inc.hip"
    src.write_text(f"#include <{header}>\n#include <{header}>\n")  # and include-guarded
    res = subprocess.run([hipcc(), "--offload-arch=gfx950", "-std=c++17", "-fsyntax-only",
                          "-I", os.path.join(ROOT, "include"), str(src)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr


def _compile(tmp_path, source):
    src = tmp_path / "k.hip"
    src.write_text("#include <thunderfft/thunderfft.cuh>\n" + source)
    return subprocess.run([hipcc(), "--offload-arch=gfx950", "-std=c++17", "-fsyntax-only",
                           "-I", os.path.join(ROOT, "include"), str(src)],
                          capture_output=True, text=True, timeout=300)


def test_reversed_layouts(tmp_path):
    """layout_t's Reversed flag (reference thunderfft.cuh:29-44): accepted on
    an input layout (the permutation the transforms expect, the identity
    here); an output layout must not be reversed, as in the reference
    (thunderfft_impl_helper.cuh:51-56), which is a compile-time error here."""
    reversed_l = "using L = thunderfft::layout_t<256, 16, 1, 272, 16, 1, true>;\n"
    ok = _compile(tmp_path, reversed_l +
                  "static_assert(L::reversed && L::at(3, 1) == 3 + 272 + (275 / 16));\n"
                  "__global__ void k(const __half2* in) {\n"
                  "  __shared__ __half2 s[16 * 289];\n"
                  "  thunderfft::ThunderFFT_gmem2smem<half, L>(s, in);\n}\n")
    assert ok.returncode == 0, ok.stderr
    bad = _compile(tmp_path, reversed_l +
                   "__global__ void k(__half2* out) {\n"
                   "  __shared__ __half2 s[16 * 289];\n"
                   "  thunderfft::ThunderFFT_smem2gmem<half, L>(out, s);\n}\n")
    assert bad.returncode != 0 and "must not be reversed" in bad.stderr


def test_precomputed_coefficients_array_size(tmp_path):
    """unit_fp16::make_reg_b_precompute (reference unit_kernel_fp16.cuh:97-108)
    writes coefficient_count<N> half2 slots: an array argument is checked at
    compile time, so a reference kernel's W[36] at N = 1024 (more slots are
    needed there) fails to compile instead of being overrun; a right-sized
    array and a pointer compile."""
    body = ("__global__ void k(const __half2* p) {{\n"
            "  vec2_t<half> W[{size}];\n"
            "  thunderfft::unit_fp16::make_reg_b_precompute<1024, true>({arg});\n"
            "  (void)p;\n}}\n")
    ok = _compile(tmp_path, body.format(
        size="thunderfft::unit_fp16::coefficient_count<1024>", arg="W"))
    assert ok.returncode == 0, ok.stderr
    ptr = _compile(tmp_path, body.format(
        size="thunderfft::unit_fp16::coefficient_count<1024>", arg="static_cast<vec2_t<half>*>(W)"))
    assert ptr.returncode == 0, ptr.stderr
    small = _compile(tmp_path, body.format(size="36", arg="W"))
    assert small.returncode != 0 and "coefficient_count" in small.stderr, small.stderr
