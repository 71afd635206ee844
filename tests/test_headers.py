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
    writes coefficient_count<N> half2 slots, never more than the reference's
    28 (N <= 128) or 36 (N >= 256), so the reference's fused kernels keep
    their arrays (W_fwd[28], sample/conv1d/main.cu:61; W_fwd[36],
    conv1d_fullfft_l4096_thunder.cu:298) at every length, as arrays or through
    a pointer.  An array below coefficient_count<N> is a compile-time error."""
    body = ("__global__ void k(const __half2* p) {{\n"
            "  vec2_t<half> W[{size}];\n"
            "  thunderfft::unit_fp16::make_reg_b_precompute<{n}, true>({arg});\n"
            "  (void)p;\n}}\n")
    checks = "".join(
        f"static_assert(thunderfft::unit_fp16::coefficient_count<{n}> <= {28 if n <= 128 else 36});\n"
        for n in (64, 128, 256, 512, 1024, 2048, 4096))
    src = checks + "".join(
        body.format(size=28 if n <= 128 else 36, n=n, arg=arg).replace("void k(", f"void k{n}{i}(")
        for n in (64, 128, 256, 512, 1024, 2048, 4096)
        for i, arg in enumerate(("W", "static_cast<vec2_t<half>*>(W)")))
    ok = _compile(tmp_path, src)
    assert ok.returncode == 0, ok.stderr
    small = _compile(tmp_path, body.format(
        size="thunderfft::unit_fp16::coefficient_count<1024> - 1", n=1024, arg="W"))
    assert small.returncode != 0 and "coefficient_count" in small.stderr, small.stderr


def _doc_block(text, signature):
    """The comment block that ends right before `signature` in a header."""
    end = text.index(signature)
    start = text.rindex("/*", 0, end)
    return " ".join(text[start:end].replace("*", " ").split())


def test_alignment_contract_matches_behaviour():
    """The public headers state the alignment rule thff_global implements
    (capi.cpp global_impl): element alignment is required (8 bytes for
    float2, 4 for half2, THFF_EINVAL / std::invalid_argument otherwise) and
    any element-aligned buffer is accepted, as in the reference
    (thunderfft_impl_kernel.cuh:18-21 checks no alignment at all); the
    convolutions keep a 16-byte rule.  The wording is checked against calls
    made without a GPU: every check runs before any HIP call."""
    import thunderfft_amd as thff

    h = open(os.path.join(ROOT, "include", "thunderfft", "thunderfft.h")).read()
    glob = _doc_block(h, "int thff_global(")
    assert "not aligned to its element (8 bytes for float2, 4 bytes for half2)" in glob
    assert "Any element-aligned buffer is accepted" in glob
    assert "not on a 16-byte boundary -> THFF_EINVAL" not in glob
    conv = _doc_block(h, "int thff_conv1d(")
    assert "must start on a 16-byte boundary" in conv
    hpp = " ".join(open(os.path.join(ROOT, "include", "thunderfft", "thunderfft.hpp")).read().split())
    assert "pointers not aligned to their // element (8 bytes for float2, 4 for half2) throw" \
        " std::invalid_argument" in hpp
    assert "not 16-byte aligned pointers throw" not in hpp

    for T, elem in (("float", 8), ("half", 4)):
        try:
            thff.ThunderFFTFinalize(T)
        except RuntimeError:
            pass
        # below the element's alignment: rejected by the argument checks
        with pytest.raises(ValueError, match=f"{elem}-byte aligned"):
            thff.ThunderFFT_global(T, 64, True, 4096 + elem // 2, 8192, 1)
        # element-aligned but not 16-byte aligned: accepted by the checks, so
        # the call gets as far as the (missing) twiddle table
        for x, y in ((4096 + elem, 8192), (4096, 8192 + elem)):
            with pytest.raises(RuntimeError):
                thff.ThunderFFT_global(T, 64, True, x, y, 1)
        # the convolutions keep the 16-byte rule
        with pytest.raises(ValueError, match="16-byte aligned"):
            thff.ThunderFFT_conv1d(T, 64, 4096 + elem, 8192, 12288, 1)
