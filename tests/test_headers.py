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
