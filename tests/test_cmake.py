"""The CMake build (CMakeLists.txt): configures with THUNDERFFT_ARCH=gfx950,
builds libthunderfft_amd through the `thunderfft` target's dependency and
exports every C ABI symbol; a consumer that links `thunderfft` compiles
against <thunderfft/thunderfft.hpp>, and its HIP kernels that instantiate the
device fusion API get the library's device flags (packed FP32 off, MFMA
results in VGPRs) from the target.  CPU only (hipcc cross-compiles)."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _tool(name):
    path = shutil.which(name)
    if not path:
        pytest.skip(f"{name} not available")
    return path


def test_cmake_target_builds(tmp_path):
    cmake = _tool("cmake")
    if not os.path.exists("/opt/rocm/llvm/bin/clang++"):
        pytest.skip("ROCm compiler not available")
    consumer = tmp_path / "consumer"
    consumer.mkdir()
    (consumer / "CMakeLists.txt").write_text(
        "cmake_minimum_required(VERSION 3.21)\n"
        "project(consumer LANGUAGES CXX HIP)\n"
        f"add_subdirectory({ROOT} thunderfft_build)\n"
        "add_executable(consumer main.cpp)\n"
        "target_link_libraries(consumer PRIVATE thunderfft)\n"
        "add_library(consumer_kernels SHARED kernels.hip)\n"
        "target_link_libraries(consumer_kernels PRIVATE thunderfft)\n")
    # A fused kernel in the consumer's own translation unit (the device API's
    # templates are instantiated here, with the consumer's flags).
    (consumer / "kernels.hip").write_text(
        "#include <thunderfft/thunderfft.cuh>\n"
        "__global__ __launch_bounds__(256) void fused(const float2* in, float2* out,\n"
        "                                             const float2* tw) {\n"
        "  constexpr int N = 1024, BPB = thunderfft::batch_per_block<N>;\n"
        "  __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];\n"
        "  float2 reg[thunderfft::elements_per_thread];\n"
        "  thunderfft::ThunderFFT_gmem2reg<float, N, BPB>(reg, in + blockIdx.x * BPB * N);\n"
        "  thunderfft::ThunderFFT_kernel_reg<float, N, BPB, true>(reg, tw, work);\n"
        "  thunderfft::ThunderFFT_reg2gmem<float, N, BPB>(out + blockIdx.x * BPB * N, reg);\n"
        "}\n")
    (consumer / "main.cpp").write_text(
        "#include <thunderfft/thunderfft.hpp>\n"
        "int main() { thunderfft::ThunderFFT_global<float, 1024>(nullptr, nullptr, 0); return 0; }\n")
    build = tmp_path / "build"
    gen = ["-G", "Ninja"] if shutil.which("ninja") else []
    cfg = subprocess.run([cmake, "-S", str(consumer), "-B", str(build), *gen,
                          "-DCMAKE_PREFIX_PATH=/opt/rocm",
                          "-DCMAKE_HIP_COMPILER=/opt/rocm/llvm/bin/clang++",
                          "-DTHUNDERFFT_ARCH=gfx950", "-DCMAKE_EXPORT_COMPILE_COMMANDS=ON"],
                         capture_output=True, text=True, timeout=300)
    assert cfg.returncode == 0, cfg.stdout[-3000:] + cfg.stderr[-3000:]
    res = subprocess.run([cmake, "--build", str(build), "-j", "8", "--target", "consumer",
                          "consumer_kernels"], capture_output=True, text=True, timeout=900)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    commands = json.loads((build / "compile_commands.json").read_text())
    kernel_cmd = next(c["command"] for c in commands if c["file"].endswith("kernels.hip"))
    assert "-target-feature -Xclang -packed-fp32-ops" in kernel_cmd, kernel_cmd
    assert "-amdgpu-mfma-vgpr-form" in kernel_cmd, kernel_cmd
    host_cmd = next(c["command"] for c in commands if c["file"].endswith("main.cpp"))
    assert "packed-fp32-ops" not in host_cmd, host_cmd
    lib = next(p for p in build.rglob("libthunderfft_amd.so"))
    syms = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True,
                          text=True).stdout
    for s in ("thff_initialize", "thff_finalize", "thff_global", "thff_global_async",
              "thff_conv1d", "thff_conv2d", "thff_twiddle_info"):
        assert f" T {s}\n" in syms, s
    # the consumer runs its zero-batch call (no GPU needed: it returns before any HIP call)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    run = subprocess.run([str(build / "consumer")], capture_output=True, text=True, env=env,
                         timeout=60)
    assert run.returncode == 0, run.stderr
