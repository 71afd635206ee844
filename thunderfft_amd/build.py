"""Build libthunderfft_amd.so in-tree with hipcc for gfx950.

    python -m thunderfft_amd.build [--jobs J] [--verbose]

Every kernel translation unit is compiled for gfx950 only, with packed FP32
instructions disabled (-Xclang -target-feature -Xclang -packed-fp32-ops) and
MFMA results kept in VGPRs (-mllvm -amdgpu-mfma-vgpr-form).  The
per-length kernel file is compiled once per transform length so the lengths
build in parallel.  Objects go to thunderfft_amd/_build/, the shared library
to thunderfft_amd/libthunderfft_amd.so (loaded by thunderfft_amd/__init__.py).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libthunderfft_amd.so")
LENGTHS = (64, 128, 256, 512, 1024, 2048, 4096)
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build thunderfft_amd)")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in ordinary VGPRs (no AGPR round trip through v_accvgpr_read)
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    ]


def units() -> list[tuple[str, str, list[str]]]:
    """(source, object, extra flags) for every translation unit."""
    out = []
    for n in LENGTHS:
        out.append((os.path.join(CSRC, "c2c_instance.hip"), os.path.join(BUILD, f"c2c_n{n}.o"),
                    [f"-DTHFF_N={n}"]))
    out.append((os.path.join(CSRC, "fill.hip"), os.path.join(BUILD, "fill.o"), []))
    out.append((os.path.join(CSRC, "capi.cpp"), os.path.join(BUILD, "capi.o"), ["-x", "hip"]))
    return out


def _compile(cc: str, src: str, obj: str, extra: list[str], verbose: bool) -> None:
    cmd = [cc, *common_flags(), *extra, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # The host pass does not know the packed-fp32 feature name; that warning is expected.
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln
             and "not a recognized feature" not in ln]
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_compile, cc, s, o, e, verbose) for s, o, e in units()]
        for f in futs:
            f.result()
    objs = [o for _, o, _ in units()]
    tmp = LIB + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


APPS = ("thff_fft", "thff_validate", "thff_paper_fft", "thff_validate_cache")
# Shared libraries of kernels written against the public device API (tests use them).
DEVICE_EXAMPLES = ("device_example", "bench_compute")


def build_apps(verbose: bool = False) -> list[str]:
    """Host programs over the C++ API, linked to the in-tree library."""
    cc = hipcc()
    out = []
    for app in APPS:
        exe = os.path.join(BUILD, app)
        cmd = [cc, *common_flags(), os.path.join(PKG, "apps", app + ".hip"), "-o", exe,
               "-L", PKG, "-lthunderfft_amd", "-lhipfft", "-Wl,-rpath,$ORIGIN/.."]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"app build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
        out.append(exe)
    for ex in DEVICE_EXAMPLES:
        so = os.path.join(BUILD, f"libthff_{ex}.so")
        cmd = [cc, *common_flags(), "-shared", os.path.join(PKG, "apps", ex + ".hip"), "-o", so,
               "-L", PKG, "-lthunderfft_amd", "-Wl,-rpath,$ORIGIN/.."]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"example build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
        out.append(so)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
    for exe in build_apps(a.verbose):
        print(exe)


if __name__ == "__main__":
    main()
