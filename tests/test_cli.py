"""The command-line programs' argument handling on the CPU (no GPU needed):
thff_fft mirrors sample/fft1d/main.cu:170-193 (--help -> 0, invalid arguments
-> 1 with "FAIL: <reason>", both before any HIP call), thff_paper_fft mirrors sample/bench/paper_fft.cu:163-170 (usage -> 2, invalid
arguments -> 1, both before any HIP call) and thff_validate_cache mirrors
sample/validation/cache_validation.cu:160-168 (--help -> 0, anything else -> 2)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "thunderfft_amd", "_build")


def exe(name):
    path = os.path.join(BUILD, name)
    if not os.path.exists(path):
        from thunderfft_amd import build
        build.build_apps()
    return path


def run(*args):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    return subprocess.run(list(args), capture_output=True, text=True, env=env, timeout=120)


def test_paper_fft_usage_and_argument_errors():
    p = exe("thff_paper_fft")
    r = run(p)
    assert r.returncode == 2 and "usage:" in r.stderr
    assert run(p, "1", "2", "3", "4", "5", "6", "7").returncode == 2
    for args in (("1024", "bf16", "register"), ("1024", "fp16", "global"),
                 ("1024", "fp16", "register", "0"), ("1024", "tf32", "shared", "10", "0")):
        r = run(p, *args)
        assert r.returncode == 1 and "ERROR: invalid arguments" in r.stderr, args
    r = run(p, "100", "fp16", "register")
    assert r.returncode == 1 and "unsupported N" in r.stderr


def test_validate_cache_arguments():
    p = exe("thff_validate_cache")
    r = run(p, "--help")
    assert r.returncode == 0 and "No FFT" in r.stdout
    r = run(p, "--bogus")
    assert r.returncode == 2 and "accepts only --help" in r.stderr


def test_fft_quick_start_arguments():
    p = exe("thff_fft")
    for flag in ("--help", "-h"):
        r = run(p, flag)
        assert r.returncode == 0 and "[batch] [device]" in r.stdout and "5e-3" in r.stdout
    for args, why in ((("16", "0", "1"), "too many arguments"),
                      (("15",), "positive multiple of 16"), (("0",), "positive multiple of 16"),
                      (("-16",), "nonnegative integer"), (("16x",), "nonnegative integer"),
                      (("4294967296",), "nonnegative integer"), (("16", "dev"), "device must be")):
        r = run(p, *args)
        assert r.returncode == 1 and r.stderr.startswith("FAIL: ") and why in r.stderr, (args, r.stderr)
