"""The command-line programs on an MI355X: thff_fft (the reference's
sample/fft1d/main.cu quick start: N=64 float forward vs the vendor FFT, rel
L2 and rel Linf <= 5e-3), thff_paper_fft (the reference's
sample/bench/paper_fft.cu timing adapter: same CSV columns, single-FFT gate
<= 5e-3 vs an fp64 FFT, differential compute time) and thff_validate_cache
(sample/validation/cache_validation.cu: same stages and CSV columns)."""
import csv
import io
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "thunderfft_amd", "_build")
# paper_fft.cu:172
PAPER_COLUMNS = ("N,precision,placement,batch,inside_repeats,trial,t_R_us,t_2R_us,compute_us,"
                 "e2e_out_of_place_us,single_fft_relL2,shared_bytes")
# cache_validation.cu:115-148, one visible device
STAGES = ["initialize", "same_length_cache_hit", "replace_length", "finalize",
          "repeated_finalize", "reinitialize_after_finalize", "final_cleanup",
          "cross_device_initialize", "return_to_device", "cross_device_cleanup"]


def exe(name):
    path = os.path.join(BUILD, name)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run __graft_entry__.build()")
    return path


@pytest.mark.parametrize("batch", [None, 4096])
def test_fft_quick_start_passes(batch):
    args = [exe("thff_fft")] + ([] if batch is None else [str(batch), "0"])
    print(" ".join(args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[0] == (f"ThunderFFT vs hipFFT: float2, N=64, forward (unscaled), "
                        f"batch={batch or 16}, device=0")
    l2 = float(lines[1].split(":")[1])
    linf = float(lines[2].split(":")[1])
    assert lines[3].startswith("Tolerance:     5.000000e-03") and lines[4] == "PASS"
    # both sides compute in fp32, so they agree to a few ulps
    assert l2 <= 1e-6 and linf <= 1e-6
    print(r.stdout, flush=True)


# Each case moves 2^22 values and repeats the transform 50 times, so that the
# 2R launch is reliably longer than the R launch (the program's own check).
@pytest.mark.parametrize("n,precision,placement", [
    (1024, "fp16", "register"), (1024, "tf32", "shared"), (64, "fp16", "shared"),
    (128, "fp32", "register"), (4096, "tf32", "register"), (2048, "fp16", "shared")])
def test_paper_fft_csv_and_gate(n, precision, placement):
    repeats, batch = 50, (1 << 22) // n
    print(f"thff_paper_fft {n} {precision} {placement} {repeats} 2 {batch}", flush=True)
    r = subprocess.run([exe("thff_paper_fft"), str(n), precision, placement, str(repeats), "2",
                        str(batch)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[0] == PAPER_COLUMNS
    rows = list(csv.DictReader(io.StringIO(r.stdout)))
    assert len(rows) == 2
    for row in rows:
        assert int(row["N"]) == n and row["precision"] == precision
        assert row["placement"] == placement and int(row["batch"]) == batch
        assert float(row["t_2R_us"]) > float(row["t_R_us"]) > 0
        assert float(row["compute_us"]) > 0 and float(row["e2e_out_of_place_us"]) > 0
        assert float(row["single_fft_relL2"]) <= (1e-3 if precision == "fp16" else 2e-6)
        assert int(row["shared_bytes"]) == 8 * (n + n // 16) * (4096 // n)
    print(r.stdout, flush=True)


def test_paper_fft_rejects_non_block_multiple_batch():
    r = subprocess.run([exe("thff_paper_fft"), "64", "fp16", "register", "10", "1", "100"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "positive BPB multiple" in r.stderr


def test_validate_cache_lifecycle():
    r = subprocess.run([exe("thff_validate_cache")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rows = list(csv.DictReader(io.StringIO(r.stdout)))
    assert r.stdout.splitlines()[0] == "precision,device,stage,N,pointer,pass"
    for precision in ("fp32", "fp16"):
        mine = [x for x in rows if x["precision"] == precision]
        assert [x["stage"] for x in mine] == STAGES
        assert all(x["pass"] == "1" for x in mine)
        n = {x["stage"]: int(x["N"]) for x in mine}
        assert n["initialize"] == 64 and n["replace_length"] == 128 and n["finalize"] == 0
        ptr = {x["stage"]: x["pointer"] for x in mine}
        assert ptr["initialize"] == ptr["same_length_cache_hit"]
    assert "checks passed" in r.stderr
