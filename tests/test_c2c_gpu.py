"""GPU parity of ThunderFFT_global against the fp64 oracle, through the C ABI.

Restates the reference's correctness matrix (sample/validation/
fft_validation.cu:194-311): every size x {float, half} x {forward, inverse}
x the four input kinds, full batch 64 and public tail batches {1, BPB-1,
BPB+1} (BPB = transforms per workgroup here), NaN-prefilled outputs with 16
trailing sentinels that must survive, inputs allocated exactly batch*N long,
reference = fp64 transform of the values the storage type represents.
Pass = finite, relative L2 <= 5e-3 (the reference's gate) and within this
build's tighter fp32-arithmetic bar (TIGHT).  The full-size configurations
are checked on a subset of signals against the oracle and over every signal
through the unnormalized round trip inverse(forward(x)) = N*x.
"""
import os

import numpy as np
import pytest

import oracle
from thff_testlib import GATE, SIZES, TIGHT, from_device, run_case, to_device

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c2c_numpy.npz")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch

    import thunderfft_amd as thff

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    thff.lib()
    yield
    thff.ThunderFFTFinalize("float")
    thff.ThunderFFTFinalize("half")


def _tails(n):
    import thunderfft_amd as thff

    bpb = thff.transforms_per_block(n)
    return sorted({b for b in (1, bpb - 1, bpb + 1) if b > 0 and b != 64})


def _check(m, T, label):
    print(f"{label}: rel_l2={m['rel_l2']:.3e} rel_linf={m['rel_linf']:.3e} "
          f"guards={m['guards_changed']}", flush=True)
    assert m["nonfinite"] == 0, label
    assert m["guards_changed"] == 0, label
    assert m["rel_l2"] <= GATE, label
    assert m["rel_l2"] <= TIGHT[T], label


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_validation_matrix(T, n):
    for kind in range(4):
        for forward in (True, False):
            for batch in [64] + _tails(n):
                x = oracle.make_input(n, batch, kind)
                m = run_case(T, n, forward, x)
                _check(m, T, f"{T} N={n} {'fwd' if forward else 'inv'} "
                             f"{oracle.INPUT_KINDS[kind]} batch={batch}")


@pytest.mark.parametrize("T", ["float", "half"])
def test_golden_fixtures(T):
    """The CPU-checkable case (N=64, batch 16, float forward) and one signal of
    every other length against numpy.fft spectra of the fixture inputs."""
    g = np.load(GOLDEN)
    for key in g.files:
        if not key.endswith("_x"):
            continue
        x = g[key]
        n = x.shape[-1]
        for forward, tag in ((True, "fwd"), (False, "inv")):
            m = run_case(T, n, forward, x)
            if T == "float":
                # float storage represents the fixture input exactly
                m2 = oracle.metrics(m["out"], g[key[:-2] + "_" + tag])
                assert m2["rel_l2"] <= TIGHT[T], key
                assert m2["rel_linf"] <= 10 * TIGHT[T], key
            _check(m, T, f"golden {key} {tag}")


def test_reinitialize_after_finalize():
    """fft_validation.cu:302-310: finalize, re-initialize at 64, transform again."""
    import thunderfft_amd as thff

    for T in ("float", "half"):
        thff.ThunderFFTInitialize(T, 4096)
        thff.ThunderFFTFinalize(T)
        thff.ThunderFFTInitialize(T, 64)
        for forward in (True, False):
            m = run_case(T, 64, forward, oracle.make_input(64, 1, 0))
            _check(m, T, f"reinit {T} {forward}")


def test_uninitialized_length_raises():
    import torch

    import thunderfft_amd as thff

    thff.ThunderFFTInitialize("float", 64)
    x = torch.zeros(2 * 128, device="cuda")
    y = torch.zeros(2 * 128, device="cuda")
    with pytest.raises(RuntimeError, match=r"\[ThunderFFT\].*ThunderFFTInitialize<float>\(128\)"):
        thff.ThunderFFT_global("float", 128, True, x, y, 1)


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_element_aligned_buffers(T, n):
    """Buffers that start on an odd element, not on a 16-byte boundary: the
    reference takes any vec2_t<T> buffer (thunderfft_impl_kernel.cuh:18-21),
    so these run the direct-movement kernel.  Input and/or output offset by 1
    or 3 elements, a partial last tile; the elements around the output must
    stay untouched."""
    import thunderfft_amd as thff

    esize = 8 if T == "float" else 4
    batch = 2 * thff.transforms_per_block(n) + 3
    count = batch * n
    xr = oracle.represent(oracle.make_input(n, batch, 0), T)
    thff.ThunderFFTInitialize(T, n)
    for in_off, out_off in ((1, 3), (0, 1), (3, 0)):
        host_in = np.zeros(count + in_off, np.complex64)
        host_in[in_off:] = xr.reshape(-1)
        d_in = to_device(host_in, T)
        guard = np.complex64(-271.0 + 137.0j)
        host_out = np.full(count + out_off + 16, guard, np.complex64)
        host_out[out_off:out_off + count] = np.nan
        d_out = to_device(host_out, T)
        for forward in (True, False):
            thff.ThunderFFT_global(T, n, forward, d_in.data_ptr() + in_off * esize,
                                   d_out.data_ptr() + out_off * esize, batch)
            out = from_device(d_out, T)
            m = oracle.metrics(out[out_off:out_off + count], oracle.fft(xr, forward).reshape(-1))
            label = f"{T} N={n} offsets in={in_off} out={out_off} {'fwd' if forward else 'inv'}"
            print(f"{label}: rel_l2={m['rel_l2']:.3e}", flush=True)
            assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T], label
            around = np.concatenate([out[:out_off], out[out_off + count:]])
            assert np.all(around == guard), label


@pytest.mark.parametrize("T", ["float", "half"])
def test_fft_convenience(T):
    """thunderfft_amd.fft: complex64 / float16[..., N, 2] tensors, with and
    without a caller's out, against the oracle; the length that was current
    for T before the call is current again afterwards."""
    import torch

    import thunderfft_amd as thff

    thff.ThunderFFTInitialize(T, 256)
    for n in (64, 1024):
        xr = oracle.represent(oracle.make_input(n, 5, 2), T)
        if T == "float":
            x = torch.from_numpy(xr).cuda()
        else:
            x = to_device(xr, T).view(5, n, 2)
        for forward in (True, False):
            y = thff.fft(x, forward=forward)
            out = torch.empty_like(x)
            y2 = thff.fft(x, forward=forward, out=out)
            assert y2 is out
            torch.cuda.synchronize()
            for got in (y, y2):
                host = got.cpu().numpy() if T == "float" else from_device(got.reshape(-1), T)
                m = oracle.metrics(host.reshape(-1), oracle.fft(xr, forward).reshape(-1))
                assert m["nonfinite"] == 0 and m["rel_l2"] <= TIGHT[T], (n, forward)
        assert thff.twiddle_info(T)[1] == 256


def test_twiddle_cache_lifecycle():
    """sample/validation/cache_validation.cu:65-121 on the current device."""
    import torch

    import thunderfft_amd as thff

    for T in ("float", "half"):
        thff.ThunderFFTFinalize(T)
        assert thff.twiddle_info(T) == (0, 0)
        thff.ThunderFFTInitialize(T, 64)
        p64, n = thff.twiddle_info(T)
        assert p64 != 0 and n == 64
        thff.ThunderFFTInitialize(T, 64)
        assert thff.twiddle_info(T) == (p64, 64), "same-length init must keep the allocation"
        thff.ThunderFFTInitialize(T, 128)
        p128, n = thff.twiddle_info(T)
        assert n == 128 and p128 != 0
        # read W[0], W[1] back through a device-to-device copy into a torch tensor
        buf = torch.empty(4, dtype=torch.float32, device="cuda")
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        assert hip.hipMemcpy(buf.data_ptr(), p128, 16, 3) == 0  # hipMemcpyDeviceToDevice
        w = buf.cpu().numpy()
        assert w[0] == 1.0 and w[1] == 0.0, "W[0] must be 1+0i"
        assert abs(w[2] - np.cos(2 * np.pi / 128)) <= 1e-6
        assert abs(w[3] - np.sin(2 * np.pi / 128)) <= 1e-6
        thff.ThunderFFTFinalize(T)
        assert thff.twiddle_info(T) == (0, 0)
        thff.ThunderFFTFinalize(T)  # repeated finalize is fine
        assert thff.twiddle_info(T) == (0, 0)
        thff.ThunderFFTInitialize(T, 64)
        assert thff.twiddle_info(T)[1] == 64
        thff.ThunderFFTFinalize(T)


@pytest.mark.parametrize("T", ["float", "half"])
def test_device_generator_matches_oracle(T):
    import torch

    import thunderfft_amd as thff

    n, batch, first = 1024, 7, 12345
    d = torch.empty(n * batch * (2 if T == "float" else 2), device="cuda",
                    dtype=torch.float32 if T == "float" else torch.float16)
    thff.fill_uniform(T, d, n * batch, oracle.BENCH_SEED_BASE + n, first)
    torch.cuda.synchronize()
    got = from_device(d, T).reshape(batch, n)
    want = oracle.represent(oracle.uniform(n, batch, first_element=first), T)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _subset_rows(batch, k=256):
    rows = np.unique(np.concatenate([np.linspace(0, batch - 1, k).astype(np.int64),
                                     np.arange(max(0, batch - 5), batch)]))
    return rows


def _large_case(T, n, batch, directions=(True, False)):
    """Full-size case: device-generated seeded input, oracle check on a subset of
    signals, round trip over every signal."""
    import torch

    import thunderfft_amd as thff

    dt = torch.float32 if T == "float" else torch.float16
    count = n * batch
    seed = oracle.BENCH_SEED_BASE + n
    x = torch.empty(2 * count, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, count, seed)
    y = torch.empty_like(x)
    z = torch.empty_like(x)
    thff.ThunderFFTInitialize(T, n)
    rows = _subset_rows(batch)
    rows_t = torch.from_numpy(rows).cuda()
    for forward in directions:
        thff.ThunderFFT_global(T, n, forward, x, y, batch)
        sub = from_device(y.view(batch, 2 * n).index_select(0, rows_t).contiguous(), T)
        sub = sub.reshape(len(rows), n)
        xin = np.concatenate([oracle.uniform(n, 1, seed, first_element=int(r) * n) for r in rows])
        ref = oracle.fft(oracle.represent(xin, T), forward)
        m = oracle.metrics(sub, ref)
        print(f"{T} N={n} batch={batch} {'fwd' if forward else 'inv'} subset rel_l2="
              f"{m['rel_l2']:.3e}", flush=True)
        assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]
        # round trip: inverse of the other direction gives N*x (unnormalized)
        thff.ThunderFFT_global(T, n, not forward, y, z, batch)
        xf = x.float()
        err = torch.linalg.vector_norm(z.float() - n * xf) / torch.linalg.vector_norm(n * xf)
        rt = float(err)
        print(f"  round trip rel_l2={rt:.3e}", flush=True)
        assert np.isfinite(rt) and rt <= GATE and rt <= 2 * TIGHT[T]
    del x, y, z
    torch.cuda.empty_cache()


@pytest.mark.parametrize("batch", [65536, 65537])
def test_config2_n1024_float(batch):
    """The headline workload: N=1024, batch 65536 (and 65537: masked partial block)."""
    _large_case("float", 1024, batch)


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_config3_sweep(T, n):
    """The size sweep: batch = 2^26 / N, so 2^26 complex values per buffer at every N."""
    _large_case(T, n, (1 << 26) // n)


@pytest.mark.parametrize("T", ["float", "half"])
@pytest.mark.parametrize("n", SIZES)
def test_grid_stride_walks(T, n):
    """Batches of 514 full tiles and one partial tile: the kernels on
    device-sized grids (2 workgroups per CU or more) hand some workgroups a
    second tile a grid apart, and the partial tile is masked.  Forward only,
    oracle on a subset of signals (first, last, spread) and the round trip."""
    tile = 4096 // n  # transforms per 4096-value tile (every kernel)
    _large_case(T, n, 514 * tile + max(1, tile // 2), directions=(True,))


@pytest.mark.parametrize("T,n", [("float", 1024), ("half", 1024), ("half", 4096), ("float", 4096),
                                 ("half", 128), ("half", 2048)])
def test_beyond_2e31_values(T, n):
    """One launch over 2^31 + 5 * 4096 complex values (17 GB per fp32 buffer,
    8.6 GB per fp16 buffer, on a 288 GB device): every signal offset past
    2^31 values needs 64-bit index arithmetic.  Forward, the first signals,
    the last ones and a spread between them against the oracle; then the
    inverse of those signals back to N * x."""
    import torch

    import thunderfft_amd as thff

    batch = (1 << 31) // n + 5 * 4096 // n
    count = n * batch
    dt = torch.float32 if T == "float" else torch.float16
    seed = oracle.BENCH_SEED_BASE + n + 31
    x = torch.empty(2 * count, dtype=dt, device="cuda")
    thff.fill_uniform(T, x, count, seed)
    y = torch.empty_like(x)
    thff.ThunderFFTInitialize(T, n)
    thff.ThunderFFT_global(T, n, True, x, y, batch)
    rows = np.unique(np.concatenate([np.arange(3), np.linspace(0, batch - 1, 24).astype(np.int64),
                                     np.arange((1 << 31) // n - 2, batch)]))
    rows_t = torch.from_numpy(rows).cuda()
    sub = y.view(batch, 2 * n).index_select(0, rows_t).contiguous()
    got = from_device(sub, T).reshape(len(rows), n)
    xin = oracle.represent(np.concatenate([oracle.uniform(n, 1, seed, first_element=int(r) * n)
                                           for r in rows]), T)
    m = oracle.metrics(got, oracle.fft(xin, True))
    print(f"{T} N={n} batch={batch} ({count} values) rows past 2^31: rel_l2={m['rel_l2']:.3e}",
          flush=True)
    assert m["nonfinite"] == 0 and m["rel_l2"] <= GATE and m["rel_l2"] <= TIGHT[T]
    del x, y
    back = torch.empty_like(sub)
    thff.ThunderFFT_global(T, n, False, sub, back, len(rows))
    rt = oracle.metrics(from_device(back, T).reshape(len(rows), n), n * xin.astype(np.complex128))
    print(f"  round trip of the sampled signals rel_l2={rt['rel_l2']:.3e}", flush=True)
    assert rt["nonfinite"] == 0 and rt["rel_l2"] <= 2 * TIGHT[T]
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", ["quick", "full"])
def test_thff_validate_matrix(mode, tmp_path):
    """The thff_validate program (the reference's sample/validation/
    fft_validation.cu matrix): direct (device API) and public paths, every
    length, both precisions and directions, the four input kinds and tail
    batches, against hipFFT Z2Z fp64; exit status 0 and every CSV row passes."""
    import csv
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "thunderfft_amd", "_build", "thff_validate")
    out = tmp_path / "validate.csv"
    args = [exe, "--csv", str(out)] + (["--quick"] if mode == "quick" else [])
    res = subprocess.run(args, capture_output=True, text=True, timeout=600)
    print(res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stderr[-2000:]
    rows = list(csv.DictReader(open(out)))
    assert len(rows) == (88 if mode == "quick" else 532)
    assert all(r["pass"] == "1" for r in rows)
    worst = {}
    for r in rows:
        k = r["precision"]
        worst[k] = max(worst.get(k, 0.0), float(r["relative_l2"]))
    print("worst relative L2 per precision:", worst, flush=True)
    assert worst["fp32"] <= TIGHT["float"] and worst["fp16"] <= TIGHT["half"]


def test_copy_nt_copies_every_byte():
    """thff_copy_nt (the bandwidth reference bench.py reports) moves exactly the
    requested bytes: whole 8 KiB blocks plus a tail, nothing past the end."""
    import torch

    import thunderfft_amd as thff

    for nbytes in (16, 8192, 16 * (512 * 37 + 13)):
        src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4 + 8,), dtype=torch.int32, device="cuda")
        dst = torch.full_like(src, 0x5A5A5A5A)
        thff.copy_nt(dst, src, nbytes)
        torch.cuda.synchronize()
        k = nbytes // 4
        assert torch.equal(dst[:k], src[:k]), nbytes
        assert bool((dst[k:] == 0x5A5A5A5A).all()), nbytes
