"""Stream semantics of the C ABI on an MI355X: the asynchronous entry points
enqueue on the caller's stream (equal, bit for bit, to the synchronous calls),
the synchronous ones return only once their stream has finished (the
reference synchronises `stream` before returning, thunderfft_impl_kernel.cuh:
36-40), and work on two streams at once (different types and lengths) stays
correct.  Streams are created at the default priority."""
import numpy as np
import pytest

import oracle
from thff_testlib import TIGHT, from_device, to_device

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("T,n", [("float", 1024), ("half", 1024), ("half", 4096), ("float", 64)])
def test_async_on_stream_equals_sync(T, n):
    import torch

    import thunderfft_amd as thff

    batch = 4096 * 16 // n + 3
    thff.ThunderFFTInitialize(T, n)
    x = to_device(oracle.uniform(n, batch, seed=n + 5), T)
    ref = torch.empty_like(x)
    thff.ThunderFFT_global(T, n, True, x, ref, batch)  # default stream, synchronous
    s = torch.cuda.Stream()
    y = torch.full_like(x, float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        thff.ThunderFFT_global_async(T, n, True, x, y, batch, s)
    s.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_sync_call_waits_for_its_stream():
    """A long transform on a side stream: right after the synchronous call
    returns, the output is complete without any further synchronisation."""
    import torch

    import thunderfft_amd as thff

    n, batch = 1024, 65536
    thff.ThunderFFTInitialize("float", n)
    x = torch.empty(2 * n * batch, dtype=torch.float32, device="cuda")
    thff.fill_uniform("float", x, n * batch, 77, 0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    y = torch.full_like(x, float("nan"))
    torch.cuda.synchronize()
    thff.ThunderFFT_global("float", n, True, x, y, batch, s)
    # read on the default stream with no synchronisation against s: correct
    # only if the call waited for s (the last signals are written last)
    sample = from_device(y[-2 * n * 8:], "float").reshape(8, n)
    xs = from_device(x[-2 * n * 8:], "float").reshape(8, n)
    m = oracle.metrics(sample, oracle.fft(xs, True))
    assert m["nonfinite"] == 0 and m["rel_l2"] <= TIGHT["float"]
    sample = from_device(y[: 2 * n * 8], "float").reshape(8, n)
    xs = from_device(x[: 2 * n * 8], "float").reshape(8, n)
    m = oracle.metrics(sample, oracle.fft(xs, True))
    assert m["nonfinite"] == 0 and m["rel_l2"] <= TIGHT["float"]


def test_two_streams_at_once():
    """float N=1024 on one stream and half N=256 on another, interleaved
    launches, both against the oracle."""
    import torch

    import thunderfft_amd as thff

    thff.ThunderFFTInitialize("float", 1024)
    thff.ThunderFFTInitialize("half", 256)
    xf = oracle.uniform(1024, 300, seed=1)
    xh = oracle.represent(oracle.uniform(256, 1200, seed=2), "half")
    d_xf, d_xh = to_device(xf, "float"), to_device(xh, "half")
    d_yf, d_yh = torch.empty_like(d_xf), torch.empty_like(d_xh)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(5):
        thff.ThunderFFT_global_async("float", 1024, True, d_xf, d_yf, 300, s1)
        thff.ThunderFFT_global_async("half", 256, False, d_xh, d_yh, 1200, s2)
    s1.synchronize()
    s2.synchronize()
    mf = oracle.metrics(from_device(d_yf, "float").reshape(300, 1024), oracle.fft(xf, True))
    mh = oracle.metrics(from_device(d_yh, "half").reshape(1200, 256), oracle.fft(xh, False))
    assert mf["rel_l2"] <= TIGHT["float"] and mh["rel_l2"] <= TIGHT["half"], (mf, mh)


def test_conv_async_on_stream():
    import torch

    import thunderfft_amd as thff

    n, batch = 1024, 37
    thff.ThunderFFTInitialize("half", n)
    rng = np.random.default_rng(3)
    x = oracle.represent(oracle.uniform(n, batch, seed=9), "half")
    h = oracle.represent((rng.normal(size=(batch, n)) + 1j * rng.normal(size=(batch, n)))
                         .astype(np.complex64) / np.sqrt(n), "half")
    d_x, d_h = to_device(x, "half"), to_device(h, "half")
    ref = torch.empty_like(d_x)
    thff.ThunderFFT_conv1d("half", n, d_x, d_h, ref, batch)
    s = torch.cuda.Stream()
    y = torch.full_like(d_x, float("nan"))
    torch.cuda.synchronize()
    thff.ThunderFFT_conv1d_async("half", n, d_x, d_h, y, batch, True, s)
    s.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_initialize_races_transforms_on_another_thread():
    """The transform path takes no lock (it reads the registry with atomic
    loads) and Initialize keeps a replaced table allocated: while one host
    thread switches the current float length between 1024 and 512, another
    runs N=1024 transforms on its own stream.  Each call either returns the
    bit-exact result of an undisturbed call or fails with the documented
    missing-table error; none crashes or reads a freed table."""
    import threading
    import time

    import torch

    import thunderfft_amd as thff

    n, batch, calls = 1024, 64, 150
    thff.ThunderFFTInitialize("float", n)
    x = oracle.uniform(n, batch, seed=11)
    d_x = to_device(x, "float")
    d_ref = torch.empty_like(d_x)
    thff.ThunderFFT_global("float", n, True, d_x, d_ref, batch)
    ref = from_device(d_ref, "float")
    m = oracle.metrics(ref.reshape(batch, n), oracle.fft(x, True))
    assert m["rel_l2"] <= TIGHT["float"], m

    stream = torch.cuda.Stream()
    outcome = {"ok": 0, "missing": 0, "mismatch": 0, "other": [], "switches": 0}
    start = threading.Barrier(2, timeout=60)
    done = threading.Event()
    errors = []  # exceptions raised in the worker threads, re-raised below

    def transforms():
        try:
            d_y = torch.empty_like(d_x)
            start.wait()
            for _ in range(calls):
                d_y.fill_(float("nan"))
                torch.cuda.synchronize()
                try:
                    thff.ThunderFFT_global("float", n, True, d_x, d_y, batch, stream)
                except RuntimeError as e:
                    if "ThunderFFTInitialize" in str(e):
                        outcome["missing"] += 1
                    else:
                        outcome["other"].append(str(e))
                    continue
                if torch.equal(d_y, d_ref):
                    outcome["ok"] += 1
                else:
                    outcome["mismatch"] += 1
        except BaseException as e:  # noqa: BLE001 - reported in the main thread
            errors.append(e)
        finally:
            done.set()  # the toggling thread stops whatever happened here

    def switches():
        deadline = time.monotonic() + 90  # bounded even if `done` were never set
        try:
            start.wait()
            while not done.is_set() and time.monotonic() < deadline:
                thff.ThunderFFTInitialize("float", 512)
                thff.ThunderFFTInitialize("float", n)
                outcome["switches"] += 1
        except BaseException as e:  # noqa: BLE001
            errors.append(e)
            done.set()

    workers = [threading.Thread(target=transforms), threading.Thread(target=switches)]
    for w in workers:
        w.start()
    for w in workers:
        w.join(timeout=120)
    assert not any(w.is_alive() for w in workers), "a worker thread did not finish"
    if errors:
        raise errors[0]
    print(f"initialize race: {outcome}", flush=True)
    assert outcome["mismatch"] == 0 and not outcome["other"], outcome
    assert outcome["ok"] + outcome["missing"] == calls, outcome
    # the replaced tables stayed allocated: N=1024 is still served afterwards
    thff.ThunderFFTInitialize("float", n)
    d_y = torch.empty_like(d_x)
    thff.ThunderFFT_global("float", n, True, d_x, d_y, batch)
    assert torch.equal(d_y, d_ref)
