"""Write tests/golden/c2c_numpy.npz: seeded inputs and fp64 spectra from an
implementation independent of this repository's oracle.

Inputs come from a pure-Python restatement of the counter-based U[-1,1)
generator (component c -> 2 * (splitmix64(seed ^ c) >> 40) * 2^-24 - 1),
spectra from numpy.fft (pocketfft) in complex128, unnormalized in both
directions (numpy's ifft scaled back by N).  The reference repository holds
no golden vectors of its own (its oracle is cuFFT run at test time), so these
fixtures pin the oracle and the GPU path against a third implementation.

    python tests/golden/make_golden.py
"""
import os

import numpy as np

MASK = (1 << 64) - 1
SEED_BASE = 0x7F4A7C15


def splitmix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & MASK
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
    return z ^ (z >> 31)


def uniform(n: int, batch: int, seed: int) -> np.ndarray:
    vals = [np.float32(2.0 * (splitmix64(seed ^ c) >> 40) / 16777216.0 - 1.0)
            for c in range(2 * n * batch)]
    return np.array(vals, dtype=np.float32).view(np.complex64).reshape(batch, n)


# (name, n, batch): the CPU-checkable case (N=64, batch 16) plus one signal of
# every other length.
CASES = [("n64_b16", 64, 16)] + [(f"n{n}_b1", n, 1) for n in (128, 256, 512, 1024, 2048, 4096)]


def main() -> None:
    out = {}
    for name, n, batch in CASES:
        x = uniform(n, batch, SEED_BASE + n)
        xd = x.astype(np.complex128)
        out[f"{name}_x"] = x
        out[f"{name}_fwd"] = np.fft.fft(xd, axis=-1)
        out[f"{name}_inv"] = np.fft.ifft(xd, axis=-1) * n
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c2c_numpy.npz")
    np.savez_compressed(path, **out)
    print(path, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
