"""Write the Bluestein golden vectors from the reference implementation (build container only).

trnfft's Bluestein path (trnfft/fft_core.py:1285-1376) computes its chirp angle in fp32, which
moves its result ~1e-4 (n=1000) / ~5e-4 (n=4099) away from the exact DFT; no closed form or
float64 check pins that behaviour, so these vectors are taken from the reference itself on the
pytorch backend.  Run from the repository root in a container where /root/reference holds the
reference checkout:

    python tests/golden/make_bluestein_vectors.py

Output: tests/golden/bluestein_vectors.npz with, per case, the seeded inputs and the
reference's fft and ifft outputs.  The GPU box never runs this script (the reference is not
there); tests only read the .npz.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bluestein_vectors.npz")

# (n, batch): the reference tests' arbitrary sizes (tests/conftest.py:21-23) plus the two
# BASELINE Bluestein lengths at small batch.
CASES = [(7, 3), (11, 2), (100, 3), (127, 2), (997, 2), (1000, 4), (4099, 2)]


def main() -> None:
    sys.path.insert(0, REF)
    import trnfft  # noqa: PLC0415  (the reference, read-only, pytorch backend on CPU)

    trnfft.set_backend("pytorch")
    trnfft.set_precision("fast")
    arrays: dict[str, np.ndarray] = {}
    for n, batch in CASES:
        g = torch.Generator().manual_seed(42)
        re = torch.randn(batch, n, generator=g)
        im = torch.randn(batch, n, generator=g)
        x = trnfft.ComplexTensor(re, im)
        fwd = trnfft.fft(x)
        inv = trnfft.ifft(x)
        arrays[f"n{n}_in_re"] = re.numpy()
        arrays[f"n{n}_in_im"] = im.numpy()
        arrays[f"n{n}_fft_re"] = fwd.real.numpy()
        arrays[f"n{n}_fft_im"] = fwd.imag.numpy()
        arrays[f"n{n}_ifft_re"] = inv.real.numpy()
        arrays[f"n{n}_ifft_im"] = inv.imag.numpy()
        print(f"n={n} batch={batch} done", flush=True)
    arrays["cases"] = np.array(CASES, dtype=np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
