"""CPU oracle for the trnfft_amd parity tests — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with torch fp32 arithmetic in the same operation order, the
reference's pytorch-backend path for the FFT hot path (trnsci/trnfft, files cited per function
in ``reference_path``).  It is the checker, never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
  import it;
* the product package ``trnfft_amd`` never imports it and has no CPU fallback of its own.

Pinning (what makes the oracle trustworthy), all exercised by ``tests/test_oracle.py``:

* power-of-two c2c (``cooley_tukey``): float64 DFT, the reference tests' known-answer vectors
  (impulse, constant, single tone, zero padding), round trip, Parseval, linearity and brute-force
  DFT for n <= 64; the vectorised form is bit-identical to the literal per-k loop
  (``cooley_tukey_loop``), which is checked on small sizes;
* Bluestein (``bluestein``): the reference's own outputs written by
  ``tests/golden/make_bluestein_vectors.py`` (imported from the reference in the build
  container), plus the fp64 DFT within the fp32-chirp error band;
* rfft/irfft/fftn/stft/istft: numpy.fft and torch.stft / round trips;
* complex_linear: float64 ``torch.nn.functional.linear`` on the same weights;
* dft_gemm: float64 DFT.
"""

from .reference_path import *  # noqa: F401,F403
