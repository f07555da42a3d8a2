"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

Each check is chosen so that a plausible slip in the restatement (dropped term, wrong sign,
wrong index, wrong scaling) fails: reference-produced golden vectors, literal-loop equality,
float64 DFT, the reference tests' known-answer vectors, and invariants.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_l2, seeded_complex

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bluestein_vectors.npz")


def _dft64(re, im, inverse=False):
    x = re.double().numpy() + 1j * im.double().numpy()
    return np.fft.ifft(x, axis=-1) if inverse else np.fft.fft(x, axis=-1)


# --- golden vectors written by the reference itself ------------------------------------------


@pytest.mark.parametrize("direction", ["fft", "ifft"])
def test_bluestein_bitexact_vs_reference_vectors(direction):
    d = np.load(GOLDEN)
    for n, _batch in d["cases"]:
        re = torch.from_numpy(d[f"n{n}_in_re"])
        im = torch.from_numpy(d[f"n{n}_in_im"])
        r, i = oracle.fft_core(re, im, direction == "ifft")
        np.testing.assert_array_equal(r.numpy(), d[f"n{n}_{direction}_re"])
        np.testing.assert_array_equal(i.numpy(), d[f"n{n}_{direction}_im"])


def test_golden_vectors_show_fp32_chirp_deviation():
    # the reference's fp32 chirp angle puts n=1000 / n=4099 at ~1.2e-4 / ~4.6e-4 from exact:
    # the vectors carry that quirk, an accurate Bluestein would not match them
    d = np.load(GOLDEN)
    for n, lo, hi in [(1000, 5e-5, 5e-4), (4099, 2e-4, 2e-3), (7, 0, 5e-6)]:
        x = d[f"n{n}_in_re"].astype(np.float64) + 1j * d[f"n{n}_in_im"]
        ref = d[f"n{n}_fft_re"] + 1j * d[f"n{n}_fft_im"]
        err = np.linalg.norm(ref - np.fft.fft(x)) / np.linalg.norm(np.fft.fft(x))
        assert lo <= err <= hi, (n, err)


# --- radix-2 (trnfft/fft_core.py:53-117) -----------------------------------------------------


@pytest.mark.parametrize("n", [2, 4, 8, 32, 128, 512])
@pytest.mark.parametrize("inverse", [False, True])
def test_vectorised_equals_literal_loop(n, inverse):
    re, im = seeded_complex(3, n, seed=n)
    a = oracle.cooley_tukey(re, im, inverse)
    b = oracle.cooley_tukey_loop(re.clone(), im.clone(), inverse)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("n", [8, 64, 1024])
def test_bit_reverse_matches_loop(n):
    bits = int(math.log2(n))
    assert torch.equal(oracle.bit_reverse_indices(n, bits), oracle.bit_reverse_indices_loop(n, bits))


@pytest.mark.parametrize("n", [8, 16, 64, 256, 1024, 4096, 1 << 16])
@pytest.mark.parametrize("inverse", [False, True])
def test_cooley_tukey_vs_float64_dft(n, inverse):
    re, im = seeded_complex(2, n)
    r, i = oracle.cooley_tukey(re, im, inverse)
    ref = _dft64(re, im, inverse)
    assert rel_l2(r, i, ref.real, ref.imag) < 1e-6 * math.log2(n)


def test_brute_force_dft_small():
    for n in [2, 4, 8, 16, 32, 64]:
        re, im = seeded_complex(1, n, seed=7)
        x = re.double() + 1j * im.double()
        k = torch.arange(n, dtype=torch.float64)
        w = torch.exp(-2j * math.pi * torch.outer(k, k) / n)
        ref = (x @ w).numpy()
        r, i = oracle.cooley_tukey(re, im, False)
        assert rel_l2(r, i, ref.real, ref.imag) < 1e-6 * max(1, math.log2(n))


def test_known_answers():
    # impulse -> ones, constant -> n*delta, tone -> bins k and n-k (reference tests/test_fft.py:12-35)
    n = 16
    x = torch.zeros(n)
    x[0] = 1.0
    r, i = oracle.fft(x)
    np.testing.assert_allclose(r.numpy(), np.ones(n), atol=1e-6)
    np.testing.assert_allclose(i.numpy(), np.zeros(n), atol=1e-6)
    r, i = oracle.fft(torch.ones(n))
    assert abs(r[0].item() - n) < 1e-5 and torch.sqrt(r[1:] ** 2 + i[1:] ** 2).max() < 1e-5
    n, k = 64, 5
    t = torch.arange(n, dtype=torch.float32)
    r, i = oracle.fft(torch.cos(2 * np.pi * k * t / n))
    mags = torch.sqrt(r**2 + i**2)
    assert mags[k] > n / 2 - 1 and mags[n - k] > n / 2 - 1
    # zero padding (tests/test_fft.py:64-69)
    r, i = oracle.fft(torch.tensor([1.0, 2.0, 3.0, 4.0]), n=8)
    e = np.fft.fft([1, 2, 3, 4, 0, 0, 0, 0])
    np.testing.assert_allclose(r.numpy(), e.real, atol=1e-5)
    np.testing.assert_allclose(i.numpy(), e.imag, atol=1e-5)


def test_invariants_roundtrip_parseval_linearity():
    n = 1024
    re, im = seeded_complex(4, n)
    r, i = oracle.fft((re, im))
    rr, ii = oracle.ifft((r, i))
    assert rel_l2(rr, ii, re, im) < 1e-6 * 10
    e_t = (re.double() ** 2 + im.double() ** 2).sum()
    e_f = (r.double() ** 2 + i.double() ** 2).sum() / n
    assert abs(e_t - e_f) / e_t < 1e-6
    re2, im2 = seeded_complex(4, n, seed=3)
    a = oracle.fft((re + 2 * re2, im + 2 * im2))
    b1, b2 = oracle.fft((re, im)), oracle.fft((re2, im2))
    assert rel_l2(a[0], a[1], b1[0] + 2 * b2[0], b1[1] + 2 * b2[1]) < 1e-5


def test_bluestein_vs_float64_within_chirp_band():
    for n in [7, 100, 997]:
        re, im = seeded_complex(2, n)
        r, i = oracle.fft((re, im))
        ref = _dft64(re, im)
        assert rel_l2(r, i, ref.real, ref.imag) < 3e-4


# --- rfft / irfft / fftn / stft / istft -------------------------------------------------------


def test_rfft_irfft_vs_numpy():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(3, 128, generator=g)
    r, i = oracle.rfft(x)
    e = np.fft.rfft(x.double().numpy(), axis=-1)
    assert rel_l2(r, i, e.real, e.imag) < 1e-5
    back = oracle.irfft((r, i), n=128)
    assert rel_l2(back, torch.zeros_like(back), x, torch.zeros_like(x)) < 1e-5


def test_fft2_fftn_vs_numpy():
    rng = np.random.default_rng(42)
    x = rng.standard_normal((3, 16, 32)).astype(np.float32)
    r, i = oracle.fft2(torch.from_numpy(x))
    e = np.fft.fft2(x.astype(np.float64))
    assert rel_l2(r, i, e.real, e.imag) < 1e-5
    r, i = oracle.fftn(torch.from_numpy(x), dim=(0,))
    e = np.fft.fftn(x.astype(np.float64), axes=(0,))
    assert rel_l2(r, i, e.real, e.imag) < 1e-5


@pytest.mark.parametrize("n_fft,hop,center", [(512, 256, True), (256, 64, True), (128, 32, False)])
def test_stft_vs_torch_stft(n_fft, hop, center):
    g = torch.Generator().manual_seed(42)
    x = torch.randn(2, 4000, generator=g)
    r, i = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center)
    e = torch.stft(x.double(), n_fft, hop_length=hop, window=torch.hann_window(n_fft, dtype=torch.float64),
                   center=center, pad_mode="reflect", onesided=True, return_complex=True)
    assert r.shape == e.shape
    assert rel_l2(r, i, e.real, e.imag) < 1e-5


@pytest.mark.parametrize("n_fft,hop,center,pad_mode,onesided,normalized", [
    (512, 256, True, "constant", True, False),
    (512, 128, True, "replicate", True, False),
    (256, 100, True, "circular", True, True),
    (256, 64, True, "constant", False, False),    # two-sided spectrum
    (400, 160, True, "reflect", True, False),     # non-power-of-two n_fft: Bluestein per frame
    (400, 160, False, "reflect", True, False),
    (400, 100, True, "constant", True, True),
    (400, 133, True, "replicate", False, False),
    (12, 3, True, "reflect", True, False),
    (12, 5, False, "constant", True, False),
    (12, 4, True, "circular", False, True),
])
def test_stft_pad_modes_and_other_lengths_vs_torch_stft(n_fft, hop, center, pad_mode, onesided, normalized):
    # the oracle's F.pad modes, framing, window, non-power-of-two per-frame transform, onesided
    # slice and normalisation against torch.stft in float64.  Power-of-two n_fft within fp32
    # rounding; non-power-of-two n_fft carry the reference's fp32 Bluestein chirp (angle rounded
    # in fp32, trnfft/fft_core.py:1317-1320; pinned bit-exact by the golden vectors above), whose
    # distance from the exact DFT is 2e-5 to 4e-5 at n_fft 400 (5e-7 at 12)
    g = torch.Generator().manual_seed(n_fft * 3 + hop)
    x = torch.randn(2, 3001, generator=g)
    r, i = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center, pad_mode=pad_mode, onesided=onesided,
                       normalized=normalized)
    e = torch.stft(x.double(), n_fft, hop_length=hop, window=torch.hann_window(n_fft, dtype=torch.float64),
                   center=center, pad_mode=pad_mode, normalized=normalized, onesided=onesided,
                   return_complex=True)
    assert r.shape == e.shape
    tol = 1e-5 if n_fft & (n_fft - 1) == 0 else 1e-4
    assert rel_l2(r, i, e.real, e.imag) < tol
    # a plausible mistake fails: the padded signal reflected with its edge sample repeated
    # (mode "symmetric") instead of torch's reflect
    if center and pad_mode == "reflect":
        xs = torch.cat([x[:, : n_fft // 2].flip(-1), x, x[:, -(n_fft // 2):].flip(-1)], dim=-1)
        rs, is_ = oracle.stft(xs, n_fft=n_fft, hop_length=hop, center=False, onesided=onesided, normalized=normalized)
        assert rel_l2(rs, is_, e.real, e.imag) > 10 * tol


def test_istft_roundtrip():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(2, 1024, generator=g)
    spec = oracle.stft(x, n_fft=256, hop_length=64)
    y = oracle.istft(spec, n_fft=256, hop_length=64, length=1024)
    np.testing.assert_allclose(y.numpy(), x.numpy(), atol=1e-3)


@pytest.mark.parametrize("n_fft,hop,center,normalized,onesided,length,win", [
    (256, 64, True, False, True, None, "hann"),
    (512, 128, True, True, True, 3000, "hann"),
    (512, 200, True, False, True, 2500, "hann"),      # hop not dividing n_fft
    (128, 32, False, False, True, None, "hann+0.1"),  # no zero in the envelope without centring
    (64, 16, True, False, False, None, "hann"),       # two-sided spectrum (real part kept)
])
def test_istft_vs_torch_istft_float64(n_fft, hop, center, normalized, onesided, length, win):
    # torch.istft divides the overlap-add by the same squared-window envelope; with a window that
    # meets NOLA the reference's raw-sum branch (trnfft/api.py:450-452) is never taken
    g = torch.Generator().manual_seed(n_fft + hop)
    x = torch.randn(2, 3000, generator=g, dtype=torch.float64)
    w = torch.hann_window(n_fft, dtype=torch.float64)
    if win == "hann+0.1":
        w = w + 0.1
    spec = torch.stft(x, n_fft, hop_length=hop, window=w, center=center, normalized=normalized,
                      onesided=onesided, return_complex=True)
    spec = spec + 0.01 * torch.randn(spec.shape, generator=g, dtype=torch.complex128)  # not an exact STFT
    got = oracle.istft((spec.real.float(), spec.imag.float()), n_fft=n_fft, hop_length=hop, window=w.float(),
                       center=center, normalized=normalized, onesided=onesided, length=length)
    ref = torch.istft(spec, n_fft, hop_length=hop, window=w, center=center, normalized=normalized,
                      onesided=onesided, length=length, return_complex=not onesided)
    ref = ref.real if torch.is_complex(ref) else ref
    assert got.shape == ref.shape
    assert rel_l2(got, torch.zeros_like(got), ref, torch.zeros_like(ref)) < 1e-6


def test_istft_raw_sum_branch_closed_form():
    # hop = n_fft (frames do not overlap) and a window with zero ends: the envelope is w[j]^2, so
    # every sample is frame[j] * w[j] / w[j]^2 except where w[j] = 0, where the reference returns
    # the raw overlap-add, i.e. the inverse-transformed frame sample itself (trnfft/api.py:446-452)
    n, frames = 64, 5
    g = torch.Generator().manual_seed(3)
    f = torch.randn(2, frames, n, generator=g, dtype=torch.float64)
    w = torch.ones(n, dtype=torch.float64)
    w[0] = w[-1] = 0.0
    w[1] = w[-2] = 0.5
    spec = torch.fft.fft(f, dim=-1).transpose(-2, -1)  # (2, n, frames), two-sided
    got = oracle.istft((spec.real.float(), spec.imag.float()), n_fft=n, hop_length=n, window=w.float(),
                       center=False, onesided=False)
    expect = torch.where(w > 0, f / torch.where(w > 0, w, torch.ones_like(w)), f).reshape(2, frames * n)
    assert got.shape == expect.shape
    assert rel_l2(got, torch.zeros_like(got), expect, torch.zeros_like(expect)) < 1e-6
    # the zero-window samples are exactly the raw frame samples
    raw = got.reshape(2, frames, n)[..., [0, n - 1]].double()
    assert torch.allclose(raw, f[..., [0, n - 1]], atol=1e-5)


@pytest.mark.parametrize("sa,sb", [((6, 5), (5, 7)), ((3, 6, 5), (3, 5, 7)), ((2, 1, 6, 5), (4, 5, 7)), ((5,), (5, 7)),
                                   ((6, 5), (5,)), ((5,), (5,)), ((3, 6, 5), (5, 7))])
def test_complex_matmul_vs_numpy_complex(sa, sb):
    # the four-real-matmul formula of trnfft/complex.py:142-150 against complex matmul in numpy:
    # float64 operands agree to rounding, float32 ones within fp32 accumulation error
    rng = np.random.default_rng(len(sa) * 7 + len(sb))
    ar, ai = rng.standard_normal(sa), rng.standard_normal(sa)
    br, bi = rng.standard_normal(sb), rng.standard_normal(sb)
    e = np.matmul(ar + 1j * ai, br + 1j * bi)
    r, i = oracle.complex_matmul((torch.from_numpy(ar), torch.from_numpy(ai)), (torch.from_numpy(br), torch.from_numpy(bi)))
    assert tuple(r.shape) == e.shape
    assert rel_l2(r, i, e.real, e.imag) < 1e-14
    f = lambda a: torch.from_numpy(a.astype(np.float32))  # noqa: E731
    r, i = oracle.complex_matmul((f(ar), f(ai)), (f(br), f(bi)))
    assert rel_l2(r, i, e.real, e.imag) < 1e-6


# --- complex linear / DFT-GEMM / row-column --------------------------------------------------


def test_complex_linear_vs_float64_and_kat():
    # (1+2i)(3+4i) = -5+10i (reference tests/test_complex.py:35-41)
    r, i = oracle.complex_linear((torch.tensor([[1.0]]), torch.tensor([[2.0]])), torch.tensor([[3.0]]), torch.tensor([[4.0]]))
    assert r.item() == -5.0 and i.item() == 10.0
    g = torch.Generator().manual_seed(42)
    xr, xi = torch.randn(16, 32, generator=g), torch.randn(16, 32, generator=g)
    wr, wi = torch.randn(24, 32, generator=g), torch.randn(24, 32, generator=g)
    br, bi = torch.randn(24, generator=g), torch.randn(24, generator=g)
    r, i = oracle.complex_linear((xr, xi), wr, wi, br, bi)
    z = (xr.double() + 1j * xi.double()) @ (wr.double() + 1j * wi.double()).T + (br.double() + 1j * bi.double())
    assert rel_l2(r, i, z.real, z.imag) < 1e-6


def test_dft_gemm_oracle():
    re, im = seeded_complex(4, 256)
    r, i = oracle.dft_gemm(re, im, False)
    e = _dft64(re, im)
    assert rel_l2(r, i, e.real, e.imag) < 1e-6
    # the reference's fp32-angle W is measurably less accurate (2e-5 at n=256)
    r2, i2 = oracle.dft_gemm(re, im, False, fp32_angles=True)
    assert rel_l2(r2, i2, e.real, e.imag) > 5e-6


def test_stage_parallel_equals_fft_core():
    re, im = seeded_complex(1, 4096)
    a = oracle.stage_parallel_fft(re[0], im[0], False)
    b = oracle.fft_core(re[0], im[0], False)
    assert rel_l2(a[0], a[1], b[0], b[1]) < 1e-5
    assert oracle.factorize(1 << 20) == (1024, 1024)
    with pytest.raises(ValueError):
        oracle.factorize(4099)
