"""GPU parity of the fused inverse STFT against the oracle's restatement of trnfft/api.py:368-470
(Hermitian completion, inverse c2c, real part, overlap-add with window-square envelope division
and raw fallback, centre trim, length handling)."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
import trnfft_amd
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _spec(lead, n_fft, frames, seed):
    g = torch.Generator().manual_seed(seed)
    f = n_fft // 2 + 1
    # arbitrary bins, imaginary parts at bins 0 and n/2 included (the real part drops them)
    return torch.randn(*lead, f, frames, generator=g), torch.randn(*lead, f, frames, generator=g)


CASES = [
    # n_fft, hop, frames, center, normalized, length
    (512, 128, 100, True, False, None),
    (512, 256, 626, True, False, None),
    (256, 64, 37, True, True, None),
    (1024, 256, 9, True, False, 1500),       # shorter than the signal: truncation
    (256, 64, 12, True, False, 2000),        # longer: zero fill
    (128, 96, 20, False, False, None),       # hop not dividing n_fft
    (64, 80, 15, False, False, None),        # hop > n_fft: gaps (raw overlap-add of nothing = 0)
    (16, 4, 50, True, False, None),
    (4096, 1024, 7, True, False, None),
    (2048, 512, 5, False, True, None),
    (512, 40, 30, True, False, None),        # long halo (12 frames): the widest tile
    (1024, 128, 40, True, False, None),      # halo 7 > half the measured 8-frame tile: widest tile
    (32, 16, 300, True, False, None),
    # interior tiles write four samples per thread when hop, trim, pitch and length allow; these
    # take the one-sample path: a hop that is not a multiple of 4, a length that is not
    (512, 126, 60, True, False, None),
    (512, 128, 60, True, False, 5001),
]


# bins-major spectra (the reference's layout, what stft returns) against the frames-major input
# path on the same spectra and against the oracle: batch, frame counts, halo 0..3, zero fill,
# leading dims
RANGE_CASES = [
    # lead, n_fft, hop, frames, center, normalized, length
    ((64,), 512, 256, 626, True, False, None),    # BASELINE config 2's inverse
    ((1,), 512, 256, 2000, True, False, None),    # one signal
    ((2,), 512, 256, 627, True, False, None),     # odd frame count
    ((300,), 512, 256, 70, True, False, None),    # more signals than CUs
    ((3,), 512, 512, 90, True, False, None),      # halo 0
    ((4,), 512, 200, 150, False, True, None),     # halo 2, hop not dividing n_fft, no centring
    ((2,), 512, 256, 300, True, False, 40000),    # length beyond the signal: zero fill
    ((2,), 512, 256, 300, True, False, 50001),    # one-sample path (length not a multiple of 4)
    ((5, 2), 256, 128, 400, True, False, None),   # leading dims; n_fft 256 (two pairs per wavefront)
    ((3,), 256, 64, 200, True, True, 12000),      # halo 3, truncation
    ((1,), 256, 100, 64, False, False, None),     # hop not a multiple of 4
]


@pytest.mark.parametrize("lead,n_fft,hop,frames,center,normalized,length", RANGE_CASES)
def test_istft_bins_major_against_frames_major(lead, n_fft, hop, frames, center, normalized, length):
    re, im = _spec(lead, n_fft, frames, seed=frames + hop)
    got = trnfft_amd.istft(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop_length=hop, center=center,
                           normalized=normalized, length=length)
    ref = oracle.istft((re, im), n_fft, hop_length=hop, center=center, normalized=normalized, length=length)
    assert got.shape == ref.shape
    assert _rel(got, ref) <= 1e-6 * math.log2(n_fft) * 4
    # the frames-major kernel on the same spectra: the same samples to rounding
    fm = trnfft_amd.istft(ComplexTensor._wrap(re.transpose(-2, -1).contiguous().cuda().transpose(-2, -1),
                                              im.transpose(-2, -1).contiguous().cuda().transpose(-2, -1)),
                          n_fft, hop_length=hop, center=center, normalized=normalized, length=length)
    assert _rel(got, fm) <= 1e-6 * math.log2(n_fft)


@pytest.mark.parametrize("n_fft,hop,frames,center,normalized,length", CASES)
def test_istft_matches_reference(n_fft, hop, frames, center, normalized, length):
    re, im = _spec((3,), n_fft, frames, seed=n_fft + hop)
    got = trnfft_amd.istft(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop_length=hop, center=center,
                           normalized=normalized, length=length)
    ref = oracle.istft((re, im), n_fft, hop_length=hop, center=center, normalized=normalized, length=length)
    assert got.shape == ref.shape
    assert _rel(got, ref) <= 1e-6 * math.log2(n_fft) * 4
    # these shapes run on the fused kernel (not the composed fallback)
    assert trnfft_amd.api._istft_fused(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop, n_fft, None, center,
                                       normalized, True, length) is not None


# two-sided spectra (n_fft bins, not Hermitian): each frame is the real part of its inverse
# transform (trnfft/api.py:397-421 with onesided=False); power-of-two n_fft on the fused kernel
TWO_SIDED_CASES = [
    # lead, n_fft, hop, frames, center, normalized, length
    ((3,), 512, 128, 100, True, False, None),
    ((64,), 512, 256, 626, True, False, None),    # C2's frame count
    ((2,), 256, 64, 37, True, True, None),
    ((2,), 1024, 256, 9, True, False, 1500),      # truncation
    ((2,), 256, 64, 12, True, False, 2000),       # zero fill
    ((2,), 128, 96, 20, False, False, None),      # hop not dividing n_fft
    ((2,), 64, 80, 15, False, False, None),       # hop > n_fft: gaps
    ((2,), 16, 4, 50, True, False, None),
    ((1,), 4096, 1024, 7, True, False, None),
    ((2,), 2048, 512, 5, False, True, None),
    ((2,), 512, 40, 30, True, False, None),       # long halo: the widest tile
    ((2, 2), 64, 32, 40, True, False, None),      # leading dims
    ((2,), 512, 126, 60, True, False, 5001),      # one-sample path
]


@pytest.mark.parametrize("lead,n_fft,hop,frames,center,normalized,length", TWO_SIDED_CASES)
def test_istft_two_sided_matches_reference(lead, n_fft, hop, frames, center, normalized, length):
    g = torch.Generator().manual_seed(n_fft + hop + frames)
    re, im = torch.randn(*lead, n_fft, frames, generator=g), torch.randn(*lead, n_fft, frames, generator=g)
    spec = ComplexTensor(re.cuda(), im.cuda())
    got = trnfft_amd.istft(spec, n_fft, hop_length=hop, center=center, normalized=normalized, onesided=False,
                           length=length)
    ref = oracle.istft((re, im), n_fft, hop_length=hop, center=center, normalized=normalized, onesided=False,
                       length=length)
    assert got.shape == ref.shape
    assert _rel(got, ref) <= 1e-6 * math.log2(n_fft) * 4
    assert trnfft_amd.api._istft_fused(spec, n_fft, hop, n_fft, None, center, normalized, False, length) is not None
    # frames-major input (transposed views of (..., frames, n_fft) buffers): the same samples
    fm = trnfft_amd.istft(ComplexTensor._wrap(re.transpose(-2, -1).contiguous().cuda().transpose(-2, -1),
                                              im.transpose(-2, -1).contiguous().cuda().transpose(-2, -1)),
                          n_fft, hop_length=hop, center=center, normalized=normalized, onesided=False, length=length)
    assert _rel(got, fm) <= 1e-6 * math.log2(n_fft)


def test_stft_istft_two_sided_roundtrip():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 20000, generator=g).cuda()
    spec = trnfft_amd.stft(x, n_fft=512, hop_length=128, onesided=False)
    assert spec.real.shape[-2] == 512
    y = trnfft_amd.istft(spec, n_fft=512, hop_length=128, onesided=False, length=20000)
    assert _rel(y, x) <= 1e-5


def test_istft_two_sided_non_pow2_composes():
    # two-sided spectra at an n_fft that is not a power of two keep the composed path
    g = torch.Generator().manual_seed(10)
    re, im = torch.randn(2, 400, 30, generator=g), torch.randn(2, 400, 30, generator=g)
    spec = ComplexTensor(re.cuda(), im.cuda())
    assert trnfft_amd.api._istft_fused(spec, 400, 160, 400, None, True, False, False, None) is None
    got = trnfft_amd.istft(spec, 400, hop_length=160, onesided=False)
    ref = oracle.istft((re, im), 400, hop_length=160, onesided=False)
    assert _rel(got, ref) <= 1e-4


def test_istft_window_with_zeros_uses_raw_sum():
    # a symmetric Hann (zero at both ends) without centring: the envelope is zero at the first
    # sample, where the reference returns the raw (unwindowed) overlap-add
    n_fft, hop, frames = 256, 64, 20
    re, im = _spec((2,), n_fft, frames, seed=3)
    w = torch.hann_window(n_fft, periodic=False)
    got = trnfft_amd.istft(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop_length=hop, window=w.cuda(), center=False)
    ref = oracle.istft((re, im), n_fft, hop_length=hop, window=w, center=False)
    assert _rel(got, ref) <= 1e-5
    torch.testing.assert_close(got[:, 0].cpu(), ref[:, 0], rtol=1e-5, atol=1e-6)


def test_istft_leading_dims_and_win_length():
    n_fft, hop, frames = 512, 128, 33
    re, im = _spec((2, 3), n_fft, frames, seed=4)
    w = torch.hann_window(400)
    got = trnfft_amd.istft(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop_length=hop, win_length=400, window=w.cuda())
    ref = oracle.istft((re, im), n_fft, hop_length=hop, win_length=400, window=w)
    assert got.shape == ref.shape == (2, 3, (frames - 1) * hop)
    assert _rel(got, ref) <= 1e-5


def test_stft_istft_roundtrip_full_size():
    # BASELINE config 2 shape: 64 waveforms x 160000 samples, n_fft 512, hop 256
    from bench import make_stft_input

    x = make_stft_input(64, 160000).cuda()
    spec = trnfft_amd.stft(x, n_fft=512, hop_length=256)
    y = trnfft_amd.istft(spec, n_fft=512, hop_length=256, length=160000)
    assert y.shape == x.shape
    assert _rel(y, x) <= 1e-5


def test_istft_small_hop_falls_back_to_composition():
    # halo too long for the fused tile: the composed path runs instead, same result
    n_fft, hop, frames = 4096, 16, 300
    re, im = _spec((1,), n_fft, frames, seed=5)
    got = trnfft_amd.istft(ComplexTensor(re.cuda(), im.cuda()), n_fft, hop_length=hop)
    ref = oracle.istft((re, im), n_fft, hop_length=hop)
    assert _rel(got, ref) <= 1e-4


BLUE_CASES = [
    # n_fft, hop, frames, center, normalized, length; m = the inverse chain's length (>= 2 n_fft - 1)
    (400, 160, 101, True, False, None),     # m 1024
    (400, 100, 60, True, True, None),
    (320, 160, 50, True, False, 9000),      # m 768; longer length: zero fill
    (9, 2, 40, True, False, None),          # m 32
    (12, 3, 80, True, False, None),
    (30, 7, 70, False, False, None),        # m 64
    (40, 10, 50, True, False, None),        # m 96
    (50, 60, 20, False, False, None),       # m 128; hop > n_fft
    (90, 30, 40, True, False, None),        # m 192
    (99, 33, 30, True, False, None),        # m 256; odd n_fft
    (100, 25, 40, True, False, 900),        # shorter length: truncation
    (150, 50, 30, True, True, None),        # m 384
    (200, 80, 30, True, False, None),       # m 512
    (600, 150, 20, True, False, None),      # m 1536
    (1000, 250, 12, False, True, None),     # m 2048
    (1500, 750, 9, True, False, None),      # m 3072
    (2047, 1024, 6, True, False, None),     # m 4096
]


@pytest.mark.parametrize("n_fft,hop,frames,center,normalized,length", BLUE_CASES)
def test_istft_non_pow2_matches_reference(n_fft, hop, frames, center, normalized, length):
    # one inverse Bluestein chain per frame (the reference's fp32 chirp), fused with the
    # completion, window, overlap-add and envelope
    from conftest import tol_bluestein

    re, im = _spec((3,), n_fft, frames, seed=n_fft * 3 + hop)
    x = ComplexTensor(re.cuda(), im.cuda())
    got = trnfft_amd.istft(x, n_fft, hop_length=hop, center=center, normalized=normalized, length=length)
    ref = oracle.istft((re, im), n_fft, hop_length=hop, center=center, normalized=normalized, length=length)
    assert got.shape == ref.shape
    assert _rel(got, ref) <= tol_bluestein(n_fft)
    assert trnfft_amd.api._istft_fused(x, n_fft, hop, n_fft, None, center, normalized, True, length) is not None


@pytest.mark.parametrize("n_fft,hop,frames", [(400, 10, 120), (2047, 512, 8)])
def test_istft_non_pow2_small_hop_composes(n_fft, hop, frames):
    # a halo of more than half the fused tile: the composed path (frame inverse transforms +
    # overlap-add)
    from conftest import tol_bluestein

    re, im = _spec((2,), n_fft, frames, seed=6)
    x = ComplexTensor(re.cuda(), im.cuda())
    assert trnfft_amd.api._istft_fused(x, n_fft, hop, n_fft, None, True, False, True, None) is None
    got = trnfft_amd.istft(x, n_fft, hop_length=hop)
    ref = oracle.istft((re, im), n_fft, hop_length=hop)
    assert _rel(got, ref) <= tol_bluestein(n_fft)


def test_stft_istft_roundtrip_non_pow2():
    # C2's signals at n_fft 400 / hop 160 through both fused per-frame Bluestein kernels
    from bench import make_stft_input

    x = make_stft_input(8, 160000).cuda()
    spec = trnfft_amd.stft(x, n_fft=400, hop_length=160)
    y = trnfft_amd.istft(spec, n_fft=400, hop_length=160, length=160000)
    assert y.shape == x.shape
    assert _rel(y, x) <= 1e-4
