"""GPU parity of the API layer: rfft/irfft/hfft, fft2/fftn/ifftn, stft/istft vs the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, tol_bluestein, tol_pow2
from trnfft_amd import ComplexTensor
from trnfft_amd.fft_core import fft2_small_ok

pytestmark = pytest.mark.gpu


def test_rfft_irfft():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(3, 128, generator=g)
    got = trnfft_amd.rfft(x.cuda())
    ref = oracle.rfft(x)
    assert got.shape == (3, 65)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(128)
    back = trnfft_amd.irfft(got, n=128)
    ref_back = oracle.irfft(ref, n=128)
    assert rel_l2(back, torch.zeros_like(back), ref_back, torch.zeros_like(ref_back)) <= tol_pow2(128)


@pytest.mark.parametrize("n,bins,batch", [(8, 5, 3), (64, 33, 2), (100, 51, 3), (1024, 513, 4), (1000, 501, 2),
                                           (256, 129, 1), (100, 60, 2), (64, 40, 3)])
def test_hfft_ihfft_vs_numpy_and_oracle(n, bins, batch):
    # hfft = irfft(conj(x), n) * n (trnfft/api.py:71-86).  At the default n = 2*(bins-1) this is
    # numpy's hfft; for a shorter n the reference's Hermitian completion (trnfft/api.py:49-68)
    # keeps every given bin and mirrors bins 1..n-bins, which numpy does not, so those cases are
    # checked against the oracle's restatement of it
    rng = np.random.default_rng(n + bins)
    re = rng.standard_normal((batch, bins)).astype(np.float32)
    im = rng.standard_normal((batch, bins)).astype(np.float32)
    got = trnfft_amd.hfft(ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda()), n=n)
    tol = tol_pow2(n) if n & (n - 1) == 0 else 3 * tol_bluestein(n)
    if n == 2 * (bins - 1):
        ref = np.fft.hfft(re.astype(np.float64) + 1j * im, n=n, axis=-1)
    else:
        ref = oracle.irfft((torch.from_numpy(re), -torch.from_numpy(im)), n=n).double().numpy() * n
    assert rel_l2(got, torch.zeros_like(got), ref, np.zeros_like(ref)) <= tol, (n, bins)
    x = rng.standard_normal((batch, n)).astype(np.float32)
    z = trnfft_amd.ihfft(torch.from_numpy(x).cuda())
    e = np.fft.ihfft(x.astype(np.float64), axis=-1)
    assert rel_l2(z.real, z.imag, e.real, e.imag) <= tol, n


def test_hfft_longer_n_than_the_spectrum_raises_like_the_reference():
    # n > 2*(bins-1): the reference's completion has no zero padding and fails on the shape
    # mismatch (trnfft/api.py:64-65); the HIP path raises the same RuntimeError
    x = ComplexTensor(torch.randn(2, 400).cuda(), torch.randn(2, 400).cuda())
    with pytest.raises(RuntimeError):
        trnfft_amd.hfft(x, n=1000)


def test_hfft_ihfft_roundtrip():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(32, generator=g)
    y = trnfft_amd.hfft(trnfft_amd.ihfft(x.cuda(), n=32), n=32)
    np.testing.assert_allclose(y.cpu().numpy(), x.numpy(), atol=1e-4)
    e = np.fft.ihfft(x.numpy(), n=32)
    z = trnfft_amd.ihfft(x, n=32)
    np.testing.assert_allclose(z.real.numpy(), e.real, atol=1e-5)
    np.testing.assert_allclose(z.imag.numpy(), e.imag, atol=1e-5)


@pytest.mark.parametrize("shape", [(8, 8), (3, 64, 32), (2, 256, 512)])
def test_fft2_vs_oracle(shape):
    rng = np.random.default_rng(42)
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    got = trnfft_amd.fft2(x.cuda())
    ref = oracle.fft2(x)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(shape[-1] * shape[-2])


def test_fftn_ifftn():
    rng = np.random.default_rng(42)
    x = torch.from_numpy(rng.standard_normal((4, 8, 16)).astype(np.float32))
    got = trnfft_amd.fftn(x.cuda())
    ref = oracle.fftn(x)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(512)
    back = trnfft_amd.ifftn(got)
    assert rel_l2(back.real, back.imag, x, torch.zeros_like(x)) <= 2 * tol_pow2(512)
    got0 = trnfft_amd.fftn(x.cuda(), dim=(0,))
    ref0 = oracle.fftn(x, dim=(0,))
    assert rel_l2(got0.real, got0.imag, *ref0) <= tol_pow2(4)


def test_fft2_config4a_one_image_and_parseval():
    # BASELINE config 4a at full shape (32 x 2048 x 2048, U[0,1)): oracle on one image, Parseval on all
    g = torch.Generator().manual_seed(42)
    x = torch.rand(32, 2048, 2048, generator=g)
    got = trnfft_amd.fft2(x.cuda())
    ref = oracle.fft2(x[5])
    assert rel_l2(got.real[5], got.imag[5], *ref) <= tol_pow2(2048)
    e_t = (x.double() ** 2).sum()
    e_f = (got.real.double() ** 2 + got.imag.double() ** 2).sum().cpu() / (2048 * 2048)
    assert abs(e_t - e_f) / e_t < 1e-5


@pytest.mark.parametrize("n_fft,hop,center,normalized,onesided", [
    (512, 256, True, False, True),
    (256, 64, True, False, True),
    (128, 32, False, False, True),
    (64, 16, True, True, False),
])
def test_stft_vs_oracle(n_fft, hop, center, normalized, onesided):
    g = torch.Generator().manual_seed(42)
    x = torch.randn(3, 4000, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center, normalized=normalized, onesided=onesided)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center, normalized=normalized, onesided=onesided)
    assert got.shape == ref[0].shape
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n_fft)


@pytest.mark.parametrize("n_fft,hop,pad_mode,center,onesided,normalized,shape", [
    (400, 160, "reflect", True, True, False, (2, 16000)),      # 25 ms @ 16 kHz: a Bluestein transform per frame
    (400, 100, "constant", True, True, True, (3, 5000)),
    (12, 3, "replicate", True, True, False, (2, 301)),         # the fused kernel's shortest convolution (32)
    (12, 5, "circular", True, False, False, (1, 200)),         # (1, L): the reference squeezes the batch axis
    (8192, 2048, "reflect", True, True, False, (2, 30000)),    # above the fused kernel's range
    (8192, 4096, "constant", True, False, True, (20000,)),
    (512, 128, "constant", True, True, False, (2, 3, 4000)),   # fused kernel on the device-padded signal
    (512, 256, "replicate", True, True, True, (4000,)),
    (1024, 300, "circular", True, False, False, (2, 5000)),
    (8, 2, "reflect", False, True, False, (2, 100)),           # below the fused kernels' range
    (1000, 250, "reflect", False, False, False, (2, 3000)),
    (2, 1, "constant", True, True, False, (3, 17)),
])
def test_stft_any_n_fft_and_pad_mode_vs_oracle(n_fft, hop, pad_mode, center, onesided, normalized, shape):
    # every stft the reference computes (trnfft/api.py:291-365: F.pad with any mode, any n_fft
    # through fft_core / Bluestein) runs here too, on the device
    g = torch.Generator().manual_seed(n_fft + hop)
    x = torch.randn(*shape, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center, pad_mode=pad_mode,
                          normalized=normalized, onesided=onesided)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center, pad_mode=pad_mode, normalized=normalized,
                      onesided=onesided)
    assert got.shape == ref[0].shape
    tol = tol_pow2(n_fft) if n_fft & (n_fft - 1) == 0 else tol_bluestein(n_fft)
    assert rel_l2(got.real, got.imag, *ref) <= tol


@pytest.mark.parametrize("n_fft,hop,center,onesided,normalized,shape", [
    # convolution length m: the shortest power of two or 3 * 2^k >= n_fft + n_bins - 1
    (9, 3, True, True, False, (2, 500)),         # m = 32
    (12, 4, False, False, False, (3, 257)),      # m = 32, two-sided
    (20, 7, True, True, True, (2, 1000)),        # m = 32 (30 points)
    (30, 12, True, True, False, (2, 1500)),      # m = 64
    (33, 11, True, False, False, (1, 999)),      # m = 96, two-sided
    (50, 20, True, True, False, (2, 2000)),      # m = 96
    (80, 30, False, True, False, (2, 2500)),     # m = 128
    (100, 40, True, True, False, (4, 3001)),     # m = 192
    (150, 60, True, True, True, (2, 4000)),      # m = 256
    (200, 64, True, True, False, (2, 8000)),     # m = 384
    (257, 128, True, True, False, (2, 5000)),    # m = 512
    (300, 450, False, True, False, (2, 9000)),   # m = 512, hop > n_fft
    (400, 160, True, True, False, (3, 16000)),   # m = 768
    (400, 160, True, True, False, (2, 201)),     # every frame reaches into the reflect padding
    (640, 160, False, True, True, (2, 9000)),    # m = 1024
    (1000, 250, True, True, False, (2, 7000)),   # m = 1536
    (1000, 250, True, False, False, (2, 7000)),  # m = 2048, two-sided
    (1025, 300, True, True, False, (2, 9000)),   # m = 2048
    (2000, 500, True, True, False, (1, 20000)),  # m = 3072
    (2500, 600, True, True, False, (1, 20000)),  # m = 4096
    (2047, 512, True, False, False, (1, 20000)), # m = 4096, two-sided
])
def test_stft_fused_bluestein_frames_vs_oracle(n_fft, hop, center, onesided, normalized, shape):
    # n_fft that is not a power of two, without autograd: one fused kernel with a Bluestein
    # transform per frame (the reference's chain, trnfft/api.py:339-349 -> fft_core.py:1285-1376)
    g = torch.Generator().manual_seed(n_fft * 7 + hop)
    x = torch.randn(*shape, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center, normalized=normalized,
                          onesided=onesided)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center, normalized=normalized, onesided=onesided)
    assert got.shape == ref[0].shape
    assert rel_l2(got.real, got.imag, *ref) <= tol_bluestein(n_fft)


@pytest.mark.parametrize("n_fft,hop,pad_mode", [(400, 160, "reflect"), (1000, 256, "constant"), (99, 33, "circular")])
def test_stft_fused_bluestein_matches_composed_path(n_fft, hop, pad_mode):
    # the reference's composition on the device (pad, frame gather, window, Bluestein rows of
    # rfft, transpose) against the fused kernel: both run the reference's chain, so they agree
    # to fp32 rounding
    g = torch.Generator().manual_seed(13)
    x = torch.randn(3, 12000, generator=g).cuda()
    fused = trnfft_amd.stft(x, n_fft=n_fft, hop_length=hop, pad_mode=pad_mode)
    w = torch.hann_window(n_fft, device="cuda")
    xp = torch.nn.functional.pad(x.unsqueeze(1), (n_fft // 2, n_fft // 2), mode=pad_mode).squeeze(1)
    spec = trnfft_amd.rfft((xp.unfold(-1, n_fft, hop) * w).contiguous())
    assert fused.shape == spec.real.transpose(-2, -1).shape
    assert rel_l2(fused.real, fused.imag, spec.real.transpose(-2, -1), spec.imag.transpose(-2, -1)) \
        <= tol_bluestein(n_fft) / 4


@pytest.mark.parametrize("n_fft,hop", [(512, 256), (256, 64), (400, 160), (8192, 2048), (8, 2)])
def test_stft_result_layout_is_the_references(n_fft, hop):
    # the reference returns ComplexTensor(result_re, result_im) of its transposed frame spectra,
    # and its constructor makes both planes contiguous (trnfft/api.py:357-365,
    # trnfft/complex.py:29-33): dense (..., freq, time) planes, the oracle's strides
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 3, 20000, generator=g)
    y = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop)
    assert y.real.shape == ref[0].shape
    assert y.real.is_contiguous() and y.imag.is_contiguous()
    assert y.real.stride() == ref[0].stride() and y.imag.stride() == ref[1].stride()
    tol = tol_pow2(n_fft) if n_fft & (n_fft - 1) == 0 else tol_bluestein(n_fft)
    assert rel_l2(y.real, y.imag, *ref) <= tol
    # the opt-in frames-major result: the same values as views of (..., time, freq) buffers (the
    # memory order of torch.stft's result); istft takes either order
    fm = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, frames_major=True)
    assert fm.real.transpose(-2, -1).is_contiguous() and fm.imag.transpose(-2, -1).is_contiguous()
    assert rel_l2(fm.real, fm.imag, y.real, y.imag) <= tol
    a = trnfft_amd.istft(y, n_fft=n_fft, hop_length=hop, length=20000)
    b = trnfft_amd.istft(fm, n_fft=n_fft, hop_length=hop, length=20000)
    assert rel_l2(a, torch.zeros_like(a), b, torch.zeros_like(b)) <= tol
    assert rel_l2(a, torch.zeros_like(a), x.cuda(), torch.zeros_like(a)) <= 100 * tol


@pytest.mark.parametrize("n_fft,hop,shape,center", [
    (512, 256, (64, 160000), True),    # 626 frames, 4 ranges per signal, 256 workgroups
    (512, 256, (1, 40192), True),      # one signal (158 frames): ranges of one sub-tile and a half
    (512, 128, (3, 9100), True),       # 72 frames: two ranges of 36
    (512, 300, (5, 50100), False),     # no padding; hop not a divisor of n_fft (166 frames)
    (512, 256, (300, 16640), True),    # more signals than CUs (66 frames, two ranges each)
    (512, 512, (7, 33536), True),      # hop = n_fft (66 frames)
    (512, 100, (2, 12445), True),      # odd frame count (125): the fixed-tile kernel
    (256, 64, (16, 30016), True),      # n_fft 256: two pair transforms per wavefront (470 frames)
    (256, 128, (130, 8320), True),
    (256, 32, (1, 4000), False),       # 118 frames
])
def test_stft_bins_major_whole_line_kernel_vs_oracle(n_fft, hop, shape, center):
    # the whole-line bins-major kernel (frame ranges per workgroup, forward and backward walks,
    # carried line parts, reflected edge frames) against the reference's composition
    g = torch.Generator().manual_seed(n_fft + hop + shape[0])
    x = torch.randn(*shape, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center)
    assert got.shape == ref[0].shape and got.real.is_contiguous()
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n_fft)
    # every element written: the frames-major kernel gives the same spectra (to rounding)
    fm = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center, frames_major=True)
    assert torch.allclose(got.real, fm.real, rtol=1e-5, atol=1e-4 * float(fm.real.abs().max()))
    assert torch.allclose(got.imag, fm.imag, rtol=1e-5, atol=1e-4 * float(fm.imag.abs().max()))


def test_stft_bins_major_into_planes_at_any_line_offset():
    # through the C ABI: output planes that start anywhere on the 8-byte grid (the kernel writes
    # whole 128-byte lines from each row's offset; other alignments take the fixed-tile kernel),
    # with sentinels around each plane: nothing is written outside the (64, 257, 626) planes
    from trnfft_amd import _lib
    from trnfft_amd.dispatch import ptr, stream_handle
    from trnfft_amd.plan import native_plan

    x = torch.randn(8, 40000, generator=torch.Generator().manual_seed(3)).cuda()
    win = torch.hann_window(512, device="cuda")
    frames = 1 + 40000 // 256
    n = 8 * 257 * frames
    plan = native_plan(_lib.KIND_STFT, 512, False, 0, hop=256, flags=_lib.STFT_CENTER | _lib.STFT_ONESIDED)
    ref = trnfft_amd.stft(x, n_fft=512, hop_length=256)
    for off_re, off_im in [(0, 0), (2, 2), (18, 18), (30, 30), (6, 22), (1, 1)]:
        bre = torch.full((n + 64,), 7.0, device="cuda")
        bim = torch.full((n + 64,), 7.0, device="cuda")
        o_re, o_im = bre[off_re:off_re + n], bim[off_im:off_im + n]
        rc = _lib.lib().tfa_stft_execute(plan.handle, 8, 40000, ptr(x), ptr(win), ptr(o_re), ptr(o_im),
                                         stream_handle(x.device))
        _lib.check(rc, "tfa_stft_execute")
        torch.cuda.synchronize()
        assert torch.allclose(o_re.view(8, 257, frames), ref.real, rtol=1e-5, atol=1e-3), (off_re, off_im)
        assert torch.allclose(o_im.view(8, 257, frames), ref.imag, rtol=1e-5, atol=1e-3), (off_re, off_im)
        assert bool((bre[:off_re] == 7.0).all()) and bool((bre[off_re + n:] == 7.0).all())
        assert bool((bim[:off_im] == 7.0).all()) and bool((bim[off_im + n:] == 7.0).all())


def test_stft_win_length_below_n_fft_and_custom_window_composed():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 6000, generator=g)
    w = torch.rand(300, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=400, hop_length=128, win_length=300, window=w.cuda())
    ref = oracle.stft(x, n_fft=400, hop_length=128, win_length=300, window=w)
    assert got.shape == ref[0].shape
    assert rel_l2(got.real, got.imag, *ref) <= tol_bluestein(400)


def test_stft_no_whole_frame_returns_empty_like_the_reference():
    # center=False and a signal shorter than n_fft by less than a hop: num_frames = 0, and the
    # reference's frame index is empty (trnfft/api.py:321-327)
    x = torch.randn(2, 300)
    got = trnfft_amd.stft(x.cuda(), n_fft=400, hop_length=200, center=False)
    ref = oracle.stft(x, n_fft=400, hop_length=200, center=False)
    assert got.shape == ref[0].shape == (2, 201, 0)


def test_stft_config2_full_size():
    # 64 x 160000 samples, 3 sinusoids + N(0, 0.1) noise, n_fft 512, hop 256
    from bench import make_stft_input

    x = make_stft_input(64, 160000, seed=42)
    got = trnfft_amd.stft(x.cuda(), n_fft=512, hop_length=256)
    assert got.shape == (64, 257, 626)
    ref = oracle.stft(x, n_fft=512, hop_length=256)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(512)


def test_istft_roundtrip():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(4, 1024, generator=g)
    spec = trnfft_amd.stft(x.cuda(), n_fft=256, hop_length=64)
    y = trnfft_amd.istft(spec, n_fft=256, hop_length=64, length=1024)
    np.testing.assert_allclose(y.cpu().numpy(), x.numpy(), atol=1e-3)
    ref = oracle.istft((spec.real.cpu(), spec.imag.cpu()), n_fft=256, hop_length=64, length=1024)
    assert float((y.cpu() - ref).abs().max()) < 1e-4


def test_stft_single_tone():
    sr, freq, n_fft = 1000, 100, 256
    t = torch.arange(0, 1.0, 1.0 / sr)
    s = torch.sin(2 * np.pi * freq * t)
    res = trnfft_amd.stft(s.cuda(), n_fft=n_fft, hop_length=64, center=False)
    peak = res.abs().mean(dim=-1).argmax().item()
    assert abs(peak - int(freq * n_fft / sr)) <= 1


@pytest.mark.parametrize("shape,dim", [
    ((6, 16, 12), None),        # 12 is not a power of two: transpose + Bluestein path on that axis
    ((3, 40, 8), (0, 1)),       # ragged column tiles (stride 8 < tile width)
    ((5, 128, 3), (1,)),        # stride 3
    ((2, 4096, 17), (1,)),      # longest strided axis
    ((4, 8, 2, 16), (0, 2)),
])
def test_fftn_strided_axes_vs_oracle(shape, dim):
    rng = np.random.default_rng(7)
    re = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    im = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    got = trnfft_amd.fftn(ComplexTensor(re.cuda(), im.cuda()), dim=dim)
    ref = oracle.fftn((re, im), dim=dim)
    dims = range(len(shape)) if dim is None else dim
    total = 1
    for d in dims:
        total *= shape[d]
    assert rel_l2(got.real, got.imag, *ref) <= 1e-5 * math.log2(total)
    back = trnfft_amd.ifftn(got, dim=dim)
    assert rel_l2(back.real, back.imag, re, im) <= 1e-5 * math.log2(total)


@pytest.mark.parametrize("n_fft", [512, 400])
def test_stft_hop_beyond_the_signal(n_fft):
    # one frame per signal; a hop beyond 32 bits is clamped on the host and the kernels' tile
    # bounds are 64-bit, so no frame offset wraps
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 3000, generator=g)
    tol = tol_pow2(n_fft) if n_fft & (n_fft - 1) == 0 else tol_bluestein(n_fft)
    for hop, center in [(5000, True), (3_000_000_000, True), (3_000_000_000, False)]:
        got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop, center=center)
        ref = oracle.stft(x, n_fft=n_fft, hop_length=hop, center=center)
        assert got.shape == ref[0].shape == (2, n_fft // 2 + 1, 1)
        assert rel_l2(got.real, got.imag, *ref) <= tol


@pytest.mark.parametrize("n_fft,hop,length,batch_shape", [
    (16, 4, 301, (2,)),
    (4096, 1024, 20000, (1,)),
    (512, 200, 9999, (2, 3)),
    (1024, 256, 5000, ()),
])
def test_stft_edge_shapes(n_fft, hop, length, batch_shape):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(*batch_shape, length, generator=g)
    got = trnfft_amd.stft(x.cuda(), n_fft=n_fft, hop_length=hop)
    ref = oracle.stft(x, n_fft=n_fft, hop_length=hop)
    assert got.shape == ref[0].shape
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n_fft)


@pytest.mark.parametrize("shape", [(2, 16, 16), (1, 4096, 16), (3, 16, 2048), (2, 512, 1024), (1, 128, 64),
                                   (2, 64, 4096), (1, 512, 4096)])
def test_fft2_complex_and_inverse(shape):
    # (16, 16) and (128, 64) take the single-pass small-image kernel; complex input routes the
    # others to the two single-axis passes, and the two-pass 2-D kernels are checked directly
    # (4096-wide rows: pass 1 exchanges its 8 rows through LDS one plane at a time)
    from trnfft_amd.fft_core import execute_fft2

    rng = np.random.default_rng(11)
    re = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    im = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    got = trnfft_amd.fft2(ComplexTensor(re.cuda(), im.cuda()))
    ref = oracle.fft2((re, im))
    n = shape[-1] * shape[-2]
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n)
    direct = execute_fft2(re.cuda(), im.cuda(), False)
    assert rel_l2(direct.real, direct.imag, *ref) <= tol_pow2(n)
    back = trnfft_amd.ifftn(got, dim=(-2, -1))
    ref_back = oracle.ifftn(ref, dim=(-2, -1))
    assert rel_l2(back.real, back.imag, *ref_back) <= tol_pow2(n)
    assert rel_l2(back.real, back.imag, re, im) <= 2 * tol_pow2(n)


@pytest.mark.parametrize("shape", [(2, 16, 16), (1, 4096, 16), (3, 16, 2048), (2, 512, 1024), (1, 128, 64), (2, 64, 32),
                                   (2, 64, 4096), (1, 256, 4096),
                                   # 16 row groups (H = 16 x HR): HR = 64, 256 and 128
                                   (2, 1024, 1024), (1, 4096, 2048), (1, 2048, 1024), (1, 1024, 2048)])
def test_fft2_real_input(shape):
    # real input.  Two-pass shapes: pass 1 writes columns 0..W/2, pass 2 completes W/2+1..W-1
    # from the 2-D Hermitian symmetry; small images are transformed whole.  Forward and inverse
    # (ifftn of a real array) against the oracle
    rng = np.random.default_rng(13)
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    n = shape[-1] * shape[-2]
    got = trnfft_amd.fft2(x.cuda())
    ref = oracle.fft2(x)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n)
    inv = trnfft_amd.ifftn(x.cuda(), dim=(-2, -1))
    ref_inv = oracle.ifftn(x, dim=(-2, -1))
    assert rel_l2(inv.real, inv.imag, *ref_inv) <= tol_pow2(n)
    g = torch.complex(got.real, got.imag).cpu()
    mirrored = torch.conj(torch.roll(torch.flip(g, dims=(-2, -1)), shifts=(1, 1), dims=(-2, -1))).resolve_conj()
    w = shape[-1]
    if fft2_small_ok(shape[-2], shape[-1]):
        # computed whole: Hermitian to rounding
        assert rel_l2(g.real, g.imag, mirrored.real, mirrored.imag) <= tol_pow2(n)
    else:
        # the completed half is the conjugate reflection of the computed one, exactly
        assert torch.equal(g[..., w // 2 + 1:], mirrored[..., w // 2 + 1:])


# Real-input shapes whose pass 2 takes runs of column tiles with whole-line mirror stores (a
# workgroup walks its tiles downwards, carrying each tile's first column into the next tile's mirror
# line), chosen for the run layouts: 1 run per group of 3 tiles (40 x 256^2, 64-column tiles), 2 runs
# of 4 + 5 tiles (16 x 1024^2), 4 runs of 4-5 of 17 tiles (8 x 2048 x 1024, 32-column tiles), 6
# uneven runs of 33 tiles (6 x 2048^2), 7 runs of 65 tiles (5 x 2048 x 4096).  Against numpy's
# float64 FFT (forward and inverse), and the mirrored half equal to the conjugate reflection of the
# computed one bit for bit, at run boundaries too.
@pytest.mark.parametrize("shape", [(40, 256, 256), (16, 1024, 1024), (8, 2048, 1024), (6, 2048, 2048),
                                   (5, 2048, 4096)])
def test_fft2_real_input_tile_runs(shape):
    rng = np.random.default_rng(29)
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    n = shape[-1] * shape[-2]
    ref = np.fft.fft2(x.double().numpy())
    got = trnfft_amd.fft2(x.cuda())
    assert rel_l2(got.real, got.imag, ref.real, ref.imag) <= tol_pow2(n), shape
    g = torch.complex(got.real, got.imag).cpu()
    del got
    mirrored = torch.conj(torch.roll(torch.flip(g, dims=(-2, -1)), shifts=(1, 1), dims=(-2, -1))).resolve_conj()
    w = shape[-1]
    assert torch.equal(g[..., w // 2 + 1:], mirrored[..., w // 2 + 1:]), shape
    del g, mirrored
    inv = trnfft_amd.ifftn(x.cuda(), dim=(-2, -1))
    ref_inv = np.fft.ifft2(x.double().numpy())
    assert rel_l2(inv.real, inv.imag, ref_inv.real, ref_inv.imag) <= tol_pow2(n), shape


# every image shape of the single-pass kernel's families (4096 elements per workgroup below
# 4096, one image at 4096..16384), ragged batches that leave a partial workgroup, complex and
# real input, forward and inverse
@pytest.mark.parametrize("shape", [(37, 4, 4), (5, 4, 64), (3, 64, 4), (19, 16, 16), (7, 8, 32), (3, 32, 64),
                                   (2, 64, 64), (3, 8, 1024), (2, 1024, 8), (3, 128, 128), (2, 16, 1024),
                                   (2, 1024, 16), (1, 256, 64)])
def test_fft2_small_images(shape):
    assert fft2_small_ok(shape[-2], shape[-1])
    rng = np.random.default_rng(21)
    re = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    im = torch.from_numpy(rng.standard_normal(shape).astype(np.float32))
    n = shape[-1] * shape[-2]
    got = trnfft_amd.fft2(ComplexTensor(re.cuda(), im.cuda()))
    ref = oracle.fft2((re, im))
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n), shape
    back = trnfft_amd.ifftn(got, dim=(-2, -1))
    assert rel_l2(back.real, back.imag, re, im) <= 2 * tol_pow2(n), shape
    x = np.fft.fft2(re.double().numpy())
    gr = trnfft_amd.fft2(re.cuda())
    assert rel_l2(gr.real, gr.imag, x.real, x.imag) <= tol_pow2(n), shape


def test_fft2_small_image_known_answers():
    # impulse -> all ones; constant -> n at DC; a pure 2-D tone -> one bin
    h, w = 16, 32
    x = torch.zeros(h, w)
    x[0, 0] = 1.0
    y = trnfft_amd.fft2(x.cuda())
    assert torch.allclose(y.real.cpu(), torch.ones(h, w)) and torch.allclose(y.imag.cpu(), torch.zeros(h, w))
    y = trnfft_amd.fft2(torch.ones(h, w).cuda())
    ref = torch.zeros(h, w)
    ref[0, 0] = h * w
    assert torch.allclose(y.real.cpu(), ref, atol=1e-4) and torch.allclose(y.imag.cpu(), torch.zeros(h, w), atol=1e-4)
    r = torch.arange(h).double()[:, None]
    c = torch.arange(w).double()[None, :]
    ang = 2 * math.pi * (3 * r / h + 5 * c / w)
    z = trnfft_amd.fft2(ComplexTensor(torch.cos(ang).float().cuda(), torch.sin(ang).float().cuda()))
    ref = torch.zeros(h, w)
    ref[3, 5] = h * w
    assert torch.allclose(z.real.cpu(), ref, atol=1e-3) and torch.allclose(z.imag.cpu(), torch.zeros(h, w), atol=1e-3)


def test_empty_batches():
    # zero rows / images / outer blocks: every entry point returns an empty result of the right
    # shape without launching anything (torch.fft gives the same shapes)
    def c(shape):
        return ComplexTensor(torch.zeros(shape, device="cuda"), torch.zeros(shape, device="cuda"))

    assert tuple(trnfft_amd.fft(c((0, 1024))).shape) == (0, 1024)
    assert tuple(trnfft_amd.ifft(c((0, 1000))).shape) == (0, 1000)              # Bluestein
    assert tuple(trnfft_amd.fft(c((0, 1 << 20))).shape) == (0, 1 << 20)         # four-step
    assert tuple(trnfft_amd.rfft(torch.zeros(0, 64, device="cuda")).shape) == (0, 33)
    assert tuple(trnfft_amd.irfft(c((0, 33))).shape) == (0, 64)
    assert tuple(trnfft_amd.fftn(c((0, 8192, 16)), dim=(1,)).shape) == (0, 8192, 16)  # strided multi-pass
    assert tuple(trnfft_amd.fftn(c((0, 64, 5)), dim=(1,)).shape) == (0, 64, 5)
    assert tuple(trnfft_amd.fft2(torch.zeros(0, 64, 64, device="cuda")).shape) == (0, 64, 64)
    assert tuple(trnfft_amd.fft2(c((0, 256, 512))).shape) == (0, 256, 512)


def test_views_are_transformed_as_their_values():
    # expanded (stride 0), strided-slice, transposed and offset views: the entry points copy them
    # to contiguous fp32 first, so each result equals the transform of the materialised values
    g = torch.Generator(device="cuda").manual_seed(3)
    base = torch.randn(64, 2048, device="cuda", generator=g)
    views = [base[:1].expand(32, 2048), base[:, ::2], base[:, :1024].t(), base[5:37, 7:1007], base[:, 1:]]
    import oracle

    # against the oracle: the 1000-point view is a Bluestein length, where the reference operator's
    # fp32 chirp sits ~1.2e-4 from the exact DFT
    for v in views:
        assert not v.is_contiguous()
        vc = v.cpu().contiguous()
        got = trnfft_amd.fft(v)
        ref = oracle.fft_core(vc, torch.zeros_like(vc), False)
        assert rel_l2(got.real, got.imag, *ref) <= tol_bluestein(v.shape[-1]), tuple(v.shape)
        got = trnfft_amd.rfft(v)
        assert rel_l2(got.real, got.imag, *oracle.rfft(vc)) <= tol_bluestein(v.shape[-1]), tuple(v.shape)
    z = ComplexTensor(base[:, ::2], base[:, 1::2])
    got = trnfft_amd.ifft(z)
    ref = np.fft.ifft(base[:, ::2].cpu().double().numpy() + 1j * base[:, 1::2].cpu().double().numpy(), axis=-1)
    assert rel_l2(got.real, got.imag, ref.real, ref.imag) <= tol_pow2(1024)


def test_one_plan_on_two_streams_at_once():
    # the cached plans (four-step with its workspace, split Bluestein, STFT) driven from two
    # streams concurrently give the same results as one stream at a time
    g = torch.Generator(device="cuda").manual_seed(4)
    shapes = [(8, 1 << 18), (3, 40000), (64, 1024)]
    xs = [[ComplexTensor(torch.randn(s, device="cuda", generator=g), torch.randn(s, device="cuda", generator=g))
           for _ in range(2)] for s in shapes]
    sig = [torch.randn(16, 50000, device="cuda", generator=g) for _ in range(2)]
    serial = [[trnfft_amd.fft(x) for x in pair] for pair in xs]
    serial_s = [trnfft_amd.stft(s, 512, hop_length=128) for s in sig]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[None] * len(shapes) for _ in range(2)]
    outs_s = [None, None]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rep in range(3):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                for j in range(len(shapes)):
                    outs[i][j] = trnfft_amd.fft(xs[j][i])
                outs_s[i] = trnfft_amd.stft(sig[i], 512, hop_length=128)
        torch.cuda.synchronize()
        for i in range(2):
            for j in range(len(shapes)):
                assert torch.equal(outs[i][j].real, serial[j][i].real) and torch.equal(outs[i][j].imag, serial[j][i].imag)
            assert torch.equal(outs_s[i].real, serial_s[i].real) and torch.equal(outs_s[i].imag, serial_s[i].imag)
