"""Batches past 2^31 elements per plane (64-bit element offsets) through every kernel family: the
batched c2c kernel on a ragged batch, r2c / c2r, the fused Bluestein kernel, the four-step passes,
the two-pass real fft2, a strided axis, the frames-major STFT (power-of-two and Bluestein n_fft),
the inverse STFT and the complex GEMM.  First and last rows (signals, images) against float64
numpy / torch.stft, the oracle for Bluestein and the GEMM, or the round trip, at the bounds of the
fixed-shape tests.  Up to ~50 GB of device memory per test, freed after each."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnfft_amd
from conftest import rel_l2, tol_bluestein, tol_pow2
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu


def _need(gib: float):
    free, _ = torch.cuda.mem_get_info()
    if free < gib * 2**30:
        pytest.skip(f"needs {gib} GiB of free device memory")


def test_c2c_batch_past_2_31_elements():
    _need(40)
    n = 1024
    rows = (1 << 21) + 3  # 2^31 + 3072 elements per plane; ragged for the 4-row workgroups
    g = torch.Generator(device="cuda").manual_seed(31)
    re = torch.randn(rows, n, device="cuda", generator=g)
    im = torch.randn(rows, n, device="cuda", generator=g)
    assert re.numel() > 2**31
    out = trnfft_amd.fft(ComplexTensor(re, im))
    torch.cuda.synchronize()
    for sl in (slice(0, 4), slice(rows - 5, rows)):
        x = re[sl].double().cpu().numpy() + 1j * im[sl].double().cpu().numpy()
        ref = np.fft.fft(x, axis=-1)
        assert rel_l2(out.real[sl], out.imag[sl], ref.real, ref.imag) < tol_pow2(n)
    del re, im, out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("frames_major", [False, True])
def test_stft_past_2_31_output_elements(frames_major):
    # the reference's bins-major layout (whole-line kernel) and the frames-major opt-in
    _need(40)
    n_fft, hop, length = 512, 256, 160000
    batch = 13500  # 13500 * 626 * 257 > 2^31 bins per plane
    g = torch.Generator(device="cuda").manual_seed(32)
    x = torch.randn(batch, length, device="cuda", generator=g)
    w = torch.hann_window(n_fft, device="cuda")
    s = trnfft_amd.stft(x, n_fft, hop_length=hop, window=w, frames_major=frames_major)
    torch.cuda.synchronize()
    assert s.real.numel() > 2**31
    assert s.real.is_contiguous() != frames_major
    for b in (0, batch - 1):
        ref = torch.stft(x[b].double().cpu(), n_fft, hop_length=hop, window=w.double().cpu(), center=True,
                         pad_mode="reflect", onesided=True, return_complex=True)
        assert rel_l2(s.real[b], s.imag[b], ref.real, ref.imag) < tol_pow2(n_fft)
    del x, s
    torch.cuda.empty_cache()


def test_rfft_irfft_batch_past_2_31_elements():
    _need(40)
    n = 1024
    rows = (1 << 21) + 3
    g = torch.Generator(device="cuda").manual_seed(33)
    x = torch.randn(rows, n, device="cuda", generator=g)
    assert x.numel() > 2**31
    X = trnfft_amd.rfft(x)
    y = trnfft_amd.irfft(X, n)
    torch.cuda.synchronize()
    for sl in (slice(0, 4), slice(rows - 5, rows)):
        ref = np.fft.rfft(x[sl].double().cpu().numpy(), axis=-1)
        assert rel_l2(X.real[sl], X.imag[sl], ref.real, ref.imag) < tol_pow2(n)
        xs = x[sl].double().cpu().numpy()
        assert rel_l2(y[sl], np.zeros_like(xs), xs, np.zeros_like(xs)) < 2 * tol_pow2(n)
    del x, X, y
    torch.cuda.empty_cache()


def test_bluestein_fused_batch_past_2_31_elements():
    import oracle

    _need(48)
    n = 1000
    rows = (1 << 31) // n + 5
    g = torch.Generator(device="cuda").manual_seed(34)
    re = torch.randn(rows, n, device="cuda", generator=g)
    im = torch.randn(rows, n, device="cuda", generator=g)
    assert re.numel() > 2**31
    out = trnfft_amd.fft(ComplexTensor(re, im))
    torch.cuda.synchronize()
    for sl in (slice(0, 3), slice(rows - 3, rows)):
        ref = oracle.fft_core(re[sl].cpu(), im[sl].cpu(), False)
        assert rel_l2(out.real[sl], out.imag[sl], *ref) < tol_bluestein(n)
    del re, im, out
    torch.cuda.empty_cache()


def test_fourstep_batch_past_2_31_elements():
    _need(64)
    n = 1 << 20
    rows = 2049
    g = torch.Generator(device="cuda").manual_seed(35)
    re = torch.randn(rows, n, device="cuda", generator=g)
    im = torch.randn(rows, n, device="cuda", generator=g)
    assert re.numel() > 2**31
    out = trnfft_amd.fft(ComplexTensor(re, im))
    torch.cuda.synchronize()
    for r in (0, rows - 1):
        x = re[r].double().cpu().numpy() + 1j * im[r].double().cpu().numpy()
        ref = np.fft.fft(x)
        assert rel_l2(out.real[r], out.imag[r], ref.real, ref.imag) < tol_pow2(n)
    del re, im, out
    torch.cuda.empty_cache()


def test_fft2_real_images_past_2_31_elements():
    _need(48)
    h = w = 2048
    imgs = (1 << 31) // (h * w) + 1  # 513 images
    g = torch.Generator(device="cuda").manual_seed(36)
    x = torch.rand(imgs, h, w, device="cuda", generator=g)
    assert x.numel() > 2**31
    out = trnfft_amd.fft2(x)
    torch.cuda.synchronize()
    for i in (0, imgs - 1):
        ref = np.fft.fft2(x[i].double().cpu().numpy())
        assert rel_l2(out.real[i], out.imag[i], ref.real, ref.imag) < 1e-6 * 22
    del x, out
    torch.cuda.empty_cache()


def test_istft_output_past_2_31_samples():
    _need(48)
    n_fft, hop, length = 512, 256, 160000
    batch = 13500  # 13500 * 160000 > 2^31 samples
    g = torch.Generator(device="cuda").manual_seed(37)
    x = torch.randn(batch, length, device="cuda", generator=g)
    w = torch.hann_window(n_fft, device="cuda")
    s = trnfft_amd.stft(x, n_fft, hop_length=hop, window=w)
    y = trnfft_amd.istft(s, n_fft, hop_length=hop, window=w, length=length)
    torch.cuda.synchronize()
    assert y.numel() > 2**31
    for b in (0, batch - 1):
        xs = x[b].double().cpu().numpy()
        assert rel_l2(y[b], np.zeros_like(xs), xs, np.zeros_like(xs)) < 4 * tol_pow2(n_fft)
    del x, s, y
    torch.cuda.empty_cache()


def test_strided_axis_past_2_31_elements():
    _need(48)
    b, n, stride = 2049, 1024, 1024  # transform along dim 1: 2^31 + 2^20 elements
    g = torch.Generator(device="cuda").manual_seed(38)
    re = torch.randn(b, n, stride, device="cuda", generator=g)
    im = torch.randn(b, n, stride, device="cuda", generator=g)
    assert re.numel() > 2**31
    out = trnfft_amd.fftn(ComplexTensor(re, im), dim=(1,))
    torch.cuda.synchronize()
    for i, cols in ((0, slice(0, 5)), (b - 1, slice(stride - 5, stride))):
        x = re[i, :, cols].double().cpu().numpy() + 1j * im[i, :, cols].double().cpu().numpy()
        ref = np.fft.fft(x, axis=0)
        assert rel_l2(out.real[i, :, cols], out.imag[i, :, cols], ref.real, ref.imag) < tol_pow2(n)
    del re, im, out
    torch.cuda.empty_cache()


def test_stft_bluestein_past_2_31_output_elements():
    import oracle

    _need(40)
    n_fft, hop, length = 400, 160, 160000
    batch = 13500  # 13500 * 1001 * 201 > 2^31 bins per plane
    g = torch.Generator(device="cuda").manual_seed(39)
    x = torch.randn(batch, length, device="cuda", generator=g)
    s = trnfft_amd.stft(x, n_fft, hop_length=hop)
    torch.cuda.synchronize()
    assert s.real.numel() > 2**31
    for i in (0, batch - 1):
        rr, ri = oracle.stft(x[i:i + 1].cpu(), n_fft=n_fft, hop_length=hop)
        assert rel_l2(s.real[i:i + 1], s.imag[i:i + 1], rr, ri) < tol_bluestein(n_fft)
    del x, s
    torch.cuda.empty_cache()


def test_complex_matmul_rows_past_2_31_elements():
    import oracle

    _need(40)
    m, k, n = (1 << 21) + 5, 1024, 64  # A has 2^31 + 5120 elements per plane
    g = torch.Generator(device="cuda").manual_seed(40)
    ar = torch.randn(m, k, device="cuda", generator=g)
    ai = torch.randn(m, k, device="cuda", generator=g)
    br = torch.randn(k, n, device="cuda", generator=g)
    bi = torch.randn(k, n, device="cuda", generator=g)
    assert ar.numel() > 2**31
    out = trnfft_amd.complex_matmul(ComplexTensor(ar, ai), ComplexTensor(br, bi))
    torch.cuda.synchronize()
    for sl in (slice(0, 4), slice(m - 4, m)):
        rr, ri = oracle.complex_matmul((ar[sl].double().cpu(), ai[sl].double().cpu()),
                                       (br.double().cpu(), bi.double().cpu()))
        assert rel_l2(out.real[sl], out.imag[sl], rr, ri) < 1e-5
    del ar, ai, br, bi, out
    torch.cuda.empty_cache()
