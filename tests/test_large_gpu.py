"""Batches past 2^31 elements per plane (64-bit element offsets): the batched c2c kernel on a ragged
batch and the frames-major STFT, first and last rows / signals against float64 numpy / torch.stft
at the same bounds as the fixed-shape tests.  About 35 GB of device memory at peak."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnfft_amd
from conftest import rel_l2, tol_pow2
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


def test_stft_frames_major_past_2_31_output_elements():
    _need(40)
    n_fft, hop, length = 512, 256, 160000
    batch = 13500  # 13500 * 626 * 257 > 2^31 bins per plane
    g = torch.Generator(device="cuda").manual_seed(32)
    x = torch.randn(batch, length, device="cuda", generator=g)
    w = torch.hann_window(n_fft, device="cuda")
    s = trnfft_amd.stft(x, n_fft, hop_length=hop, window=w)
    torch.cuda.synchronize()
    assert s.real.numel() > 2**31
    for b in (0, batch - 1):
        ref = torch.stft(x[b].double().cpu(), n_fft, hop_length=hop, window=w.double().cpu(), center=True,
                         pad_mode="reflect", onesided=True, return_complex=True)
        assert rel_l2(s.real[b], s.imag[b], ref.real, ref.imag) < tol_pow2(n_fft)
    del x, s
    torch.cuda.empty_cache()
