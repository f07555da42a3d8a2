"""GPU parity of the real-row kernels (rfft as r2c, irfft as c2r) against the oracle's restatement
of trnfft/api.py:38-68 (full complex transform + slice; Hermitian completion + real part)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, tol_pow2
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu

# (n, batch): batches not a multiple of the rows per workgroup run the guarded kernel variant over
# the whole grid, whose last workgroup is partial (n = 8, 16 run one row per thread with 256-row
# staging tiles: 300, 257, 1000 rows leave a partial tile after full ones; n = 32, 64 and 128 move
# their bins through LDS as one run per workgroup of 64 / 32 / 16 rows: 65, 513 and 77 rows end
# in a partial run, 1024 rows are whole runs only)
CASES = [(4, 300), (4, 1024), (8, 257), (16, 33), (16, 1000), (32, 65), (32, 1024), (64, 7), (64, 513), (64, 1024),
         (128, 5), (128, 77), (128, 1024), (256, 3), (512, 3), (1024, 5), (2048, 3), (4096, 2), (8192, 2), (16384, 1),
         (32768, 2)]


@pytest.mark.parametrize("n,batch", CASES)
def test_rfft_matches_reference(n, batch):
    g = torch.Generator().manual_seed(42)
    x = torch.randn(batch, n, generator=g)
    got = trnfft_amd.rfft(x.cuda())
    assert got.shape == (batch, n // 2 + 1)
    ref = oracle.rfft(x)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n)
    # independent pin: numpy's float64 rfft
    e = np.fft.rfft(x.double().numpy(), axis=-1)
    assert rel_l2(got.real, got.imag, torch.from_numpy(e.real), torch.from_numpy(e.imag)) <= tol_pow2(n)


@pytest.mark.parametrize("n,batch", CASES)
def test_irfft_matches_reference(n, batch):
    g = torch.Generator().manual_seed(7)
    h = n // 2 + 1
    # arbitrary bins, including imaginary parts at bins 0 and n/2, which the reference's real
    # part of the Hermitian-completed inverse ignores
    re = torch.randn(batch, h, generator=g)
    im = torch.randn(batch, h, generator=g)
    got = trnfft_amd.irfft(ComplexTensor(re.cuda(), im.cuda()))
    assert got.shape == (batch, n)
    ref = oracle.irfft((re, im))
    z = torch.zeros_like(ref)
    assert rel_l2(got, torch.zeros_like(got), ref, z) <= tol_pow2(n)
    # independent pin: numpy's float64 c2r (which also ignores Im of bins 0 and n/2)
    e = torch.from_numpy(np.fft.irfft(re.double().numpy() + 1j * im.double().numpy(), n=n, axis=-1))
    assert rel_l2(got, torch.zeros_like(got), e, torch.zeros_like(e)) <= tol_pow2(n)


def test_real_roundtrip_and_leading_dims():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 3, 1024, generator=g)
    X = trnfft_amd.rfft(x.cuda())
    assert X.shape == (2, 3, 513)
    back = trnfft_amd.irfft(X)
    assert back.shape == (2, 3, 1024)
    assert rel_l2(back, torch.zeros_like(back), x, torch.zeros_like(x)) <= 2 * tol_pow2(1024)


def test_rfft_unaligned_view():
    # a contiguous view starting 4 bytes into its storage: the host copies it to an aligned buffer
    g = torch.Generator().manual_seed(5)
    flat = torch.randn(1 + 4 * 256, generator=g).cuda()
    x = flat[1:].view(4, 256)
    assert x.data_ptr() % 8 != 0
    got = trnfft_amd.rfft(x)
    ref = oracle.rfft(x.cpu())
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(256)


def test_rfft_closed_forms():
    n = 64
    # impulse -> all-ones spectrum; constant -> n at bin 0; cosine at bin 5 -> n/2 at bin 5
    t = torch.arange(n, dtype=torch.float32)
    x = torch.stack([torch.nn.functional.one_hot(torch.tensor(0), n).float(), torch.ones(n),
                     torch.cos(2 * torch.pi * 5 * t / n)])
    X = trnfft_amd.rfft(x.cuda())
    re, im = X.real.cpu(), X.imag.cpu()
    torch.testing.assert_close(re[0], torch.ones(n // 2 + 1), atol=1e-6, rtol=0)
    expect = torch.zeros(n // 2 + 1)
    expect[0] = n
    torch.testing.assert_close(re[1], expect, atol=1e-5, rtol=0)
    expect = torch.zeros(n // 2 + 1)
    expect[5] = n / 2
    torch.testing.assert_close(re[2], expect, atol=1e-4, rtol=0)
    torch.testing.assert_close(im, torch.zeros_like(im), atol=1e-4, rtol=0)


def test_irfft_other_n_keeps_reference_semantics():
    # n other than 2*(bins-1) keeps the reference's completion (no c2r kernel)
    g = torch.Generator().manual_seed(9)
    re, im = torch.randn(3, 9, generator=g), torch.randn(3, 9, generator=g)
    for n in (12, 17):
        got = trnfft_amd.irfft(ComplexTensor(re.cuda(), im.cuda()), n=n)
        ref = oracle.irfft((re, im), n=n)
        assert got.shape == ref.shape
        torch.testing.assert_close(got.cpu(), ref, atol=1e-5, rtol=1e-4)
