"""Gradients of the HIP path (adjoints on the native kernels) against torch autograd through
float64 references: torch.fft / torch.stft / real matmuls on the CPU, and the oracle's
restatement of the reference's own differentiable pytorch path (trnfft/api.py, fft_core.py,
nn.py:33-49) where that is cheap.  Mirrors trnfft's tests/test_nn.py:62-98 (gradients exist
and are finite) and checks their values."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, tol_bluestein
from trnfft_amd import ComplexTensor
from trnfft_amd.nn import ComplexLinear

pytestmark = pytest.mark.gpu

TOL = 1e-5  # fp32 kernels vs fp64 reference, relative L2 of the gradient


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _leaf(t):
    return t.clone().cuda().requires_grad_(True)


def _cotangent(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64), torch.randn(*shape, generator=g, dtype=torch.float64)


@pytest.mark.parametrize("n,batch,inverse", [(1024, 8, False), (1024, 8, True), (1000, 4, False), (4099, 2, True),
                                             (1 << 20, 1, False), (16, 5, True)])
def test_c2c_gradient(n, batch, inverse):
    g = torch.Generator().manual_seed(n)
    xr, xi = torch.randn(batch, n, generator=g), torch.randn(batch, n, generator=g)
    cr, ci = _cotangent((batch, n), 1)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = (trnfft_amd.ifft if inverse else trnfft_amd.fft)(ComplexTensor(a_r, a_i))
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    if n & (n - 1) == 0:
        r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
        z = (torch.fft.ifft if inverse else torch.fft.fft)(torch.complex(r_r, r_i))
        (z.real * cr + z.imag * ci).sum().backward()
        assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL
    else:
        # Bluestein: the reference's operator carries its fp32 chirp (~1e-4 off the exact DFT),
        # so the gradient is pinned against autograd through the oracle's restatement of it
        r_r, r_i = xr.clone().requires_grad_(True), xi.clone().requires_grad_(True)
        z_r, z_i = oracle.fft_core(r_r, r_i, inverse)
        (z_r * cr.float() + z_i * ci.float()).sum().backward()
        assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= tol_bluestein(n)


def test_real_input_fft_gradient_matches_reference_test():
    # trnfft tests/test_nn.py:77-86, plus the value
    x_re = torch.randn(16, requires_grad=True, device="cuda")
    X = trnfft_amd.fft(ComplexTensor(x_re))
    (X.real**2 + X.imag**2).sum().backward()
    assert x_re.grad is not None and torch.all(torch.isfinite(x_re.grad))
    # |FFT x|^2 summed = n |x|^2 (Parseval) -> gradient 2 n x
    torch.testing.assert_close(x_re.grad, 2 * 16 * x_re.detach(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n", [8, 1024, 4096, 1000])
def test_rfft_gradient(n):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, n, generator=g)
    h = n // 2 + 1
    cr, ci = _cotangent((6, h), 2)
    a = _leaf(x)
    y = trnfft_amd.rfft(a)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    if n & (n - 1) == 0:
        r = x.double().requires_grad_(True)
        z = torch.fft.rfft(r)
        (z.real * cr + z.imag * ci).sum().backward()
        assert _rel(a.grad, r.grad) <= TOL
    else:
        r = x.clone().requires_grad_(True)
        z_r, z_i = oracle.rfft(r)
        (z_r * cr.float() + z_i * ci.float()).sum().backward()
        assert _rel(a.grad, r.grad) <= tol_bluestein(n)


@pytest.mark.parametrize("n", [8, 1024, 8192])
def test_irfft_gradient(n):
    g = torch.Generator().manual_seed(4)
    h = n // 2 + 1
    xr, xi = torch.randn(3, h, generator=g), torch.randn(3, h, generator=g)
    c, _ = _cotangent((3, n), 5)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = trnfft_amd.irfft(ComplexTensor(a_r, a_i))
    (y * c.float().cuda()).sum().backward()
    # the reference's own composition (Hermitian completion + inverse c2c + real part), in fp64
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    full_r = torch.cat([r_r, r_r[..., 1:h - 1].flip(-1)], -1)
    full_i = torch.cat([r_i, -r_i[..., 1:h - 1].flip(-1)], -1)
    z = torch.fft.ifft(torch.complex(full_r, full_i)).real
    (z * c).sum().backward()
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL
    assert torch.count_nonzero(a_i.grad[:, 0]) == 0 and torch.count_nonzero(a_i.grad[:, -1]) == 0


def test_irfft_general_n_gradient_via_oracle():
    # n != 2*(bins-1): the composition path; the oracle's restatement is differentiable too
    g = torch.Generator().manual_seed(6)
    xr, xi = torch.randn(2, 9, generator=g), torch.randn(2, 9, generator=g)
    c, _ = _cotangent((2, 12), 7)
    a_r, a_i = _leaf(xr), _leaf(xi)
    (trnfft_amd.irfft(ComplexTensor(a_r, a_i), n=12) * c.float().cuda()).sum().backward()
    r_r, r_i = xr.clone().requires_grad_(True), xi.clone().requires_grad_(True)
    (oracle.irfft((r_r, r_i), n=12) * c.float()).sum().backward()
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= 1e-5


@pytest.mark.parametrize("shape,real_in", [((2, 64, 128), False), ((2, 64, 128), True), ((3, 16, 2048), False),
                                           ((1, 512, 256), True), ((1, 64, 4096), True)])
def test_fft2_gradient(shape, real_in):
    g = torch.Generator().manual_seed(8)
    xr = torch.randn(*shape, generator=g)
    xi = torch.randn(*shape, generator=g)
    cr, ci = _cotangent(shape, 9)
    a_r = _leaf(xr)
    a_i = None if real_in else _leaf(xi)
    y = trnfft_amd.fft2(a_r if real_in else ComplexTensor(a_r, a_i))
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r_r = xr.double().requires_grad_(True)
    r_i = None if real_in else xi.double().requires_grad_(True)
    z = torch.fft.fft2(r_r if real_in else torch.complex(r_r, r_i))
    (z.real * cr + z.imag * ci).sum().backward()
    if real_in:
        assert _rel(a_r.grad, r_r.grad) <= TOL
    else:
        assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL


def test_strided_axis_gradient():
    g = torch.Generator().manual_seed(10)
    xr, xi = torch.randn(4, 256, 24, generator=g), torch.randn(4, 256, 24, generator=g)
    cr, ci = _cotangent((4, 256, 24), 11)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = trnfft_amd.ifftn(ComplexTensor(a_r, a_i), dim=(1,))
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    z = torch.fft.ifftn(torch.complex(r_r, r_i), dim=(1,))
    (z.real * cr + z.imag * ci).sum().backward()
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL


def test_strided_non_pow2_axis_gradient():
    # a Bluestein length down a strided axis: forward and adjoint both on the strided kernel
    g = torch.Generator().manual_seed(14)
    xr, xi = torch.randn(3, 100, 24, generator=g), torch.randn(3, 100, 24, generator=g)
    cr, ci = _cotangent((3, 100, 24), 15)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = trnfft_amd.fftn(ComplexTensor(a_r, a_i), dim=(1,))
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    z = torch.fft.fftn(torch.complex(r_r, r_i), dim=(1,))
    (z.real * cr + z.imag * ci).sum().backward()
    # the reference's fp32 chirp keeps Bluestein results ~1e-5 from exact
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= 1e-4


@pytest.mark.parametrize("shape", [(2, 8192, 6), (1, 1 << 21, 8)])
def test_strided_long_axis_gradient(shape):
    # power-of-two axes above 4096 down a strided dimension (the two- and three-pass strided
    # four-step through a workspace): forward and adjoint both on it
    from trnfft_amd.fft_core import strided_ok

    assert strided_ok(shape[1], shape[2])
    g = torch.Generator().manual_seed(16)
    xr, xi = torch.randn(*shape, generator=g), torch.randn(*shape, generator=g)
    cr, ci = _cotangent(shape, 17)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = trnfft_amd.fftn(ComplexTensor(a_r, a_i), dim=(1,))
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    z = torch.fft.fftn(torch.complex(r_r, r_i), dim=(1,))
    (z.real * cr + z.imag * ci).sum().backward()
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= 1e-6 * math.log2(shape[1])


@pytest.mark.parametrize("n_fft,hop,center,normalized,onesided", [(512, 256, True, False, True), (256, 64, True, True, True),
                                                                   (128, 100, False, False, True), (64, 16, True, False, False)])
def test_stft_gradient(n_fft, hop, center, normalized, onesided):
    g = torch.Generator().manual_seed(12)
    x = torch.randn(3, 4000, generator=g)
    w = torch.hann_window(n_fft) + 0.1 * torch.rand(n_fft, generator=g)
    a = _leaf(x)
    aw = _leaf(w)
    y = trnfft_amd.stft(a, n_fft, hop_length=hop, window=aw, center=center, normalized=normalized, onesided=onesided)
    cr, ci = _cotangent(tuple(y.shape), 13)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r = x.double().requires_grad_(True)
    rw = w.double().requires_grad_(True)
    z = torch.stft(r, n_fft, hop_length=hop, window=rw, center=center, pad_mode="reflect", normalized=normalized,
                   onesided=onesided, return_complex=True)
    assert tuple(z.shape) == tuple(y.shape)
    (z.real * cr + z.imag * ci).sum().backward()
    assert _rel(a.grad, r.grad) <= TOL
    assert _rel(aw.grad, rw.grad) <= TOL


@pytest.mark.parametrize("n_fft,hop,center,normalized,shape", [
    (512, 256, True, False, (3, 4000)),
    (512, 128, True, True, (2, 3, 3000)),     # leading dims
    (256, 100, False, False, (2, 5000)),      # no centre padding; samples past the last frame
    (16, 4, True, False, (2, 301)),
    (1024, 256, True, False, (1, 9000)),
    (2048, 512, False, True, (2, 10000)),
    (4096, 1024, True, False, (1, 20000)),
    (512, 600, True, False, (2, 3000)),       # hop > n_fft: gaps between frames
    (512, 130, True, False, (2, 5000)),       # a hop that is not a multiple of 4: one sample per thread
    (512, 128, False, False, (2, 5001)),      # a padded length that is not
    (512, 256, True, False, (2, 257)),        # every frame reaches into both reflected edges
])
def test_stft_gradient_fused_backward(n_fft, hop, center, normalized, shape, monkeypatch):
    # window without gradient: the signal gradient is one fused kernel (r2c adjoint per frame,
    # window, overlap-add) plus the reflected-edge fold; against torch.stft in float64
    from trnfft_amd import fft_core

    calls = []
    real = fft_core.execute_stft_backward

    def counted(*args, **kw):
        out = real(*args, **kw)
        calls.append(out is not None)
        return out

    monkeypatch.setattr(fft_core, "execute_stft_backward", counted)
    g = torch.Generator().manual_seed(n_fft + hop)
    x = torch.randn(*shape, generator=g)
    w = torch.hann_window(n_fft) + 0.1 * torch.rand(n_fft, generator=g)
    a = _leaf(x)
    y = trnfft_amd.stft(a, n_fft, hop_length=hop, window=w.cuda(), center=center, normalized=normalized)
    cr, ci = _cotangent(tuple(y.shape), 21)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    assert calls == [True]
    r = x.double().requires_grad_(True)
    z = torch.stft(r.reshape(-1, shape[-1]), n_fft, hop_length=hop, window=w.double(), center=center,
                   pad_mode="reflect", normalized=normalized, onesided=True, return_complex=True)
    # (a (1, L) signal comes back without its batch axis, as in the reference)
    z = z.reshape(tuple(y.shape))
    (z.real * cr + z.imag * ci).sum().backward()
    assert _rel(a.grad, r.grad) <= TOL


@pytest.mark.parametrize("n_fft,hop,center,normalized,shape", [
    (400, 160, True, False, (2, 4000)),       # convolution length 768
    (400, 100, False, True, (2, 3, 3000)),
    (12, 4, True, False, (2, 301)),           # 32
    (30, 10, True, False, (2, 500)),          # 64
    (100, 40, True, False, (2, 2000)),        # 192
    (257, 128, True, False, (2, 3000)),       # 512
    (600, 200, True, False, (1, 5000)),       # 1024
    (1000, 300, True, True, (1, 6000)),       # 1536
    (2000, 1000, True, False, (1, 9000)),     # 3072
    (400, 500, True, False, (2, 2000)),       # hop > n_fft
])
def test_stft_gradient_fused_backward_non_pow2(n_fft, hop, center, normalized, shape, monkeypatch):
    # n_fft that is not a power of two, window without gradient: the adjoint Bluestein chain per
    # frame in one kernel, against autograd through the oracle's restatement of the reference's
    # pytorch path (the reference's operator carries its fp32 chirp)
    from trnfft_amd import fft_core

    calls = []
    real = fft_core.execute_stft_backward

    def counted(*args, **kw):
        out = real(*args, **kw)
        calls.append(out is not None)
        return out

    monkeypatch.setattr(fft_core, "execute_stft_backward", counted)
    g = torch.Generator().manual_seed(n_fft + hop)
    x = torch.randn(*shape, generator=g)
    w = torch.hann_window(n_fft) + 0.1 * torch.rand(n_fft, generator=g)
    a = _leaf(x)
    y = trnfft_amd.stft(a, n_fft, hop_length=hop, window=w.cuda(), center=center, normalized=normalized)
    cr, ci = _cotangent(tuple(y.shape), 22)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    assert calls == [True]
    r = x.clone().requires_grad_(True)
    zr, zi = oracle.stft(r, n_fft, hop_length=hop, window=w, center=center, normalized=normalized)
    assert tuple(zr.shape) == tuple(y.shape)
    (zr * cr.float() + zi * ci.float()).sum().backward()
    assert _rel(a.grad, r.grad) <= tol_bluestein(n_fft)


@pytest.mark.parametrize("onesided", [True, False])
def test_stft_gradient_non_pow2_window_and_two_sided_compose(onesided):
    # window gradients (and two-sided spectra) take the composed adjoint, which zero-fills the
    # bins above n/2 before the inverse transform when n_fft is not a power of two
    g = torch.Generator().manual_seed(23)
    x = torch.randn(2, 3000, generator=g)
    w = torch.hann_window(400) + 0.1 * torch.rand(400, generator=g)
    a, aw = _leaf(x), _leaf(w)
    y = trnfft_amd.stft(a, 400, hop_length=160, window=aw, onesided=onesided)
    cr, ci = _cotangent(tuple(y.shape), 24)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r, rw = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    zr, zi = oracle.stft(r, 400, hop_length=160, window=rw, onesided=onesided)
    (zr * cr.float() + zi * ci.float()).sum().backward()
    assert _rel(a.grad, r.grad) <= tol_bluestein(400)
    assert _rel(aw.grad, rw.grad) <= tol_bluestein(400)


def test_stft_gradient_short_hop_composes():
    # a hop the inverse-STFT tile refuses: the backward falls back to the composed adjoint
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 1500, generator=g)
    a = _leaf(x)
    y = trnfft_amd.stft(a, 512, hop_length=2)
    cr, ci = _cotangent(tuple(y.shape), 4)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r = x.double().requires_grad_(True)
    z = torch.stft(r, 512, hop_length=2, window=torch.hann_window(512, dtype=torch.float64), center=True,
                   pad_mode="reflect", onesided=True, return_complex=True)
    (z.real * cr + z.imag * ci).sum().backward()
    assert _rel(a.grad, r.grad) <= TOL


@pytest.mark.parametrize("n_fft,hop,pad_mode", [(8192, 2048, "replicate"), (512, 128, "circular"), (12, 4, "constant")])
def test_stft_gradient_composed_pow2(n_fft, hop, pad_mode):
    # power-of-two n_fft outside the fused kernel's range or with a non-reflect pad: device F.pad +
    # (fused kernel or frame gather + transform kernels), against torch.stft in float64
    g = torch.Generator().manual_seed(15)
    x = torch.randn(2, 20000 if n_fft > 1000 else 900, generator=g)
    a = _leaf(x)
    y = trnfft_amd.stft(a, n_fft, hop_length=hop, pad_mode=pad_mode)
    cr, ci = _cotangent(tuple(y.shape), 16)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r = x.double().requires_grad_(True)
    z = torch.stft(r, n_fft, hop_length=hop, window=torch.hann_window(n_fft, dtype=torch.float64), center=True,
                   pad_mode=pad_mode, onesided=True, return_complex=True)
    assert tuple(z.shape) == tuple(y.shape)
    (z.real * cr + z.imag * ci).sum().backward()
    assert _rel(a.grad, r.grad) <= TOL


def test_stft_gradient_composed_bluestein():
    # n_fft = 400 (Bluestein frames): against autograd through the oracle's restatement of the
    # reference's own pytorch path in fp32 (its fp32 chirp differs from the exact DFT)
    g = torch.Generator().manual_seed(17)
    x = torch.randn(2, 4000, generator=g)
    a = _leaf(x)
    y = trnfft_amd.stft(a, 400, hop_length=160, pad_mode="constant")
    cr, ci = _cotangent(tuple(y.shape), 18)
    (y.real * cr.float().cuda() + y.imag * ci.float().cuda()).sum().backward()
    r = x.clone().requires_grad_(True)
    zr, zi = oracle.stft(r, 400, hop_length=160, pad_mode="constant")
    assert tuple(zr.shape) == tuple(y.shape)
    (zr * cr.float() + zi * ci.float()).sum().backward()
    assert _rel(a.grad, r.grad) <= tol_bluestein(400)


def test_stft_gradient_matches_reference_test():
    # trnfft tests/test_nn.py:88-96
    signal = torch.randn(512, requires_grad=True, device="cuda")
    S = trnfft_amd.stft(signal, n_fft=64, hop_length=32, center=False)
    S.abs().sum().backward()
    assert signal.grad is not None and torch.all(torch.isfinite(signal.grad))


def test_complex_linear_gradients():
    torch.manual_seed(0)
    layer = ComplexLinear(96, 80).cuda()
    with torch.no_grad():
        layer.bias_re.normal_()
        layer.bias_im.normal_()
    g = torch.Generator().manual_seed(14)
    xr, xi = torch.randn(3, 50, 96, generator=g), torch.randn(3, 50, 96, generator=g)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y = layer(ComplexTensor(a_r, a_i))
    (y.real**2 + y.imag**2).sum().backward()
    # the reference's pytorch formula (trnfft/nn.py:46-48) in fp64 on the CPU
    wr = layer.W_re.weight.detach().double().cpu().requires_grad_(True)
    wi = layer.W_im.weight.detach().double().cpu().requires_grad_(True)
    br = layer.bias_re.detach().double().cpu().requires_grad_(True)
    bi = layer.bias_im.detach().double().cpu().requires_grad_(True)
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    re = r_r @ wr.T - r_i @ wi.T + br
    im = r_i @ wr.T + r_r @ wi.T + bi
    (re**2 + im**2).sum().backward()
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL
    assert rel_l2(layer.W_re.weight.grad, layer.W_im.weight.grad, wr.grad, wi.grad) <= TOL
    assert rel_l2(layer.bias_re.grad, layer.bias_im.grad, br.grad, bi.grad) <= TOL


@pytest.mark.parametrize("sa,sb", [((3, 20, 13), (3, 13, 30)), ((3, 20, 13), (13, 30)), ((20, 13), (4, 13, 30)),
                                   ((2, 1, 9, 13), (3, 13, 6)), ((13,), (2, 13, 5)), ((4, 20, 13), (13,))])
def test_complex_matmul_batched_gradients(sa, sb):
    # batched / broadcast products: the adjoints run on the batched kernel and are summed over
    # the axes an operand was broadcast along, as torch.matmul's autograd does
    g = torch.Generator().manual_seed(len(sa) + 3 * len(sb))
    ar, ai = torch.randn(*sa, generator=g), torch.randn(*sa, generator=g)
    br, bi = torch.randn(*sb, generator=g), torch.randn(*sb, generator=g)
    A = torch.complex(ar.double(), ai.double()).requires_grad_(True)
    B = torch.complex(br.double(), bi.double()).requires_grad_(True)
    z = torch.matmul(A, B)
    cr, ci = _cotangent(tuple(z.shape), 19)
    (z.real * cr + z.imag * ci).sum().backward()
    l_ar, l_ai, l_br, l_bi = (_leaf(t) for t in (ar, ai, br, bi))
    c = trnfft_amd.complex_matmul(ComplexTensor(l_ar, l_ai), ComplexTensor(l_br, l_bi))
    assert tuple(c.real.shape) == tuple(z.shape)
    (c.real * cr.float().cuda() + c.imag * ci.float().cuda()).sum().backward()
    assert rel_l2(l_ar.grad, l_ai.grad, A.grad.real, A.grad.imag) <= TOL
    assert rel_l2(l_br.grad, l_bi.grad, B.grad.real, B.grad.imag) <= TOL


def test_complex_matmul_gradients():
    g = torch.Generator().manual_seed(15)
    ar, ai = torch.randn(70, 33, generator=g), torch.randn(70, 33, generator=g)
    br, bi = torch.randn(33, 130, generator=g), torch.randn(33, 130, generator=g)
    cr, ci = _cotangent((70, 130), 16)
    l_ar, l_ai, l_br, l_bi = (_leaf(t) for t in (ar, ai, br, bi))
    c = trnfft_amd.complex_matmul(ComplexTensor(l_ar, l_ai), ComplexTensor(l_br, l_bi))
    (c.real * cr.float().cuda() + c.imag * ci.float().cuda()).sum().backward()
    A = torch.complex(ar.double(), ai.double()).requires_grad_(True)
    B = torch.complex(br.double(), bi.double()).requires_grad_(True)
    z = A @ B
    (z.real * cr + z.imag * ci).sum().backward()
    # torch's complex gradient convention: grad = dL/dRe + i dL/dIm
    assert rel_l2(l_ar.grad, l_ai.grad, A.grad.real, A.grad.imag) <= TOL
    assert rel_l2(l_br.grad, l_bi.grad, B.grad.real, B.grad.imag) <= TOL


def test_istft_gradient_flows():
    g = torch.Generator().manual_seed(17)
    x = torch.randn(2, 3000, generator=g)
    spec = trnfft_amd.stft(x.cuda(), 256, hop_length=64)
    sr, si = _leaf(spec.real.cpu()), _leaf(spec.imag.cpu())
    y = trnfft_amd.istft(ComplexTensor(sr, si), 256, hop_length=64, length=3000)
    c, _ = _cotangent(tuple(y.shape), 18)
    (y * c.float().cuda()).sum().backward()
    r_r, r_i = spec.real.cpu().double().requires_grad_(True), spec.imag.cpu().double().requires_grad_(True)
    z = torch.istft(torch.complex(r_r, r_i), 256, hop_length=64, window=torch.hann_window(256, dtype=torch.float64),
                    length=3000)
    (z * c).sum().backward()
    assert rel_l2(sr.grad, si.grad, r_r.grad, r_i.grad) <= 1e-4


ISTFT_GRAD_CASES = [
    # lead, n_fft, hop, frames, center, normalized, onesided, length
    ((2,), 256, 64, 40, True, False, True, 3000),
    ((2,), 512, 128, 30, False, False, True, None),   # no centring: env[0] = 0, the raw-sum branch
    ((2, 2), 512, 256, 25, True, True, True, None),   # normalized, leading dims
    ((2,), 256, 64, 40, True, False, False, 3000),    # two-sided spectra
    ((1,), 1024, 256, 12, True, False, True, 5000),   # zero fill past the signal
    ((3,), 64, 16, 50, False, True, False, None),     # two-sided, no centring
]


@pytest.mark.parametrize("lead,n_fft,hop,frames,center,normalized,onesided,length", ISTFT_GRAD_CASES)
def test_istft_gradient_fused_path(lead, n_fft, hop, frames, center, normalized, onesided, length):
    # power-of-two n_fft: the fused kernel forward, the spectra gradient as the fused forward STFT of
    # the envelope-divided gradient; against autograd through the oracle's float64 restatement
    bins = n_fft // 2 + 1 if onesided else n_fft
    g = torch.Generator().manual_seed(n_fft + hop + frames)
    re, im = torch.randn(*lead, bins, frames, generator=g), torch.randn(*lead, bins, frames, generator=g)
    sr, si = _leaf(re), _leaf(im)
    y = trnfft_amd.istft(ComplexTensor(sr, si), n_fft, hop_length=hop, center=center, normalized=normalized,
                         onesided=onesided, length=length)
    assert type(y.grad_fn).__name__ == "_IstftFnBackward"
    c, _ = _cotangent(tuple(y.shape), 5)
    (y * c.float().cuda()).sum().backward()
    r_r, r_i = re.double().requires_grad_(True), im.double().requires_grad_(True)
    z = oracle.istft((r_r, r_i), n_fft, hop_length=hop, window=torch.hann_window(n_fft, dtype=torch.float64),
                     center=center, normalized=normalized, onesided=onesided, length=length)
    assert tuple(z.shape) == tuple(y.shape)
    (z * c).sum().backward()
    # the inverse STFT's own parity bound: the gradient divides by the window envelope, which at
    # the first kept samples without centring is ~1e-8 (Hann tails), so edge frames carry values
    # ~1e4 larger than their neighbours, and the STFT pairs two frames per complex transform
    tol = 4e-6 * math.log2(n_fft)
    assert rel_l2(sr.grad, si.grad, r_r.grad, r_i.grad) <= tol
    # frames-major input (transposed views): the same gradient, in the input's shape
    fr, fi = (_leaf(t.transpose(-2, -1).contiguous()) for t in (re, im))
    y2 = trnfft_amd.istft(ComplexTensor._wrap(fr.transpose(-2, -1), fi.transpose(-2, -1)), n_fft, hop_length=hop,
                          center=center, normalized=normalized, onesided=onesided, length=length)
    (y2 * c.float().cuda()).sum().backward()
    assert rel_l2(fr.grad.transpose(-2, -1), fi.grad.transpose(-2, -1), r_r.grad, r_i.grad) <= tol


def test_istft_window_gradient_composes():
    # a window that needs a gradient keeps the composed path (its gradient included)
    g = torch.Generator().manual_seed(41)
    re, im = torch.randn(2, 129, 30, generator=g), torch.randn(2, 129, 30, generator=g)
    w = torch.hann_window(256) + 0.1
    sr, si, aw = _leaf(re), _leaf(im), _leaf(w)
    y = trnfft_amd.istft(ComplexTensor(sr, si), 256, hop_length=64, window=aw)
    assert type(y.grad_fn).__name__ != "_IstftFnBackward"
    c, _ = _cotangent(tuple(y.shape), 6)
    (y * c.float().cuda()).sum().backward()
    r_r, r_i, rw = re.double().requires_grad_(True), im.double().requires_grad_(True), w.double().requires_grad_(True)
    z = oracle.istft((r_r, r_i), 256, hop_length=64, window=rw)
    (z * c).sum().backward()
    assert rel_l2(sr.grad, si.grad, r_r.grad, r_i.grad) <= TOL
    assert _rel(aw.grad, rw.grad) <= TOL


def test_reference_named_autograd_entry_points():
    # the names trnfft's NKI autograd module exposes (trnfft/nki/autograd.py:115-116, 158-159,
    # 204-205), here on the HIP kernels: values and gradients against fp64 torch
    from trnfft_amd import autograd as ag

    g = torch.Generator().manual_seed(31)
    xr, xi = torch.randn(6, 64, generator=g), torch.randn(6, 64, generator=g)
    a_r, a_i = _leaf(xr), _leaf(xi)
    y_re, y_im = ag.fft_autograd(a_r, a_i, False)
    (y_re.square().sum() + y_im.sum()).backward()
    r_r, r_i = xr.double().requires_grad_(True), xi.double().requires_grad_(True)
    z = torch.fft.fft(torch.complex(r_r, r_i))
    (z.real.square().sum() + z.imag.sum()).backward()
    assert rel_l2(y_re, y_im, z.real.detach(), z.imag.detach()) <= TOL
    assert rel_l2(a_r.grad, a_i.grad, r_r.grad, r_i.grad) <= TOL

    ar, ai = torch.randn(8, 16, generator=g), torch.randn(8, 16, generator=g)
    br, bi = torch.randn(16, 5, generator=g), torch.randn(16, 5, generator=g)
    la_r, la_i, lb_r, lb_i = _leaf(ar), _leaf(ai), _leaf(br), _leaf(bi)
    c_re, c_im = ag.complex_gemm_autograd(la_r, la_i, lb_r, lb_i)
    (c_re.sum() + 2 * c_im.sum()).backward()
    rar, rai = ar.double().requires_grad_(True), ai.double().requires_grad_(True)
    rbr, rbi = br.double().requires_grad_(True), bi.double().requires_grad_(True)
    C = torch.complex(rar, rai) @ torch.complex(rbr, rbi)
    (C.real.sum() + 2 * C.imag.sum()).backward()
    assert rel_l2(c_re, c_im, C.real.detach(), C.imag.detach()) <= TOL
    assert rel_l2(la_r.grad, la_i.grad, rar.grad, rai.grad) <= TOL
    assert rel_l2(lb_r.grad, lb_i.grad, rbr.grad, rbi.grad) <= TOL

    wr, wi = torch.randn(5, 16, generator=g), torch.randn(5, 16, generator=g)
    y_re, y_im = ag.complex_linear_autograd(_leaf(ar), _leaf(ai), _leaf(wr), _leaf(wi))
    Y = torch.complex(ar.double(), ai.double()) @ torch.complex(wr.double(), wi.double()).T
    assert rel_l2(y_re, y_im, Y.real, Y.imag) <= TOL
