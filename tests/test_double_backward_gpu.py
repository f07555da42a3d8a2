"""Second derivatives of the HIP path.  trnfft's pytorch path (trnfft/fft_core.py:53-117,
api.py:22-139,291-365, nn.py:33-49) is made of torch ops, so its gradients can be differentiated
again (create_graph=True).  Here each case forms a Hessian-vector product of a quadratic loss of the
outputs, L = sum(w * y^2), H v = d/dx <dL/dx, v>, through the native kernels and checks it against
the same product through float64 torch (torch.fft, torch.stft, complex matmul) or, for Bluestein
lengths, through the oracle's fp32 restatement of the reference's own operator."""

from __future__ import annotations

import pytest
import torch

import oracle
import trnfft_amd
from conftest import tol_bluestein
from trnfft_amd import ComplexTensor
from trnfft_amd.nn import ComplexLinear

pytestmark = pytest.mark.gpu

TOL = 2e-5  # fp32 kernels (forward, adjoint, adjoint of the adjoint) vs float64, relative L2


def _rel_all(got, ref):
    num = sum(float((g.detach().double().cpu() - r.detach().double().cpu()).norm() ** 2) for g, r in zip(got, ref))
    den = sum(float(r.detach().double().cpu().norm() ** 2) for r in ref)
    return (num / den) ** 0.5


def _hvp(outs_fn, leaves, weights, vs):
    outs = outs_fn(*leaves)
    loss = sum((w * o * o).sum() for w, o in zip(weights, outs))
    gs = torch.autograd.grad(loss, leaves, create_graph=True)
    s = sum((g * v).sum() for g, v in zip(gs, vs))
    return torch.autograd.grad(s, leaves)


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


def _pair(ours_fn, ref_fn, inputs, out_shapes, seed, ref_dtype=torch.float64):
    """HVP of sum(w * y^2) through ours (fp32, cuda) and the reference (ref_dtype, cpu)."""
    ws = [_rand(s, seed + i).abs() for i, s in enumerate(out_shapes)]
    vs = [_rand(tuple(x.shape), seed + 10 + i) for i, x in enumerate(inputs)]
    mine = [x.float().cuda().requires_grad_(True) for x in inputs]
    got = _hvp(ours_fn, mine, [w.float().cuda() for w in ws], [v.float().cuda() for v in vs])
    ref_in = [x.to(ref_dtype).requires_grad_(True) for x in inputs]
    ref = _hvp(ref_fn, ref_in, [w.to(ref_dtype) for w in ws], [v.to(ref_dtype) for v in vs])
    return got, ref


@pytest.mark.parametrize("n,batch,inverse", [(1024, 6, False), (1024, 6, True), (1 << 15, 2, False), (16, 5, True)])
def test_c2c_second_derivative(n, batch, inverse):
    xr, xi = _rand((batch, n), 1), _rand((batch, n), 2)

    def ours(re, im):
        y = (trnfft_amd.ifft if inverse else trnfft_amd.fft)(ComplexTensor(re, im))
        return y.real, y.imag

    def ref(re, im):
        z = (torch.fft.ifft if inverse else torch.fft.fft)(torch.complex(re, im))
        return z.real, z.imag

    got, want = _pair(ours, ref, [xr, xi], [(batch, n)] * 2, 3)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("n,inverse", [(1000, False), (127, True)])
def test_bluestein_second_derivative_vs_oracle(n, inverse):
    # the reference's operator carries its fp32 chirp: pinned against the oracle's restatement
    xr, xi = _rand((3, n), 4), _rand((3, n), 5)

    def ours(re, im):
        y = (trnfft_amd.ifft if inverse else trnfft_amd.fft)(ComplexTensor(re, im))
        return y.real, y.imag

    def ref(re, im):
        return oracle.fft_core(re, im, inverse)

    got, want = _pair(ours, ref, [xr, xi], [(3, n)] * 2, 6, ref_dtype=torch.float32)
    assert _rel_all(got, want) <= tol_bluestein(n)


def test_real_input_fft_second_derivative():
    x = _rand((4, 256), 7)

    def ours(a):
        y = trnfft_amd.fft(ComplexTensor(a))
        return y.real, y.imag

    def ref(a):
        z = torch.fft.fft(a)
        return z.real, z.imag

    got, want = _pair(ours, ref, [x], [(4, 256)] * 2, 8)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("n", [1024, 64])
def test_rfft_irfft_second_derivative(n):
    x = _rand((5, n), 9)

    def ours(a):
        y = trnfft_amd.rfft(a)
        return y.real, y.imag

    def ref(a):
        z = torch.fft.rfft(a)
        return z.real, z.imag

    got, want = _pair(ours, ref, [x], [(5, n // 2 + 1)] * 2, 10)
    assert _rel_all(got, want) <= TOL

    sr, si = _rand((5, n // 2 + 1), 11), _rand((5, n // 2 + 1), 12)
    got, want = _pair(lambda r, i: (trnfft_amd.irfft(ComplexTensor(r, i), n=n),),
                      lambda r, i: (torch.fft.irfft(torch.complex(r, i), n=n),), [sr, si], [(5, n)], 13)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("real_in,inverse", [(True, False), (False, False), (False, True)])
def test_fft2_second_derivative(real_in, inverse):
    shape = (3, 64, 128)
    xr, xi = _rand(shape, 14), _rand(shape, 15)
    f_ours = (lambda t: trnfft_amd.ifftn(t, dim=(-2, -1))) if inverse else trnfft_amd.fft2
    f_ref = torch.fft.ifft2 if inverse else torch.fft.fft2
    if real_in:
        got, want = _pair(lambda a: (lambda y: (y.real, y.imag))(f_ours(ComplexTensor(a))),
                          lambda a: (lambda z: (z.real, z.imag))(f_ref(a)), [xr], [shape] * 2, 16)
    else:
        got, want = _pair(lambda r, i: (lambda y: (y.real, y.imag))(f_ours(ComplexTensor(r, i))),
                          lambda r, i: (lambda z: (z.real, z.imag))(f_ref(torch.complex(r, i))), [xr, xi], [shape] * 2,
                          16)
    assert _rel_all(got, want) <= TOL


def test_strided_axis_second_derivative():
    shape = (4, 256, 8)
    xr, xi = _rand(shape, 17), _rand(shape, 18)
    got, want = _pair(lambda r, i: (lambda y: (y.real, y.imag))(trnfft_amd.fftn(ComplexTensor(r, i), dim=(1,))),
                      lambda r, i: (lambda z: (z.real, z.imag))(torch.fft.fft(torch.complex(r, i), dim=1)), [xr, xi],
                      [shape] * 2, 19)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("n_fft,hop,center,normalized", [(256, 64, True, False), (512, 128, False, True)])
def test_stft_second_derivative_signal_and_window(n_fft, hop, center, normalized):
    x = _rand((2, 3000), 20)
    w = torch.hann_window(n_fft, dtype=torch.float64) + 0.1 * _rand((n_fft,), 21).abs()

    def ours(a, win):
        y = trnfft_amd.stft(a, n_fft, hop_length=hop, window=win, center=center, normalized=normalized)
        return y.real, y.imag

    def ref(a, win):
        z = torch.stft(a, n_fft, hop_length=hop, window=win, center=center, pad_mode="reflect", normalized=normalized,
                       onesided=True, return_complex=True)
        return z.real, z.imag

    bins = n_fft // 2 + 1
    frames = (3000 + (n_fft if center else 0) - n_fft) // hop + 1
    got, want = _pair(ours, ref, [x, w], [(2, bins, frames)] * 2, 22)
    assert _rel_all(got, want) <= TOL


def test_stft_second_derivative_bluestein_vs_oracle():
    x = _rand((2, 3000), 23)

    def ours(a):
        y = trnfft_amd.stft(a, 400, hop_length=160)
        return y.real, y.imag

    def ref(a):
        return oracle.stft(a, 400, hop_length=160)

    frames = 3000 // 160 + 1
    got, want = _pair(ours, ref, [x], [(2, 201, frames)] * 2, 24, ref_dtype=torch.float32)
    assert _rel_all(got, want) <= tol_bluestein(400)


def test_complex_linear_second_derivative():
    torch.manual_seed(0)
    layer = ComplexLinear(48, 40).cuda()
    with torch.no_grad():
        layer.bias_re.normal_()
        layer.bias_im.normal_()
    xr, xi = _rand((30, 48), 25), _rand((30, 48), 26)
    wr0 = layer.W_re.weight.detach().double().cpu()
    wi0 = layer.W_im.weight.detach().double().cpu()
    br0 = layer.bias_re.detach().double().cpu()
    bi0 = layer.bias_im.detach().double().cpu()

    def ref(ar, ai, wr, wi):  # the reference's formula (trnfft/nn.py:46-48)
        re = ar @ wr.T - ai @ wi.T + br0
        im = ai @ wr.T + ar @ wi.T + bi0
        return re, im

    ws = [_rand((30, 40), 27 + i).abs() for i in range(2)]
    vs = [_rand((30, 48), 29), _rand((30, 48), 30), _rand((40, 48), 31), _rand((40, 48), 32)]
    ar, ai = xr.float().cuda().requires_grad_(True), xi.float().cuda().requires_grad_(True)
    leaves = [ar, ai, layer.W_re.weight, layer.W_im.weight]  # input and weights (bias terms are linear)
    y = layer(ComplexTensor(ar, ai))
    loss = (ws[0].float().cuda() * y.real**2).sum() + (ws[1].float().cuda() * y.imag**2).sum()
    gs = torch.autograd.grad(loss, leaves, create_graph=True)
    got = torch.autograd.grad(sum((g * v.float().cuda()).sum() for g, v in zip(gs, vs)), leaves)
    ref_in = [xr.clone().requires_grad_(True), xi.clone().requires_grad_(True), wr0.clone().requires_grad_(True),
              wi0.clone().requires_grad_(True)]
    want = _hvp(ref, ref_in, ws, vs)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("sa,sb", [((3, 20, 13), (13, 30)), ((20, 13), (4, 13, 30)), ((70, 33), (33, 50))])
def test_complex_matmul_second_derivative(sa, sb):
    ar, ai, br, bi = _rand(sa, 33), _rand(sa, 34), _rand(sb, 35), _rand(sb, 36)
    out = torch.matmul(torch.complex(ar, ai), torch.complex(br, bi)).shape

    def ours(a_r, a_i, b_r, b_i):
        c = trnfft_amd.complex_matmul(ComplexTensor(a_r, a_i), ComplexTensor(b_r, b_i))
        return c.real, c.imag

    def ref(a_r, a_i, b_r, b_i):
        z = torch.matmul(torch.complex(a_r, a_i), torch.complex(b_r, b_i))
        return z.real, z.imag

    got, want = _pair(ours, ref, [ar, ai, br, bi], [tuple(out)] * 2, 37)
    assert _rel_all(got, want) <= TOL


@pytest.mark.parametrize("n_fft,hop,center,onesided", [(256, 64, True, True), (128, 32, False, False)])
def test_istft_second_derivative(n_fft, hop, center, onesided):
    # the fused path's spectra gradient (a forward STFT) recorded under create_graph
    bins = n_fft // 2 + 1 if onesided else n_fft
    sr, si = _rand((2, bins, 30), 40), _rand((2, bins, 30), 41)

    def ours(r, i):
        return (trnfft_amd.istft(ComplexTensor(r, i), n_fft, hop_length=hop, center=center, onesided=onesided),)

    def ref(r, i):
        return (oracle.istft((r, i), n_fft, hop_length=hop, window=torch.hann_window(n_fft, dtype=torch.float64),
                             center=center, onesided=onesided),)

    length = (30 - 1) * hop + (0 if center else n_fft)
    got, want = _pair(ours, ref, [sr, si], [(2, length)], 42)
    assert _rel_all(got, want) <= TOL

