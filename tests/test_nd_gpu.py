"""GPU parity of the n-D real and complex front ends (trnfft/api.py:105-288): rfft2/irfft2,
rfftn/irfftn, fftn/ifftn with s= and dim=, and fft/ifft with n=, mirroring the reference's
tests/test_fft.py:108-162 and :682-719, checked against numpy float64 and the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, tol_bluestein, tol_pow2
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu


def _np_rel(got: ComplexTensor, ref: np.ndarray) -> float:
    return rel_l2(got.real, got.imag, torch.from_numpy(ref.real.copy()), torch.from_numpy(ref.imag.copy()))


@pytest.mark.parametrize("shape", [(8, 16), (16, 32), (3, 64, 128), (2, 2048, 16)])
def test_rfft2_vs_numpy(shape):
    x = torch.from_numpy(np.random.default_rng(42).standard_normal(shape).astype(np.float32))
    got = trnfft_amd.rfft2(x.cuda())
    assert got.shape == (*shape[:-1], shape[-1] // 2 + 1)
    assert _np_rel(got, np.fft.rfft2(x.double().numpy())) <= tol_pow2(shape[-1] * shape[-2])
    back = trnfft_amd.irfft2(got, s=shape[-2:])
    assert rel_l2(back, torch.zeros_like(back), x, torch.zeros_like(x)) <= 2 * tol_pow2(shape[-1] * shape[-2])
    assert trnfft_amd.irfft2(got).shape == x.shape  # default s: last dim 2*(bins-1)


def test_rfft2_with_s_param():
    x = torch.from_numpy(np.random.default_rng(7).standard_normal((8, 16)).astype(np.float32))
    got = trnfft_amd.rfft2(x.cuda(), s=(16, 32))
    assert got.shape == (16, 17)
    assert _np_rel(got, np.fft.rfft2(x.double().numpy(), s=(16, 32))) <= tol_pow2(512)
    got = trnfft_amd.rfft2(x.cuda(), s=(6, 10))  # truncation and non-power-of-two axes
    assert _np_rel(got, np.fft.rfft2(x.double().numpy(), s=(6, 10))) <= tol_bluestein(10)


@pytest.mark.parametrize("shape,dim", [((4, 8, 16), None), ((4, 8, 16), (0, 2)), ((5, 12, 10), None), ((3, 4, 256), (-1,))])
def test_rfftn_irfftn_vs_numpy(shape, dim):
    x = torch.from_numpy(np.random.default_rng(3).standard_normal(shape).astype(np.float32))
    axes = tuple(range(len(shape))) if dim is None else dim
    got = trnfft_amd.rfftn(x.cuda(), dim=dim)
    ref = np.fft.rfftn(x.double().numpy(), axes=axes)
    assert got.shape == ref.shape
    tol = tol_bluestein(max(shape)) if any(shape[d] & (shape[d] - 1) for d in axes) else tol_pow2(max(shape))
    assert _np_rel(got, ref) <= 3 * tol
    s = [shape[d] for d in axes]
    back = trnfft_amd.irfftn(got, s=s, dim=dim)
    assert back.shape == x.shape
    assert rel_l2(back, torch.zeros_like(back), x, torch.zeros_like(x)) <= 6 * tol


@pytest.mark.parametrize("shape,dim,s", [((4, 8, 8), None, None), ((4, 8, 16), (-2, -1), None),
                                         ((4, 8), (0,), None), ((6, 10, 12), (0, 2), (8, 16)),
                                         ((3, 33, 64), (1,), (40,))])
def test_fftn_ifftn_vs_numpy(shape, dim, s):
    rng = np.random.default_rng(42)
    re = rng.standard_normal(shape).astype(np.float32)
    im = rng.standard_normal(shape).astype(np.float32)
    axes = tuple(range(len(shape))) if dim is None else dim
    x = ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda())
    got = trnfft_amd.fftn(x, s=s, dim=dim)
    ref = np.fft.fftn(re.astype(np.float64) + 1j * im, s=s, axes=axes)
    assert got.shape == ref.shape
    assert _np_rel(got, ref) <= 3 * tol_bluestein(max(shape))
    back = trnfft_amd.ifftn(got, dim=dim)
    ref_back = np.fft.ifftn(ref, axes=axes)
    assert _np_rel(back, ref_back) <= 6 * tol_bluestein(max(shape))
    if s is None:
        # the oracle's restatement of the reference (same axis order) agrees as well
        ref_o = oracle.fftn((torch.from_numpy(re), torch.from_numpy(im)), dim=dim)
        assert rel_l2(got.real, got.imag, *ref_o) <= 3 * tol_bluestein(max(shape))


# transforms along axis -2 with few trailing columns: whole (n x s) blocks staged through LDS
# (s <= half the strided kernel's column tile), ragged block counts, complex and real input
@pytest.mark.parametrize("shape", [(37, 2, 3), (9, 16, 1), (11, 64, 5), (5, 128, 3), (7, 512, 7), (3, 1024, 8),
                                   (5, 1024, 2), (3, 4096, 2), (2, 4096, 1), (65, 32, 31)])
def test_fft_along_axis_with_few_trailing_columns(shape):
    rng = np.random.default_rng(5)
    re = rng.standard_normal(shape).astype(np.float32)
    im = rng.standard_normal(shape).astype(np.float32)
    x = ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda())
    n = shape[1]
    for inverse in (False, True):
        got = trnfft_amd.fftn(x, dim=(1,)) if not inverse else trnfft_amd.ifftn(x, dim=(1,))
        z = re.astype(np.float64) + 1j * im
        ref = np.fft.ifft(z, axis=1) if inverse else np.fft.fft(z, axis=1)
        assert _np_rel(got, ref) <= tol_pow2(n), (shape, inverse)
    got = trnfft_amd.fftn(torch.from_numpy(re).cuda(), dim=(1,))
    assert _np_rel(got, np.fft.fft(re.astype(np.float64), axis=1)) <= tol_pow2(n), shape


# non-power-of-two axes along a strided dimension (Bluestein in place down the columns, padded
# length m <= 4096): against numpy float64 and against the last-axis Bluestein path on the moved
# axis (same chirp and filter, so the two agree far inside the parity tolerance)
@pytest.mark.parametrize("shape", [(3, 3, 70), (2, 5, 3), (4, 12, 16), (3, 17, 33), (2, 100, 64), (2, 480, 40),
                                   (2, 1000, 8), (1, 2047, 5), (2, 2000, 100)])
def test_non_pow2_axis_strided_bluestein(shape):
    from trnfft_amd.fft_core import strided_ok

    rng = np.random.default_rng(17)
    re = rng.standard_normal(shape).astype(np.float32)
    im = rng.standard_normal(shape).astype(np.float32)
    n, stride = shape[1], shape[2]
    assert strided_ok(n, stride)
    x = ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda())
    z = re.astype(np.float64) + 1j * im
    for inverse in (False, True):
        got = trnfft_amd.ifftn(x, dim=(1,)) if inverse else trnfft_amd.fftn(x, dim=(1,))
        ref = np.fft.ifft(z, axis=1) if inverse else np.fft.fft(z, axis=1)
        assert _np_rel(got, ref) <= 3 * tol_bluestein(n), (shape, inverse)
        moved = ComplexTensor(x.real.transpose(1, 2).contiguous(), x.imag.transpose(1, 2).contiguous())
        last = trnfft_amd.ifft(moved) if inverse else trnfft_amd.fft(moved)
        assert rel_l2(got.real, got.imag, last.real.transpose(1, 2), last.imag.transpose(1, 2)) <= 1e-5, shape
    got = trnfft_amd.fftn(torch.from_numpy(re).cuda(), dim=(1,))
    assert _np_rel(got, np.fft.fft(re.astype(np.float64), axis=1)) <= 3 * tol_bluestein(n), shape


# power-of-two axes longer than 4096 along a strided dimension (stride >= 4): the two-pass
# strided four-step (n = n1 * n2, every split from 64 x 128 up), against numpy float64 at sizes
# numpy finishes quickly, with ragged strides (down to the minimum of 4) and real input
@pytest.mark.parametrize("shape", [(3, 4096, 16), (2, 4096, 40), (3, 8192, 16), (2, 16384, 17), (1, 32768, 48),
                                   (2, 65536, 16), (1, 131072, 24), (1, 262144, 16), (5, 8192, 4), (3, 65536, 5),
                                   (1, 262144, 7)])
def test_long_pow2_axis_strided_fourstep_vs_numpy(shape):
    from trnfft_amd.fft_core import strided_ok

    n, stride = shape[1], shape[2]
    assert strided_ok(n, stride)
    rng = np.random.default_rng(23)
    re = rng.standard_normal(shape).astype(np.float32)
    im = rng.standard_normal(shape).astype(np.float32)
    x = ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda())
    z = re.astype(np.float64) + 1j * im
    for inverse in (False, True):
        got = trnfft_amd.ifftn(x, dim=(1,)) if inverse else trnfft_amd.fftn(x, dim=(1,))
        ref = np.fft.ifft(z, axis=1) if inverse else np.fft.fft(z, axis=1)
        assert _np_rel(got, ref) <= tol_pow2(n), (shape, inverse)
    got = trnfft_amd.fftn(torch.from_numpy(re).cuda(), dim=(1,))
    assert _np_rel(got, np.fft.fft(re.astype(np.float64), axis=1)) <= tol_pow2(n), shape


# the largest splits (2^19 .. 2^24 along the axis, up to 2^28 elements; three factors from 2^21,
# with the minimum 8 columns there), where numpy float64 is too slow: against the contiguous
# four-step on the moved axis (different kernels over another split) and through the inverse
# round trip
@pytest.mark.parametrize("lg,stride", [(19, 16), (20, 16), (21, 16), (21, 8), (22, 16), (22, 9), (23, 16), (24, 16)])
def test_long_pow2_axis_strided_fourstep_large(lg, stride):
    from trnfft_amd.fft_core import strided_ok

    n = 1 << lg
    assert strided_ok(n, stride)
    g = torch.Generator(device="cuda").manual_seed(lg)
    re = torch.randn((1, n, stride), generator=g, device="cuda")
    im = torch.randn((1, n, stride), generator=g, device="cuda")
    x = ComplexTensor(re, im)

    def rel(a_re, a_im, b_re, b_im):  # relative L2 on the GPU, float64 accumulation
        num = ((a_re.double() - b_re.double()) ** 2).sum() + ((a_im.double() - b_im.double()) ** 2).sum()
        return float(torch.sqrt(num / ((b_re.double() ** 2).sum() + (b_im.double() ** 2).sum())))

    got = trnfft_amd.fftn(x, dim=(1,))
    moved = ComplexTensor(re.transpose(1, 2).contiguous(), im.transpose(1, 2).contiguous())
    last = trnfft_amd.fft(moved)
    assert rel(got.real, got.imag, last.real.transpose(1, 2), last.imag.transpose(1, 2)) <= 2 * tol_pow2(n), lg
    del last, moved
    back = trnfft_amd.ifftn(got, dim=(1,))
    assert rel(back.real, back.imag, re, im) <= 2 * tol_pow2(n), lg


def test_strided_fourstep_abi_in_place_and_workspace():
    # tfa_execute_strided_ws through the C ABI: workspace size, in place (out == in), and the
    # missing-workspace error
    import ctypes

    from trnfft_amd import _lib
    from trnfft_amd.dispatch import ptr, stream_handle
    from trnfft_amd.plan import native_plan

    outer, n, stride = 2, 16384, 20
    rng = np.random.default_rng(29)
    re = rng.standard_normal((outer, n, stride)).astype(np.float32)
    im = rng.standard_normal((outer, n, stride)).astype(np.float32)
    d_re, d_im = torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda()
    lib = _lib.lib()
    plan = native_plan(_lib.KIND_C2C, n, False, 0)
    nbytes = ctypes.c_size_t(0)
    assert lib.tfa_strided_workspace_size(plan.handle, outer, stride, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 2 * 4 * outer * n * stride
    ws = torch.empty(nbytes.value // 4, device="cuda")
    dev = torch.device("cuda", 0)
    assert lib.tfa_execute_strided_ws(plan.handle, outer, stride, ptr(d_re), ptr(d_im), ptr(d_re), ptr(d_im),
                                      None, stream_handle(dev)) != 0
    rc = lib.tfa_execute_strided_ws(plan.handle, outer, stride, ptr(d_re), ptr(d_im), ptr(d_re), ptr(d_im), ptr(ws),
                                    stream_handle(dev))
    assert rc == 0
    torch.cuda.synchronize()
    ref = np.fft.fft(re.astype(np.float64) + 1j * im, axis=1)
    assert rel_l2(d_re, d_im, ref.real, ref.imag) <= tol_pow2(n)
    # short axes and small strides need no workspace; n = 4096 takes the two passes from 16 columns
    small = native_plan(_lib.KIND_C2C, 2048, False, 0)
    assert lib.tfa_strided_workspace_size(small.handle, outer, stride, ctypes.byref(nbytes)) == 0 and nbytes.value == 0
    p4096 = native_plan(_lib.KIND_C2C, 4096, False, 0)
    assert lib.tfa_strided_workspace_size(p4096.handle, outer, 15, ctypes.byref(nbytes)) == 0 and nbytes.value == 0
    assert lib.tfa_strided_workspace_size(p4096.handle, outer, 16, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 2 * 4 * outer * 4096 * 16
    assert lib.tfa_strided_workspace_size(plan.handle, outer, 3, ctypes.byref(nbytes)) == 0 and nbytes.value == 0


def test_fft2_non_pow2_image():
    # 480 x 640: the 640 axis runs the contiguous Bluestein kernel, the 480 axis the strided one
    rng = np.random.default_rng(19)
    x = rng.standard_normal((2, 480, 640)).astype(np.float32)
    got = trnfft_amd.fft2(torch.from_numpy(x).cuda())
    assert _np_rel(got, np.fft.fft2(x.astype(np.float64))) <= 3 * tol_bluestein(640)
    back = trnfft_amd.ifftn(got, dim=(-2, -1))
    assert rel_l2(back.real, back.imag, torch.from_numpy(x), torch.zeros(2, 480, 640)) <= 6 * tol_bluestein(640)


@pytest.mark.parametrize("n_in,n", [(100, 128), (300, 256), (1000, 1000), (64, 100), (4096, 4000)])
def test_fft_ifft_n_param(n_in, n):
    rng = np.random.default_rng(5)
    re = rng.standard_normal((3, n_in)).astype(np.float32)
    im = rng.standard_normal((3, n_in)).astype(np.float32)
    x = ComplexTensor(torch.from_numpy(re).cuda(), torch.from_numpy(im).cuda())
    tol = tol_pow2(n) if n & (n - 1) == 0 else tol_bluestein(n)
    got = trnfft_amd.fft(x, n=n)
    assert got.shape == (3, n)
    assert _np_rel(got, np.fft.fft(re.astype(np.float64) + 1j * im, n=n)) <= 50 * tol
    ref_o = oracle.fft((torch.from_numpy(re), torch.from_numpy(im)), n=n)
    assert rel_l2(got.real, got.imag, *ref_o) <= tol
    got_i = trnfft_amd.ifft(x, n=n)
    ref_oi = oracle.ifft((torch.from_numpy(re), torch.from_numpy(im)), n=n)
    assert rel_l2(got_i.real, got_i.imag, *ref_oi) <= tol
