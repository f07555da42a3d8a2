"""GPU parity of the matrix-core paths: complex GEMM, ComplexLinear and DFT-as-GEMM.

Oracle: the reference's four-real-matmul formulas (oracle.complex_matmul / complex_linear,
trnfft/complex.py:142-150, trnfft/nn.py:43-48) evaluated in float64 on the same inputs;
tolerance 1e-6*log2(K) relative L2 (K = contraction length).
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, seeded_complex, tol_pow2
from trnfft_amd import ComplexTensor
from trnfft_amd.nn import ComplexLinear

pytestmark = pytest.mark.gpu


def _tol_k(k):
    return 1e-6 * max(1.0, math.log2(k))


def _planes(shape, g):
    return torch.randn(*shape, generator=g), torch.randn(*shape, generator=g)


@pytest.mark.parametrize("m,k,n", [(128, 128, 128), (100, 33, 70), (1, 5, 3), (257, 1024, 129), (512, 64, 1000)])
def test_complex_gemm_vs_float64(m, k, n):
    g = torch.Generator().manual_seed(m * 7 + k)
    a = _planes((m, k), g)
    b = _planes((k, n), g)
    got = trnfft_amd.complex_matmul(ComplexTensor(a[0].cuda(), a[1].cuda()), ComplexTensor(b[0].cuda(), b[1].cuda()))
    ref = oracle.complex_matmul((a[0].double(), a[1].double()), (b[0].double(), b[1].double()))
    assert got.shape == (m, n)
    assert rel_l2(got.real, got.imag, *ref) <= _tol_k(k), (m, k, n)


@pytest.mark.parametrize("sa,sb", [
    ((4, 50, 33), (4, 33, 70)),        # batched
    ((4, 50, 33), (33, 70)),           # batched A, shared 2-D B (one GEMM over all rows)
    ((50, 33), (3, 33, 70)),           # shared A, batched B
    ((2, 1, 17, 9), (3, 9, 20)),       # broadcast batch axes -> (2, 3, 17, 20)
    ((2, 3, 17, 9), (1, 3, 9, 20)),
    ((33,), (33, 70)),                 # vector @ matrix
    ((50, 33), (33,)),                 # matrix @ vector
    ((5, 50, 33), (33,)),              # batched matrix @ vector
    ((33,), (4, 33, 7)),               # vector @ batched matrix
    ((33,), (33,)),                    # dot product -> 0-d
    ((0, 8, 5), (0, 5, 3)),            # empty batch
    ((70000, 2, 3), (70000, 3, 2)),    # more products than one launch's grid.y (65535)
])
def test_complex_matmul_torch_matmul_shapes(sa, sb):
    # the reference's complex_matmul is four torch.matmul (trnfft/complex.py:142-150), so it takes
    # every torch.matmul shape; the result and its shape match the same formula in float64
    g = torch.Generator().manual_seed(len(sa) * 10 + len(sb))
    a = _planes(sa, g)
    b = _planes(sb, g)
    got = ComplexTensor(a[0].cuda(), a[1].cuda()) @ ComplexTensor(b[0].cuda(), b[1].cuda())
    ref = oracle.complex_matmul((a[0].double(), a[1].double()), (b[0].double(), b[1].double()))
    assert tuple(got.real.shape) == tuple(ref[0].shape)
    if ref[0].numel():
        assert rel_l2(got.real, got.imag, *ref) <= _tol_k(sa[-1]), (sa, sb)


def test_complex_matmul_shape_mismatch_raises_like_torch():
    a = ComplexTensor(torch.randn(4, 5).cuda(), torch.randn(4, 5).cuda())
    b = ComplexTensor(torch.randn(2, 6, 3).cuda(), torch.randn(2, 6, 3).cuda())
    with pytest.raises(RuntimeError):
        a @ b


def test_complex_gemm_kat():
    a = ComplexTensor(torch.tensor([[1.0]]).cuda(), torch.tensor([[2.0]]).cuda())
    b = ComplexTensor(torch.tensor([[3.0]]).cuda(), torch.tensor([[4.0]]).cuda())
    c = a @ b
    assert c.real.item() == -5.0 and c.imag.item() == 10.0


@pytest.mark.parametrize("m,k,n,bias", [(64, 32, 48, True), (8192, 1024, 1024, False), (300, 129, 77, True)])
def test_complex_linear_vs_float64(m, k, n, bias):
    g = torch.Generator().manual_seed(42)
    x = _planes((m, k), g)
    w_re = torch.empty(n, k).uniform_(-1 / math.sqrt(k), 1 / math.sqrt(k), generator=g)
    w_im = torch.empty(n, k).uniform_(-1 / math.sqrt(k), 1 / math.sqrt(k), generator=g)
    b = _planes((n,), g) if bias else (None, None)
    got = trnfft_amd.complex_linear(
        ComplexTensor(x[0].cuda(), x[1].cuda()), w_re.cuda(), w_im.cuda(),
        None if b[0] is None else b[0].cuda(), None if b[1] is None else b[1].cuda(),
    )
    ref = oracle.complex_linear(
        (x[0].double(), x[1].double()), w_re.double(), w_im.double(),
        None if b[0] is None else b[0].double(), None if b[1] is None else b[1].double(),
    )
    assert rel_l2(got.real, got.imag, *ref) <= _tol_k(k), (m, k, n)


def test_complex_linear_module_matches_reference_formula():
    torch.manual_seed(42)
    layer = ComplexLinear(64, 96)
    assert set(layer.state_dict()) == {"W_re.weight", "W_im.weight", "bias_re", "bias_im"}
    with torch.no_grad():
        layer.bias_re.normal_()
        layer.bias_im.normal_()
    x = ComplexTensor(torch.randn(16, 64), torch.randn(16, 64))
    ref = oracle.complex_linear(
        (x.real.double(), x.imag.double()), layer.W_re.weight.detach().double(), layer.W_im.weight.detach().double(),
        layer.bias_re.detach().double(), layer.bias_im.detach().double(),
    )
    layer = layer.cuda()
    y = layer(ComplexTensor(x.real.cuda(), x.imag.cuda()))
    assert y.shape == (16, 96)
    assert rel_l2(y.real, y.imag, *ref) <= _tol_k(64)


@pytest.mark.parametrize("n", [8, 64, 256])
@pytest.mark.parametrize("inverse", [False, True])
def test_dft_gemm_vs_oracle(n, inverse):
    from trnfft_amd import fft_core as fc

    re, im = seeded_complex(1000, n)
    x = ComplexTensor(re.cuda(), im.cuda())
    got = fc._fft_via_gemm(x, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(n), (n, inverse)


def test_config5b_full_size_both_formulations():
    # BASELINE config 5b at full size (65536 x 256, forward): the DFT-as-GEMM on the matrix cores
    # and the Stockham kernel, each against the oracle on all rows
    from trnfft_amd import fft_core as fc

    re, im = seeded_complex(65536, 256)
    x = ComplexTensor(re.cuda(), im.cuda())
    ref = oracle.fft_core(re, im, False)
    gemm = fc._fft_via_gemm(x, False)
    assert rel_l2(gemm.real, gemm.imag, *ref) <= tol_pow2(256)
    stockham = trnfft_amd.fft(x)
    assert rel_l2(stockham.real, stockham.imag, *ref) <= tol_pow2(256)


def test_dft_gemm_threshold_routing():
    from trnfft_amd import fft_core as fc

    re, im = seeded_complex(64, 256)
    old = fc._DFT_GEMM_THRESHOLD
    fc._DFT_GEMM_THRESHOLD = 256
    try:
        got = trnfft_amd.fft(ComplexTensor(re.cuda(), im.cuda()))
    finally:
        fc._DFT_GEMM_THRESHOLD = old
    ref = oracle.fft_core(re, im, False)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(256)
