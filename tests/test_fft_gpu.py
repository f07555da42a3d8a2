"""GPU parity: power-of-two c2c (LDS Stockham and four-step) and Bluestein vs the CPU oracle.

Tolerances (relative L2 over both planes): 1e-6*log2(n) for power-of-two transforms and
1e-5*log2(n) for Bluestein; inputs seeded as the reference's tests (seed 42, re then im).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
import trnfft_amd
from conftest import rel_l2, seeded_complex, tol_bluestein, tol_pow2
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bluestein_vectors.npz")


def _gpu_fft(re, im, inverse=False):
    x = ComplexTensor(re.cuda(), im.cuda())
    y = trnfft_amd.ifft(x) if inverse else trnfft_amd.fft(x)
    torch.cuda.synchronize()
    return y.real.cpu(), y.imag.cpu()


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384])
@pytest.mark.parametrize("inverse", [False, True])
def test_pow2_lds_vs_oracle(n, inverse):
    batch = max(3, min(257, (1 << 16) // n))  # ragged batch: not a multiple of the per-block count
    re, im = seeded_complex(batch, n, seed=n)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_pow2(n), (n, inverse)


@pytest.mark.parametrize("n", [1 << 15, 1 << 16, 1 << 17, 1 << 18, 1 << 19, 1 << 20, 1 << 21])
@pytest.mark.parametrize("inverse", [False, True])
def test_pow2_fourstep_vs_oracle(n, inverse):
    # every (n1, n2) split of the two-pass path up to 1024 x 2048; two rows run the narrow
    # 8-transform tiles below 2^21 (too few workgroups for the wide ones), the wide tiles at 2^21
    re, im = seeded_complex(2, n, seed=n)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_pow2(n), (n, inverse)


@pytest.mark.parametrize("n,batch", [(1 << 15, 64), (1 << 16, 32), (1 << 17, 16), (1 << 18, 16), (1 << 19, 8),
                                     (1 << 20, 4), (1 << 20, 3)])
def test_pow2_fourstep_wide_tiles_vs_numpy(n, batch):
    # batches large enough for the wide column tiles (32 transforms per workgroup; 4 x 2^20 is
    # the smallest 2^20 batch on them, 3 x 2^20 the largest on the narrow ones), both directions,
    # against numpy float64 (the oracle's radix-2 loop is too slow at these batches)
    re, im = seeded_complex(batch, n, seed=n + batch)
    x = re.double().numpy() + 1j * im.double().numpy()
    for inverse in (False, True):
        got = _gpu_fft(re, im, inverse)
        ref = np.fft.ifft(x, axis=-1) if inverse else np.fft.fft(x, axis=-1)
        assert rel_l2(*got, ref.real, ref.imag) <= tol_pow2(n), (n, batch, inverse)


@pytest.mark.parametrize("lg,batch", [(22, 1), (23, 1), (24, 1), (24, 2)])
def test_pow2_fourstep_largest_vs_numpy(lg, batch):
    # splits 2048 x 2048 and 2048 x 4096 (16- and 8-transform tiles), and 2^24 as three strided
    # passes of 256 with the last pass staged through LDS: rows against numpy's float64 FFT (the
    # oracle's radix-2 loop is too slow at these sizes), forward and inverse
    n = 1 << lg
    re, im = seeded_complex(batch, n, seed=lg)
    x = re.double().numpy() + 1j * im.double().numpy()
    for inverse in (False, True):
        got = _gpu_fft(re, im, inverse)
        ref = np.fft.ifft(x, axis=-1) if inverse else np.fft.fft(x, axis=-1)
        assert rel_l2(*got, ref.real, ref.imag) <= tol_pow2(n), (n, inverse)


def test_pow2_2_24_real_input_and_in_place():
    # 2^24 real input (the first strided pass's real-input variant) and an in-place call through
    # the C ABI (the last pass writes the output after the first has read all input)
    import ctypes

    from trnfft_amd import _lib
    from trnfft_amd.dispatch import ptr, stream_handle
    from trnfft_amd.plan import native_plan

    n = 1 << 24
    re, im = seeded_complex(1, n, seed=5)
    X = trnfft_amd.fft(re.cuda())
    e = np.fft.fft(re.double().numpy(), axis=-1)
    assert rel_l2(X.real, X.imag, e.real, e.imag) <= tol_pow2(n)
    plan = native_plan(_lib.KIND_C2C, n, False, 0)
    nbytes = ctypes.c_size_t(0)
    lib = _lib.lib()
    assert lib.tfa_plan_workspace_size(plan.handle, 1, ctypes.byref(nbytes)) == 0
    ws = torch.empty(nbytes.value // 4, device="cuda")
    d_re, d_im = re.cuda(), im.cuda()
    rc = lib.tfa_execute(plan.handle, 1, ptr(d_re), ptr(d_im), ptr(d_re), ptr(d_im), ptr(ws),
                         stream_handle(torch.device("cuda", 0)))
    assert rc == 0
    torch.cuda.synchronize()
    e = np.fft.fft(re.double().numpy() + 1j * im.double().numpy(), axis=-1)
    assert rel_l2(d_re, d_im, e.real, e.imag) <= tol_pow2(n)


@pytest.mark.parametrize("n", [1 << 15, 1 << 20])
def test_pow2_fourstep_real_input(n):
    # real rows take the column pass's real-input variant (imaginary plane never read)
    re, _ = seeded_complex(3, n, seed=7)
    X = trnfft_amd.fft(re.cuda())
    ref = oracle.fft_core(re, torch.zeros_like(re), False)
    assert rel_l2(X.real, X.imag, *ref) <= tol_pow2(n)


def test_config1_batched_1024_roundtrip():
    # 4096 x 1024, forward then inverse, each against the oracle
    re, im = seeded_complex(4096, 1024)
    x = ComplexTensor(re.cuda(), im.cuda())
    X = trnfft_amd.fft(x)
    ref = oracle.fft_core(re, im, False)
    assert rel_l2(X.real, X.imag, *ref) <= tol_pow2(1024)
    back = trnfft_amd.ifft(X)
    ref_back = oracle.fft_core(ref[0], ref[1], True)
    assert rel_l2(back.real, back.imag, *ref_back) <= tol_pow2(1024)
    assert rel_l2(back.real, back.imag, re, im) <= 2 * tol_pow2(1024)


def test_config4b_large_n_properties():
    # BASELINE config 4b at full size (16 x 2^20): oracle on one row, round trip + Parseval on all
    n = 1 << 20
    re, im = seeded_complex(16, n)
    x = ComplexTensor(re.cuda(), im.cuda())
    X = trnfft_amd.fft(x)
    ref0 = oracle.fft_core(re[:1], im[:1], False)
    assert rel_l2(X.real[:1], X.imag[:1], *ref0) <= tol_pow2(n)
    e_t = (re.double() ** 2 + im.double() ** 2).sum()
    e_f = (X.real.double() ** 2 + X.imag.double() ** 2).sum().cpu() / n
    assert abs(e_t - e_f) / e_t < 1e-5
    back = trnfft_amd.ifft(X)
    assert rel_l2(back.real, back.imag, re, im) <= 2 * tol_pow2(n)


def test_real_input_and_known_answers():
    n = 16
    x = torch.zeros(n)
    x[0] = 1.0
    y = trnfft_amd.fft(x)  # CPU tensor in, CPU result out
    assert y.real.device.type == "cpu"
    np.testing.assert_allclose(y.real.numpy(), np.ones(n), atol=1e-6)
    np.testing.assert_allclose(y.imag.numpy(), np.zeros(n), atol=1e-6)
    g = torch.Generator().manual_seed(42)
    r = torch.randn(5, 1024, generator=g)
    got = trnfft_amd.fft(r.cuda())
    ref = oracle.fft_core(r, torch.zeros_like(r), False)
    assert rel_l2(got.real, got.imag, *ref) <= tol_pow2(1024)
    z = trnfft_amd.fft(torch.tensor([1.0, 2.0, 3.0, 4.0]), n=8)
    e = np.fft.fft([1, 2, 3, 4, 0, 0, 0, 0])
    np.testing.assert_allclose(z.real.numpy(), e.real, atol=1e-5)
    np.testing.assert_allclose(z.imag.numpy(), e.imag, atol=1e-5)


def test_leading_dims_and_empty_batch():
    re, im = seeded_complex(6, 256)
    x = ComplexTensor(re.reshape(2, 3, 256).cuda(), im.reshape(2, 3, 256).cuda())
    y = trnfft_amd.fft(x)
    assert y.shape == (2, 3, 256)
    ref = oracle.fft_core(re, im, False)
    assert rel_l2(y.real.reshape(6, 256), y.imag.reshape(6, 256), *ref) <= tol_pow2(256)
    e = trnfft_amd.fft(ComplexTensor(torch.zeros(0, 64, device="cuda"), torch.zeros(0, 64, device="cuda")))
    assert e.shape == (0, 64)


@pytest.mark.parametrize("direction", ["fft", "ifft"])
def test_bluestein_vs_reference_golden(direction):
    d = np.load(GOLDEN)
    for n, _b in d["cases"]:
        re = torch.from_numpy(d[f"n{n}_in_re"])
        im = torch.from_numpy(d[f"n{n}_in_im"])
        got = _gpu_fft(re, im, direction == "ifft")
        err = rel_l2(*got, d[f"n{n}_{direction}_re"], d[f"n{n}_{direction}_im"])
        assert err <= tol_bluestein(int(n)), (int(n), direction, err)


@pytest.mark.parametrize("n,batch", [(1000, 1024), (4099, 256), (3, 5), (17, 33), (8193, 4), (20000, 2),
                                     # the mixed-radix fused length 9216 = 12^2 * 64 covers
                                     # 4104 < n <= 4608 (reference m = 16384; 4097..4104 wrap at
                                     # 8192), 12288 = 24 * 8^3 covers 4608 < n <= 6144 from 28 rows
                                     # (fewer: the split path at 16384); 6145 pads to 16384
                                     (4097, 3), (4097, 300), (4200, 9), (4608, 70), (4609, 70), (4609, 5),
                                     (5000, 27), (5000, 28), (6144, 41), (6145, 41),
                                     # short rows (m <= 64 staged through LDS as one run per
                                     # workgroup): full tiles plus a ragged one, every padded length
                                     # 4..256 and real input below
                                     (2, 600), (5, 1000), (7, 257), (12, 300), (31, 513), (33, 129),
                                     (60, 200), (100, 130), (127, 65), (129, 3)])
@pytest.mark.parametrize("inverse", [False, True])
def test_bluestein_vs_oracle(n, batch, inverse):
    re, im = seeded_complex(batch, n, seed=n)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_bluestein(n), (n, inverse)


@pytest.mark.parametrize("n", [3, 12, 100])
def test_bluestein_short_rows_real_input(n):
    re, _ = seeded_complex(301, n, seed=n + 1)
    X = trnfft_amd.fft(re.cuda())
    ref = oracle.fft_core(re, torch.zeros_like(re), False)
    assert rel_l2(X.real, X.imag, *ref) <= tol_bluestein(n)


@pytest.mark.parametrize("n,batch,real_in", [(257, 40, False), (300, 64, True), (384, 33, False), (513, 20, False),
                                              (700, 17, True), (768, 9, False), (1025, 12, False), (1300, 7, True),
                                              (1536, 5, False), (1537, 3, False), (4200, 9, False)])
def test_bluestein_mixed_radix_lengths_vs_oracle(n, batch, real_in):
    # the fused kernel convolves at 768, 1536, 3072 or 9216 points where those hold 2n - 1 and are
    # shorter than the reference's power of two (n = 1537 stays at 4096)
    g = torch.Generator().manual_seed(n)
    re = torch.randn(batch, n, generator=g)
    im = torch.zeros_like(re) if real_in else torch.randn(batch, n, generator=g)
    x = re.cuda() if real_in else ComplexTensor(re.cuda(), im.cuda())
    got = trnfft_amd.fft(x)
    ref = oracle.fft_core(re, im, False)
    assert rel_l2(got.real, got.imag, *ref) <= tol_bluestein(n)
    # the inverse against the oracle's inverse of the same spectrum (the reference's fp32 chirp
    # keeps its own round trip ~1e-4 from the identity at n in the thousands)
    back = trnfft_amd.ifft(got)
    ref_back = oracle.fft_core(got.real.cpu(), got.imag.cpu(), True)
    assert rel_l2(back.real, back.imag, *ref_back) <= tol_bluestein(n)


@pytest.mark.parametrize("n,batch", [(129, 300), (136, 64), (1025, 40), (1032, 7), (2049, 33), (2056, 3),
                                     (4097, 256), (4099, 256), (4104, 5), (8193, 64), (8200, 70),
                                     # below 64 rows n = 8193..8200 take the split path at 32768
                                     (8193, 3), (8200, 20)])
@pytest.mark.parametrize("inverse", [False, True])
def test_bluestein_wrapped_lengths_vs_oracle(n, batch, inverse):
    # n = 2^k + 1 .. 2^k + 8: the fused kernel convolves circularly at 2^(k+1) < 2n - 1 and corrects
    # the 2 * (2n - 1 - 2^(k+1)) outputs the wrapped filter taps reach (wrap 1 .. 15)
    re, im = seeded_complex(batch, n, seed=n + 5)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_bluestein(n), (n, inverse)
    # the corrected outputs at both ends, against the exact DFT of the same rows (the fp32 chirp's
    # deviation is spread over all bins, so the ends must not stand out from the rest)
    x = re.double().numpy() + 1j * im.double().numpy()
    exact = np.fft.ifft(x, axis=-1) if inverse else np.fft.fft(x, axis=-1)
    g = got[0].double().numpy() + 1j * got[1].double().numpy()
    ends = np.r_[0:16, n - 16:n]
    e_ends = np.linalg.norm(g[:, ends] - exact[:, ends]) / np.linalg.norm(exact[:, ends])
    e_all = np.linalg.norm(g - exact) / np.linalg.norm(exact)
    assert e_ends <= 3 * e_all + 1e-6, (n, e_ends, e_all)


@pytest.mark.parametrize(
    "n,batch",
    [(769, 70), (1000, 33), (1024, 5), (1031, 129), (1537, 40), (1700, 257), (2048, 9), (2057, 64), (3000, 130),
     (4096, 17), (6145, 40), (7000, 36), (8192, 37), (8193, 9), (8200, 50)],
)
@pytest.mark.parametrize("inverse", [False, True])
def test_bluestein_two_level_lengths_vs_oracle(n, batch, inverse):
    # convolution lengths 2048 (n = 769..1024, and 1031 wrapped by 13), 4096 (n = 1537..2048),
    # 8192 (n = 2057..4096) and 16384 (n = 6145..8192 from 36 rows, 8193..8200 wrapped at every
    # batch) run the two-level fused kernel (one exchange into 512-point wave transforms, 1024-point
    # ones at 16384, and one back, the filter spectrum in the waves' frequency order, the cross
    # factors formed from a per-lane and a wave-uniform part); complex and real input, against
    # the oracle's Bluestein
    re, im = seeded_complex(batch, n, seed=n + 13)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_bluestein(n), (n, inverse)
    X = trnfft_amd.ifft(re.cuda()) if inverse else trnfft_amd.fft(re.cuda())
    ref = oracle.fft_core(re, torch.zeros_like(re), inverse)
    assert rel_l2(X.real, X.imag, *ref) <= tol_bluestein(n), (n, inverse, "real input")


@pytest.mark.parametrize("n", [1027, 4099])
def test_bluestein_wrapped_real_input_and_strided_axis(n):
    # real input through the wrapped fused kernel, and a strided axis (n = 1027: m = 4096 runs the
    # strided-axis kernel at the reference's length while the contiguous rows wrap at 2048)
    re, _ = seeded_complex(9, n, seed=3)
    X = trnfft_amd.fft(re.cuda())
    ref = oracle.fft_core(re, torch.zeros_like(re), False)
    assert rel_l2(X.real, X.imag, *ref) <= tol_bluestein(n)
    if n <= 4096:
        xt = re.t().contiguous()  # (n, 9): transform along dim 0
        Y = trnfft_amd.fftn(xt.cuda(), dim=(0,))
        assert rel_l2(Y.real.t(), Y.imag.t(), *ref) <= tol_bluestein(n)


@pytest.mark.parametrize("n", [4099, 6000, 7000])
@pytest.mark.parametrize("inverse", [False, True])
def test_bluestein_fused_and_split_paths_agree(n, inverse):
    # n = 6000 (m = 16384) runs the fused one-row-per-workgroup kernel at 12288 points for large
    # batches and the split three-pass path at 16384 for small ones; n = 4099 runs the wrapped
    # 8192-point fused kernel at every batch; rows must agree across batch sizes, and both are
    # checked against the oracle
    re, im = seeded_complex(2048, n, seed=11)
    fused = _gpu_fft(re, im, inverse)  # 2048 rows: fused kernel
    small = _gpu_fft(re[:5], im[:5], inverse)  # 5 rows: split path for n = 6000
    assert rel_l2(fused[0][:5], fused[1][:5], *small) <= tol_bluestein(n)
    ref = oracle.fft_core(re[:5], im[:5], inverse)
    assert rel_l2(fused[0][:5], fused[1][:5], *ref) <= tol_bluestein(n)
    assert rel_l2(*small, *ref) <= tol_bluestein(n)


@pytest.mark.parametrize("n,batch", [(70000, 1), ((1 << 20) + 1, 1)])
@pytest.mark.parametrize("inverse", [False, True])
def test_bluestein_split_large_vs_oracle(n, batch, inverse):
    # split path at m = 262144 (512 x 512) and m = 2^22 (2048 x 2048).  The reference's fp32
    # chirp angle makes its operator drift from the exact DFT as n grows, so parity is against
    # the oracle's restatement of that operator, not a round trip
    re, im = seeded_complex(batch, n, seed=n % 997)
    got = _gpu_fft(re, im, inverse)
    ref = oracle.fft_core(re, im, inverse)
    assert rel_l2(*got, *ref) <= tol_bluestein(n), (n, inverse)


def test_bluestein_largest_length_and_beyond():
    # the longest Bluestein axis the library takes, n = 2^23 - 1 (padded m = 2^24, the split
    # three-pass path), against the oracle (fp32 chirp included) in both directions; one sample
    # more would pad to 2^25 and is refused with NotImplementedError
    n = (1 << 23) - 1
    assert trnfft_amd.create_plan(n).padded_n == 1 << 24
    re, im = seeded_complex(1, n, seed=9)
    for inverse in (False, True):
        y = _gpu_fft(re, im, inverse)
        ref = oracle.fft_core(re, im, inverse)
        assert rel_l2(*y, *ref) <= tol_bluestein(n), inverse
    big = (1 << 23) + 1
    with pytest.raises(NotImplementedError):
        trnfft_amd.fft(ComplexTensor(torch.zeros(1, big, device="cuda"), torch.zeros(1, big, device="cuda")))
