"""C ABI argument checking on a GPU (plans need a device): every rejected call returns its status
code and leaves a message, as include/trnfft_amd.h documents, and launches nothing."""

from __future__ import annotations

import ctypes

import pytest
import torch

from trnfft_amd import _lib

pytestmark = pytest.mark.gpu

VP = ctypes.c_void_p


def _plan(kind, n, inverse=0, hop=0, flags=0, n2=0):
    h = VP()
    d = _lib.PlanDesc(kind=kind, inverse=inverse, n=n, hop=hop, flags=flags, reserved=0, n2=n2)
    rc = _lib.lib().tfa_plan_create(ctypes.byref(h), ctypes.byref(d))
    return rc, h


def _err():
    return _lib.lib().tfa_last_error().decode()


def P(t):
    return VP(t.data_ptr()) if t is not None else None


def test_plan_kind_limits():
    lib = _lib.lib()
    for kind, n, extra in [(_lib.KIND_REAL, 3, {}), (_lib.KIND_REAL, 65536, {}), (_lib.KIND_C2C, 1000, {}),
                           (_lib.KIND_STFT, 3000, {"hop": 10}), (_lib.KIND_STFT, 6, {"hop": 2}),
                           (_lib.KIND_STFT, 2049, {"hop": 10}),  # two-sided: 4097 points
                           (_lib.KIND_STFT, 400, {"hop": 100, "inverse": 1}),  # two-sided inverse
                           (_lib.KIND_STFT, 400, {"hop": 10, "inverse": 1, "flags": _lib.STFT_ONESIDED}),  # halo
                           (_lib.KIND_STFT, 2049, {"hop": 500, "inverse": 1, "flags": _lib.STFT_ONESIDED}),
                           (_lib.KIND_STFT, 8192, {"hop": 10}), (_lib.KIND_FFT2, 8192, {"n2": 64}),
                           (_lib.KIND_STFT, 512, {"hop": 0}), (_lib.KIND_DFT_GEMM, 8192, {}), (99, 8, {})]:
        rc, h = _plan(kind, n, **extra)
        assert rc in (_lib.TFA_ERR_INVALID, _lib.TFA_ERR_UNSUPPORTED), (kind, n, rc)
        assert not h.value and _err()
    # inverse STFT: two-sided spectra at a power-of-two n_fft are accepted, at other n_fft refused;
    # too-short hops are refused at plan time
    rc, h = _plan(_lib.KIND_STFT, 512, inverse=1, hop=128, flags=_lib.STFT_CENTER)
    assert rc == 0 and h.value
    lib.tfa_plan_destroy(h)
    rc, _ = _plan(_lib.KIND_STFT, 400, inverse=1, hop=160, flags=_lib.STFT_CENTER)
    assert rc == _lib.TFA_ERR_UNSUPPORTED and "onesided" in _err()
    rc, _ = _plan(_lib.KIND_STFT, 4096, inverse=1, hop=16, flags=_lib.STFT_ONESIDED)
    assert rc == _lib.TFA_ERR_UNSUPPORTED and "hop" in _err()
    # n_fft 4096, hop 512 (halo 7): the onesided tile holds 8 frames, the two-sided one 4
    rc, h = _plan(_lib.KIND_STFT, 4096, inverse=1, hop=512, flags=_lib.STFT_ONESIDED)
    assert rc == 0 and h.value
    lib.tfa_plan_destroy(h)
    rc, _ = _plan(_lib.KIND_STFT, 4096, inverse=1, hop=512, flags=0)
    assert rc == _lib.TFA_ERR_UNSUPPORTED and "hop" in _err()
    assert lib.tfa_abi_version() >> 16 == 1


def test_real_plan_argument_checks():
    lib = _lib.lib()
    st = VP(torch.cuda.current_stream().cuda_stream)
    rc, fwd = _plan(_lib.KIND_REAL, 256)
    assert rc == 0
    rc, inv = _plan(_lib.KIND_REAL, 256, inverse=1)
    assert rc == 0
    x = torch.randn(4, 256, device="cuda")
    re = torch.empty(4, 129, device="cuda")
    im = torch.empty_like(re)
    # r2c takes real input: an imaginary plane is refused
    assert lib.tfa_execute(fwd, 4, P(x), P(x), P(re), P(im), None, st) == _lib.TFA_ERR_INVALID
    # real rows must be 8-byte aligned
    flat = torch.randn(1 + 4 * 256, device="cuda")
    assert lib.tfa_execute(fwd, 4, VP(flat.data_ptr() + 4), None, P(re), P(im), None, st) == _lib.TFA_ERR_INVALID
    # c2r: both input planes needed, no aliasing of the output with an input
    y = torch.empty(4, 256, device="cuda")
    assert lib.tfa_execute(inv, 4, P(re), None, P(y), None, None, st) == _lib.TFA_ERR_INVALID
    assert lib.tfa_execute(inv, 4, P(re), P(im), P(re), None, None, st) == _lib.TFA_ERR_INVALID
    # valid calls succeed
    assert lib.tfa_execute(fwd, 4, P(x), None, P(re), P(im), None, st) == 0
    assert lib.tfa_execute(inv, 4, P(re), P(im), P(y), None, None, st) == 0
    torch.cuda.synchronize()
    torch.testing.assert_close(y, x, rtol=1e-5, atol=1e-5)
    lib.tfa_plan_destroy(fwd)
    lib.tfa_plan_destroy(inv)


def test_gemm_ex_argument_checks():
    lib = _lib.lib()
    st = VP(torch.cuda.current_stream().cuda_stream)
    a = torch.randn(8, 4, device="cuda")
    b = torch.randn(4, 6, device="cuda")
    c = torch.empty(8, 6, device="cuda")
    d = torch.empty_like(c)
    ok = lib.tfa_complex_gemm_ex(8, 6, 4, P(a), P(a), 4, _lib.OP_N, P(b), P(b), 6, _lib.OP_N, 1.0, None, None,
                                 P(c), P(d), 6, st)
    assert ok == 0
    assert lib.tfa_complex_gemm_ex(8, 6, 4, P(a), P(a), 4, 7, P(b), P(b), 6, _lib.OP_N, 1.0, None, None,
                                   P(c), P(d), 6, st) == _lib.TFA_ERR_INVALID
    # transposed A is stored (k, m): lda must cover m
    assert lib.tfa_complex_gemm_ex(8, 6, 4, P(a), P(a), 4, _lib.OP_T, P(b), P(b), 6, _lib.OP_N, 1.0, None, None,
                                   P(c), P(d), 6, st) == _lib.TFA_ERR_INVALID
    assert lib.tfa_complex_gemm_ex(8, 6, 4, P(a), P(a), 4, _lib.OP_N, P(b), P(b), 6, _lib.OP_N, 1.0, P(b), None,
                                   P(c), P(d), 6, st) == _lib.TFA_ERR_INVALID
    torch.cuda.synchronize()


def test_bluestein_split_needs_workspace():
    lib = _lib.lib()
    st = VP(torch.cuda.current_stream().cuda_stream)
    # m = 32768: split path only (n = 8193..8200 wrap the fused kernel's 16384-point convolution)
    rc, p = _plan(_lib.KIND_BLUESTEIN, 8201)
    assert rc == 0
    size = ctypes.c_size_t()
    assert lib.tfa_plan_workspace_size(p, 2, ctypes.byref(size)) == 0 and size.value == 2 * 4 * 2 * 32768
    x = torch.randn(2, 8201, device="cuda")
    y = torch.empty_like(x)
    assert lib.tfa_execute(p, 2, P(x), P(x), P(y), P(y), None, st) == _lib.TFA_ERR_INVALID
    assert "workspace" in _err()
    lib.tfa_plan_destroy(p)


@pytest.mark.parametrize("n_fft,hop,onesided", [(512, 256, True), (400, 160, True), (64, 16, False), (100, 40, False)])
def test_stft_frames_major_planes_off_the_line_grid(n_fft, hop, onesided):
    # output planes that start 1 and 7 floats past a 128-byte line (the stores of each tile start
    # their lanes on a line, whatever the plane's alignment): the same values as aligned planes
    lib = _lib.lib()
    st = VP(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda").manual_seed(n_fft + 1)
    length = 7001
    x = torch.randn(2, length, device="cuda", generator=g)
    w = torch.hann_window(n_fft, device="cuda")
    bins = n_fft // 2 + 1 if onesided else n_fft
    frames = 1 + (length + 2 * (n_fft // 2) - n_fft) // hop
    fl = _lib.STFT_CENTER | _lib.STFT_FRAMES_MAJOR | (_lib.STFT_ONESIDED if onesided else 0)
    rc, h = _plan(_lib.KIND_STFT, n_fft, hop=hop, flags=fl)
    assert rc == 0, _err()
    cnt = 2 * frames * bins
    a_re, a_im = torch.empty(cnt, device="cuda"), torch.empty(cnt, device="cuda")
    flat_re = torch.full((cnt + 64,), float("nan"), device="cuda")
    flat_im = torch.full((cnt + 64,), float("nan"), device="cuda")
    b_re, b_im = flat_re[1:1 + cnt], flat_im[7:7 + cnt]
    assert lib.tfa_stft_execute(h, 2, length, P(x), P(w), P(a_re), P(a_im), st) == 0, _err()
    assert lib.tfa_stft_execute(h, 2, length, P(x), P(w), P(b_re), P(b_im), st) == 0, _err()
    torch.testing.assert_close(a_re, b_re, rtol=0, atol=0)
    torch.testing.assert_close(a_im, b_im, rtol=0, atol=0)
    # nothing written outside the planes
    assert torch.isnan(flat_re[:1]).all() and torch.isnan(flat_re[1 + cnt:]).all()
    assert torch.isnan(flat_im[:7]).all() and torch.isnan(flat_im[7 + cnt:]).all()
    torch.cuda.synchronize()
    lib.tfa_plan_destroy(h)


@pytest.mark.parametrize("n_fft,hop,onesided", [(512, 256, True), (400, 160, True), (64, 16, False), (100, 40, False),
                                                 (2048, 512, True)])
def test_stft_frames_major_layout(n_fft, hop, onesided):
    # TFA_STFT_FRAMES_MAJOR stores the same values as (batch, frames, bins): the forward output,
    # the inverse input and the backward's gradient input, bit for bit
    lib = _lib.lib()
    st = VP(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda").manual_seed(n_fft)
    length = 5000
    x = torch.randn(3, length, device="cuda", generator=g)
    w = torch.hann_window(n_fft, device="cuda")
    base = _lib.STFT_CENTER | (_lib.STFT_ONESIDED if onesided else 0)
    bins = n_fft // 2 + 1 if onesided else n_fft
    frames = 1 + (length + 2 * (n_fft // 2) - n_fft) // hop
    plans = []
    for fl in (base, base | _lib.STFT_FRAMES_MAJOR):
        rc, h = _plan(_lib.KIND_STFT, n_fft, hop=hop, flags=fl)
        assert rc == 0, _err()
        plans.append(h)
    a_re, a_im = torch.empty(3, bins, frames, device="cuda"), torch.empty(3, bins, frames, device="cuda")
    b_re, b_im = torch.empty(3, frames, bins, device="cuda"), torch.empty(3, frames, bins, device="cuda")
    assert lib.tfa_stft_execute(plans[0], 3, length, P(x), P(w), P(a_re), P(a_im), st) == 0
    assert lib.tfa_stft_execute(plans[1], 3, length, P(x), P(w), P(b_re), P(b_im), st) == 0
    torch.testing.assert_close(a_re, b_re.transpose(1, 2), rtol=0, atol=0)
    torch.testing.assert_close(a_im, b_im.transpose(1, 2), rtol=0, atol=0)
    if onesided:
        # the signal gradient on the forward plans: (gradient planes in each plan's layout)
        outs = []
        for h, (gr, gi) in zip(plans, [(a_re, a_im), (b_re, b_im)]):
            d = torch.empty(3, length + 2 * (n_fft // 2), device="cuda")
            rc = lib.tfa_stft_backward_execute(h, 3, frames, P(gr), P(gi), P(w), P(d), d.shape[1], st)
            assert rc == 0, _err()
            outs.append(d)
        torch.testing.assert_close(outs[0], outs[1], rtol=0, atol=0)
        # the inverse
        inv = []
        for fl in (base, base | _lib.STFT_FRAMES_MAJOR):
            rc, h = _plan(_lib.KIND_STFT, n_fft, inverse=1, hop=hop, flags=fl)
            assert rc == 0, _err()
            inv.append(h)
        ys = []
        for h, (gr, gi) in zip(inv, [(a_re, a_im), (b_re, b_im)]):
            y = torch.empty(3, length, device="cuda")
            assert lib.tfa_istft_execute(h, 3, frames, P(gr), P(gi), P(w), P(y), length, st) == 0, _err()
            ys.append(y)
        torch.testing.assert_close(ys[0], ys[1], rtol=0, atol=0)
        plans += inv
    torch.cuda.synchronize()
    for h in plans:
        lib.tfa_plan_destroy(h)
