"""Host-side logic that runs without a GPU: C ABI exports and argument errors, plan selection,
backend dispatch semantics, ComplexTensor arithmetic (reference tests/test_complex.py)."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import trnfft_amd
from trnfft_amd import ComplexTensor, _lib
from trnfft_amd.plan import FFTAlgorithm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trnfft_amd.h")


def _declared_symbols() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"\b(tfa_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_symbols()
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.tfa_abi_version() >> 16 == 1


def test_abi_rejects_bad_arguments_without_gpu():
    lib = _lib.lib()
    h = ctypes.c_void_p()
    assert lib.tfa_plan_create(ctypes.byref(h), None) == _lib.TFA_ERR_INVALID
    desc = _lib.PlanDesc(kind=_lib.KIND_C2C, inverse=0, n=0, hop=0, flags=0, reserved=0)
    assert lib.tfa_plan_create(ctypes.byref(h), ctypes.byref(desc)) == _lib.TFA_ERR_INVALID
    assert b"length" in lib.tfa_last_error()
    assert lib.tfa_execute(None, 1, None, None, None, None, None, None) == _lib.TFA_ERR_INVALID
    nbytes = ctypes.c_size_t(7)
    assert lib.tfa_strided_workspace_size(None, 1, 16, ctypes.byref(nbytes)) == _lib.TFA_ERR_INVALID
    assert lib.tfa_execute_strided_ws(None, 1, 16, None, None, None, None, None, None) == _lib.TFA_ERR_INVALID
    assert lib.tfa_execute_strided(None, 1, 16, None, None, None, None, None) == _lib.TFA_ERR_INVALID
    with pytest.raises(ValueError):
        _lib.check(_lib.TFA_ERR_INVALID, "x")


def test_create_plan_matches_reference_choice():
    # trnfft/plan.py:34-46
    trnfft_amd.clear_plan_cache()
    p = trnfft_amd.create_plan(1024)
    assert p.algorithm == FFTAlgorithm.COOLEY_TUKEY and p.padded_n is None and p.is_power_of_2
    for n, m in [(1000, 2048), (4099, 16384), (997, 2048), (4097, 16384), (7, 16)]:
        p = trnfft_amd.create_plan(n, inverse=True)
        assert p.algorithm == FFTAlgorithm.BLUESTEIN and p.padded_n == m and p.inverse
    assert trnfft_amd.create_plan(1000, True) is trnfft_amd.create_plan(1000, True)


def test_fft2_shape_gates():
    # the single-pass small-image kernel: powers of two, h*w <= 16384, both axes >= 4 and >= its
    # elements per thread (4 up to 4096 elements, 8 at 8192, 16 at 16384); two passes otherwise
    from trnfft_amd.fft_core import fft2_ok, fft2_small_ok

    for h, w in [(4, 4), (4, 64), (64, 4), (16, 16), (128, 128), (8, 1024), (1024, 8), (16, 1024), (1024, 16)]:
        assert fft2_small_ok(h, w), (h, w)
    for h, w in [(2, 64), (64, 2), (4, 2048), (8, 2048), (256, 128), (12, 16), (3, 3)]:
        assert not fft2_small_ok(h, w), (h, w)
    assert fft2_ok(4, 4) and fft2_ok(16, 2048) and fft2_ok(4096, 16) and not fft2_ok(4, 2048)
    assert fft2_ok(16, 4096) and fft2_ok(4096, 4096) and not fft2_ok(8192, 16) and not fft2_ok(16, 8192)
    # complex input: two-pass kernels only for 256 <= w <= 512 with h >= 512; small images always
    assert fft2_ok(512, 512, False) and fft2_ok(4096, 256, False) and fft2_ok(64, 64, False)
    assert not fft2_ok(1024, 1024, False) and not fft2_ok(256, 256, False) and not fft2_ok(2048, 64, False)


def test_strided_axis_gates():
    # strided-axis kernels in place of transposes: power-of-two n <= 4096 and other n <= 2048 at
    # any stride; power-of-two n up to 2^24 with >= 4 trailing columns (>= 8 from 2^21)
    from trnfft_amd.fft_core import strided_ok

    for n, s in [(2, 1), (4096, 1), (3, 7), (2047, 1), (2048, 1), (8192, 4), (1 << 20, 4), (1 << 21, 8),
                 (1 << 24, 8), (1 << 24, 1000)]:
        assert strided_ok(n, s), (n, s)
    for n, s in [(8192, 3), (1 << 20, 1), (1 << 21, 7), (1 << 24, 4), (1 << 25, 64), (2049, 16), (4099, 64),
                 (1, 4), (16, 0)]:
        assert not strided_ok(n, s), (n, s)


def test_backend_selection_semantics():
    assert trnfft_amd.get_backend() == "auto"
    with pytest.raises(AssertionError):
        trnfft_amd.set_backend("nki")
    trnfft_amd.set_backend("pytorch")
    try:
        with pytest.raises(RuntimeError, match="pytorch"):
            trnfft_amd.fft(torch.randn(8))
    finally:
        trnfft_amd.set_backend("auto")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_fails_loudly_without_gpu():
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        trnfft_amd.fft(torch.randn(4, 64))
    with pytest.raises(RuntimeError):
        trnfft_amd.set_backend("hip")


def test_precision_modes():
    assert trnfft_amd.get_precision() == "fast"
    with pytest.raises(ValueError):
        trnfft_amd.set_precision("bogus")
    from trnfft_amd.precision import _resolve

    assert _resolve(None) == "fast"
    with pytest.raises(NotImplementedError):
        _resolve("double")
    # the reference's Ozaki toggle exists (trnfft/__init__.py:66); the modes stay unsupported
    trnfft_amd.set_ozaki_product_precision_verified(True)
    with pytest.raises(NotImplementedError):
        _resolve("ozaki")
    trnfft_amd.set_ozaki_product_precision_verified(False)


def test_hip_accepts_only_fp32_under_fast_precision(monkeypatch):
    # the integration hooks route a call here only when this predicate holds; everything else
    # stays on trnfft's own path (the reference computes in the input's dtype, fft_core.py:84-88,
    # and runs "kahan"/"double" itself)
    from trnfft_amd import dispatch

    monkeypatch.setattr(dispatch, "_use_hip", lambda: True)
    x32, x64 = torch.randn(4, 8), torch.randn(4, 8, dtype=torch.float64)
    assert trnfft_amd.hip_accepts(x32, x32, precision="fast")
    assert trnfft_amd.hip_accepts(x32, None)
    assert not trnfft_amd.hip_accepts(x64, x64, precision="fast")
    assert not trnfft_amd.hip_accepts(x32, x64)
    assert not trnfft_amd.hip_accepts(x32.half())
    assert not trnfft_amd.hip_accepts(x32.to(torch.bfloat16))
    assert not trnfft_amd.hip_accepts(torch.complex(x32, x32))
    assert not trnfft_amd.hip_accepts(torch.arange(8))
    for mode in ("kahan", "double", "bf16", "bf16_refined", "ozaki", "ozaki_hq", "bogus"):
        assert not trnfft_amd.hip_accepts(x32, precision=mode), mode
    # the backend's own switch still decides for fp32 / "fast"
    monkeypatch.setattr(dispatch, "_use_hip", lambda: False)
    assert not trnfft_amd.hip_accepts(x32, x32, precision="fast")


def test_hook_keeps_other_precisions_and_dtypes_off_the_hip_path(monkeypatch):
    # the fft_core hook of the integration guide: resolve trnfft's precision first, then route by
    # the predicate; a stand-in for trnfft's own path records what it was given
    from trnfft_amd import dispatch

    monkeypatch.setattr(dispatch, "_use_hip", lambda: True)
    routed = []

    def hook(x_re, x_im, precision, global_mode):
        prec = global_mode if precision is None else precision  # trnfft/precision.py:88-94
        if trnfft_amd.hip_accepts(x_re, x_im, precision=prec):
            routed.append(("hip", prec))
        else:
            routed.append(("trnfft", prec))

    x = torch.randn(2, 16)
    hook(x, x, None, "fast")
    hook(x, x, None, "double")
    hook(x, x, "kahan", "fast")
    hook(x.double(), x.double(), None, "fast")
    assert routed == [("hip", "fast"), ("trnfft", "double"), ("trnfft", "kahan"), ("trnfft", "fast")]


def test_backend_refuses_rather_than_computing_fp32():
    # asked directly, the backend raises for what it does not compute: another precision mode
    # (NotImplementedError, before any device work) or non-fp32 data (TypeError)
    x = ComplexTensor(torch.randn(2, 16), torch.randn(2, 16))
    for mode in ("double", "kahan"):
        with pytest.raises(NotImplementedError):
            trnfft_amd.fft_core.fft_core(x, precision=mode)
    trnfft_amd.set_precision("double")
    try:
        for call in (lambda: trnfft_amd.fft(x), lambda: trnfft_amd.stft(torch.randn(2, 600), 64),
                     lambda: trnfft_amd.fft2(torch.randn(2, 8, 8)), lambda: trnfft_amd.rfft(torch.randn(2, 16))):
            with pytest.raises(NotImplementedError):
                call()
    finally:
        trnfft_amd.set_precision("fast")
    from trnfft_amd.dispatch import to_device_f32

    with pytest.raises(TypeError):
        to_device_f32(torch.randn(4, dtype=torch.float64), torch.device("cpu"))


class TestComplexTensor:
    def test_from_real_and_complex(self):
        x = ComplexTensor(torch.tensor([1.0, 2.0, 3.0]))
        assert x.imag.sum().item() == 0.0
        z = torch.complex(torch.tensor([1.0, 2.0]), torch.tensor([3.0, 4.0]))
        y = ComplexTensor(z)
        np.testing.assert_allclose(y.real.numpy(), [1.0, 2.0])
        np.testing.assert_allclose(y.imag.numpy(), [3.0, 4.0])

    def test_arithmetic(self):
        a = ComplexTensor(torch.tensor([1.0]), torch.tensor([2.0]))
        b = ComplexTensor(torch.tensor([3.0]), torch.tensor([4.0]))
        c = a * b
        assert c.real.item() == -5.0 and c.imag.item() == 10.0
        d = a + b
        assert d.real.item() == 4.0 and d.imag.item() == 6.0
        e = b - a
        assert e.real.item() == 2.0 and e.imag.item() == 2.0
        f = -a
        assert f.real.item() == -1.0
        g = a.conj()
        assert g.imag.item() == -2.0
        assert abs(ComplexTensor(torch.tensor([3.0]), torch.tensor([4.0])).abs().item() - 5.0) < 1e-6

    def test_views_are_contiguous_copies(self):
        x = ComplexTensor(torch.randn(3, 4), torch.randn(3, 4))
        t = x.transpose(0, 1)
        assert t.shape == (4, 3) and t.real.is_contiguous()
        assert x.reshape(12).shape == (12,)
        assert x[1].shape == (4,)
        with pytest.raises(AssertionError):
            ComplexTensor(torch.randn(2), torch.randn(3))


def test_reference_public_names_are_exported():
    # every name of the reference's public API (trnfft/__init__.py:36-68, __all__) exists here
    names = ["fft", "ifft", "rfft", "hfft", "ihfft", "irfft", "fft2", "fftn", "ifftn", "rfft2", "irfft2", "rfftn",
             "irfftn", "stft", "istft", "ComplexTensor", "complex_matmul", "create_plan", "clear_plan_cache", "FFTPlan",
             "HAS_NKI", "set_backend", "get_backend", "set_precision", "set_ozaki_product_precision_verified",
             "get_precision"]
    missing = [n for n in names if not hasattr(trnfft_amd, n)]
    assert not missing, missing
    assert trnfft_amd.HAS_NKI is False


class _FakePlan:
    """Stand-in for NativePlan (no device): records its own release."""

    released: list = []

    def __init__(self, kind, n, inverse, device, hop=0, flags=0, n2=0):
        self.key = (kind, n, inverse)

    def __del__(self):
        _FakePlan.released.append(self.key)


def test_plan_cache_keeps_a_held_plan_alive_across_clear():
    # a caller that fetched a plan keeps it until it drops the reference: clear_plan_cache only
    # drops the cache's own reference (no explicit destroy under a running call)
    import gc

    from trnfft_amd import plan as P

    P.clear_plan_cache()
    _FakePlan.released.clear()
    held = P.native_plan(99, 8, False, 0, _factory=_FakePlan)
    assert P.native_plan(99, 8, False, 0, _factory=_FakePlan) is held
    P.clear_plan_cache()
    gc.collect()
    assert _FakePlan.released == []
    del held
    gc.collect()
    assert _FakePlan.released == [(99, 8, False)]


def test_plan_cache_is_bounded_lru():
    import gc

    from trnfft_amd import plan as P

    P.clear_plan_cache()
    _FakePlan.released.clear()
    first = [P.native_plan(98, n, False, 0, _factory=_FakePlan) for n in range(P.NATIVE_CACHE_MAX)]
    keep = first[0]
    P.native_plan(98, 0, False, 0, _factory=_FakePlan)  # touch: most recently used now
    del first
    extra = [P.native_plan(98, 1000 + i, False, 0, _factory=_FakePlan) for i in range(5)]
    gc.collect()
    assert len(P._native_cache) == P.NATIVE_CACHE_MAX
    # the five least recently used (1..5) were evicted; 0 was touched and is held anyway
    assert sorted(k[1] for k in _FakePlan.released) == [1, 2, 3, 4, 5]
    assert (98, 0, False, 0, 0, 0, 0) in P._native_cache
    del keep, extra
    P.clear_plan_cache()
    gc.collect()


def _wrapped_bluestein(x, m, sign=-1):
    """Bluestein at a circular length m < 2n - 1 with the colliding filter taps summed and the
    outputs they reach corrected (the fused kernel's wrapped lengths), in float64."""
    n = len(x)
    d = 2 * n - 1 - m
    k = np.arange(n)
    chirp = np.exp(sign * 1j * np.pi * ((k * k) % (2 * n)) / n)
    y = x * chirp
    h = np.zeros(m, complex)
    for i in range(n):
        h[i] += np.conj(chirp[i])
        if i > 0:
            h[m - i] += np.conj(chirp[i])
    yp = np.zeros(m, complex)
    yp[:n] = y
    conv = np.fft.ifft(np.fft.fft(yp) * np.fft.fft(h))[:n]
    lo = n - d
    yl, yh, ct = y[:d], y[lo:n], chirp[lo:n]
    for i in range(min(d, n)):  # outputs k < d: extra taps from y[lo + c], c >= k
        conv[i] -= sum(yh[c] * np.conj(ct[d - 1 + i - c]) for c in range(i, d))
    for i in range(lo, n):  # outputs k >= n - d: extra taps from y[j], j <= k - lo
        a = i - lo
        conv[i] -= sum(yl[j] * np.conj(ct[d - 1 - a + j]) for j in range(a + 1))
    return conv * chirp


@pytest.mark.parametrize("n,m", [(3, 4), (5, 8), (7, 8), (65, 128), (72, 128), (129, 256), (4099, 8192),
                                 (4104, 8192)])
def test_wrapped_bluestein_correction_is_exact(n, m):
    # the identity the fused kernel's wrapped lengths rely on, against numpy's DFT (float64);
    # dropping either correction (or flipping a conjugate) leaves errors of order 1e-3 at the ends
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    got = _wrapped_bluestein(x, m)
    ref = np.fft.fft(x)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-13
