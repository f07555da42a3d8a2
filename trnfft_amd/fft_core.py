"""1-D FFT entry point on the HIP kernels (contract of trnfft/fft_core.py:22-50).

``fft_core(x, inverse, plan, precision)`` transforms the last dimension of a ComplexTensor,
treating every leading dimension as batch, and returns new tensors:

* n == 1: a clone (trnfft/fft_core.py:41-42);
* power-of-two n: the LDS-resident Stockham kernel (n <= 16384) or the two-pass four-step
  kernel pair (n > 16384), replacing the radix-2 ``_cooley_tukey`` (:53-117) and the NKI
  Stockham/butterfly chain (:548-1238);
* any other n: the fused Bluestein kernel, replacing ``_bluestein`` (:1285-1376), with the chirp
  built from the reference's fp32 angle expression so results agree with the reference;
* ``_fft_via_gemm`` (:221-251): DFT as one complex GEMM on the matrix cores, taken when
  n <= ``_DFT_GEMM_THRESHOLD`` (0 by default: the Stockham kernel is faster on MI355X; the
  reference only routes here on its NKI backend).

Inverse transforms are scaled by 1/n inside the kernels, as the reference scales after its loop.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .complex import ComplexTensor
from .dispatch import _require_hip, ptr, stream_handle, target_device, to_device_f32
from .plan import FFTAlgorithm, FFTPlan, create_plan, native_plan
from .precision import _resolve

# n at or below which power-of-two transforms run as a DFT-GEMM (trnfft/fft_core.py:138 uses
# 256 on NKI); 0 keeps every length on the Stockham kernel.
_DFT_GEMM_THRESHOLD = 0


def fft_core(
    x: ComplexTensor,
    inverse: bool = False,
    plan: FFTPlan | None = None,
    precision: str | None = None,
) -> ComplexTensor:
    """Compute the 1-D FFT along the last dimension on the GPU."""
    _resolve(precision)
    n = x.shape[-1]
    if n == 1:
        return x.clone()
    if plan is None:
        plan = create_plan(n, inverse=inverse)
    _require_hip("fft_core")
    from . import autograd as _ag

    if plan.algorithm == FFTAlgorithm.COOLEY_TUKEY and n <= _DFT_GEMM_THRESHOLD and not _ag._grad_on(x.real, x.imag):
        return _fft_via_gemm(x, inverse)
    # differentiable when the planes require grad (adjoint on the same kernels)
    return _ag.c2c(x.real, x.imag, inverse)


def execute_1d(re: torch.Tensor, im: torch.Tensor | None, inverse: bool) -> ComplexTensor:
    """Run the batched transform of the last dimension; ``im=None`` means real input."""
    n = re.shape[-1]
    dev = target_device(re, im)
    out_dev = re.device
    re = to_device_f32(re, dev)
    im = to_device_f32(im, dev)
    if n == 1:
        out = ComplexTensor._wrap(re.clone(), im.clone() if im is not None else torch.zeros_like(re))
        return out if out_dev == dev else out.to(out_dev)
    batch = re.numel() // n if n else 0
    kind = _lib.KIND_C2C if (n & (n - 1)) == 0 else _lib.KIND_BLUESTEIN
    plan = native_plan(kind, n, inverse, dev.index)
    out_re = torch.empty_like(re)
    out_im = torch.empty_like(re)
    ws = None
    ws_bytes = plan.workspace_bytes(batch)
    if ws_bytes:
        ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_execute(
            plan.handle, batch, ptr(re), ptr(im), ptr(out_re), ptr(out_im), ptr(ws), stream_handle(dev)
        )
    _lib.check(rc, "tfa_execute")
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)


# real-row transforms through a half-length complex transform: power-of-two n in this range
_REAL_MIN_N, _REAL_MAX_N = 4, 32768


def real_ok(n: int) -> bool:
    return _REAL_MIN_N <= n <= _REAL_MAX_N and (n & (n - 1)) == 0


def _aligned8(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 8 == 0 else t.clone()


def execute_r2c(x: torch.Tensor) -> ComplexTensor:
    """Bins 0..n/2 of the transform of real rows (the last dimension), n a power of two in
    [4, 32768]: one half-length complex transform per row (replaces trnfft/api.py:38-46, which
    runs a full complex transform of (x, 0) and slices)."""
    n = x.shape[-1]
    dev = target_device(x, None)
    out_dev = x.device
    x = _aligned8(to_device_f32(x, dev).contiguous())
    batch = x.numel() // n
    plan = native_plan(_lib.KIND_REAL, n, False, dev.index)
    shape = (*x.shape[:-1], n // 2 + 1)
    out_re = torch.empty(shape, dtype=torch.float32, device=dev)
    out_im = torch.empty(shape, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_execute(plan.handle, batch, ptr(x), None, ptr(out_re), ptr(out_im), None, stream_handle(dev))
    _lib.check(rc, "tfa_execute")
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)


def execute_c2r(re: torch.Tensor, im: torch.Tensor, n: int) -> torch.Tensor:
    """Real rows of length n from bins 0..n/2 (n = 2*(bins-1), a power of two in [4, 32768]),
    scaled 1/n (replaces trnfft/api.py:49-68's Hermitian completion + complex inverse + .real)."""
    assert re.shape[-1] == n // 2 + 1
    dev = target_device(re, im)
    out_dev = re.device
    re = to_device_f32(re, dev).contiguous()
    im = to_device_f32(im, dev).contiguous()
    batch = re.numel() // (n // 2 + 1)
    plan = native_plan(_lib.KIND_REAL, n, True, dev.index)
    out = torch.empty((*re.shape[:-1], n), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_execute(plan.handle, batch, ptr(re), ptr(im), ptr(out), None, None, stream_handle(dev))
    _lib.check(rc, "tfa_execute")
    return out if out_dev == dev else out.to(out_dev)


# longest power-of-two axis the single-pass strided kernel transforms in place of a transpose
# round trip, longest other axis (Bluestein padded length m <= 4096), and the strided multi-pass
# path's reach (longer power-of-two axes: two passes with >= 4 trailing columns, three passes from
# 2^21 with >= 8; mirror of tfa::strided_fs_min_stride)
_STRIDED_MAX_N = 4096
_STRIDED_BLUE_MAX_N = 2048
_STRIDED_FS_MAX_N = 1 << 24
_STRIDED_FS_THREE_PASS_N = 1 << 21


def _strided_fs_min_stride(n: int) -> int:
    return 8 if n >= _STRIDED_FS_THREE_PASS_N else 4


def execute_strided(re: torch.Tensor, im: torch.Tensor | None, dim: int, inverse: bool) -> ComplexTensor:
    """Transform along a non-last axis `dim` without moving it: power-of-two n <= 4096 and
    other n <= 2048 in one strided pass, power-of-two 4096 < n <= 2^24 (stride >= 4, >= 8 from
    2^21) as a two- or three-pass strided four-step through a workspace (the library also takes
    that path for n = 4096 over 16 or more columns: it reports a non-zero workspace then).

    The contiguous tensor is viewed as (outer, n, stride); every column is transformed along
    its n elements (replaces trnfft/api.py:496-516's transposes).
    """
    shape = re.shape
    n = shape[dim]
    dev = target_device(re, im)
    out_dev = re.device
    re = to_device_f32(re, dev)
    im = to_device_f32(im, dev)
    outer = 1
    for s_ in shape[:dim]:
        outer *= s_
    stride = 1
    for s_ in shape[dim + 1 :]:
        stride *= s_
    kind = _lib.KIND_C2C if (n & (n - 1)) == 0 else _lib.KIND_BLUESTEIN
    plan = native_plan(kind, n, inverse, dev.index)
    out_re = torch.empty_like(re)
    out_im = torch.empty_like(re)
    lib = _lib.lib()
    with torch.cuda.device(dev):
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.tfa_strided_workspace_size(plan.handle, outer, stride, ctypes.byref(nbytes)),
                   "tfa_strided_workspace_size")
        if nbytes.value:
            ws = torch.empty(nbytes.value // 4, dtype=torch.float32, device=dev)
            rc = lib.tfa_execute_strided_ws(plan.handle, outer, stride, ptr(re), ptr(im), ptr(out_re), ptr(out_im),
                                            ptr(ws), stream_handle(dev))
            _lib.check(rc, "tfa_execute_strided_ws")
        else:
            rc = lib.tfa_execute_strided(plan.handle, outer, stride, ptr(re), ptr(im), ptr(out_re), ptr(out_im),
                                         stream_handle(dev))
            _lib.check(rc, "tfa_execute_strided")
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)


def fft2_small_ok(h: int, w: int) -> bool:
    """Images the single-pass 2-D kernel holds in LDS (mirror of tfa::fft2_small_ok): powers of
    two, h*w <= 16384, both axes >= 4 and >= the kernel's elements per thread."""
    def p2(v):
        return v > 0 and (v & (v - 1)) == 0

    if not (p2(h) and p2(w) and h >= 4 and w >= 4 and h * w <= 16384):
        return False
    img = 1 if h * w >= 4096 else 4096 // (h * w)
    e = img * h * w // 1024
    return h >= e and w >= e


def fft2_ok(h: int, w: int, real_in: bool = True) -> bool:
    """Shapes routed to the 2-D kernels: the single-pass small-image kernel, or the two-pass
    kernels (power-of-two 16 <= w <= 4096, 16 <= h <= 4096).  Complex input takes the two-pass
    kernels only for 256 <= w <= 512 with h >= 512: elsewhere the strided-axis pass plus the
    contiguous row pass measured faster (16 x 1024^2 155 -> 117 us, 4 x 2048^2 150 -> 140,
    against 64 x 512^2 123 vs 145 and 16 x 4096 x 256 146 vs 176 in favour of the two passes);
    real input takes them wherever they apply (32 x 2048^2 648 vs 898 us, 1 x 4096^2 115 vs 168)."""
    def p2(v):
        return v > 0 and (v & (v - 1)) == 0

    if fft2_small_ok(h, w):
        return True
    if not (p2(h) and p2(w) and 16 <= w <= 4096 and 16 <= h <= 4096):
        return False
    return real_in or (256 <= w <= 512 and h >= 512)


def execute_fft2(re: torch.Tensor, im: torch.Tensor | None, inverse: bool) -> ComplexTensor:
    """2-D transform over the last two axes (two HBM passes; replaces trnfft/api.py:105-139)."""
    h, w = re.shape[-2], re.shape[-1]
    dev = target_device(re, im)
    out_dev = re.device
    re = to_device_f32(re, dev)
    im = to_device_f32(im, dev)
    batch = re.numel() // (h * w) if re.numel() else 0
    plan = native_plan(_lib.KIND_FFT2, w, inverse, dev.index, n2=h)
    out_re = torch.empty(re.shape, dtype=torch.float32, device=dev)
    out_im = torch.empty_like(out_re)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_execute(
            plan.handle, batch, ptr(re), ptr(im), ptr(out_re), ptr(out_im), ptr(None), stream_handle(dev)
        )
    _lib.check(rc, "tfa_execute(fft2)")
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)


def execute_fft2_any(re: torch.Tensor, im: torch.Tensor | None, inverse: bool) -> ComplexTensor:
    """2-D transform over the last two axes by whichever route measured faster for this input
    (``fft2_ok``): the 2-D kernels, or the strided pass over axis -2 then the contiguous pass
    over axis -1 (used for the adjoint of a real-input fft2, whose gradient is complex)."""
    h, w = re.shape[-2], re.shape[-1]
    if fft2_ok(h, w, im is None):
        return execute_fft2(re, im, inverse)
    y = execute_strided(re, im, re.dim() - 2, inverse)
    return execute_1d(y.real, y.imag, inverse)


def execute_istft(re: torch.Tensor, im: torch.Tensor, win: torch.Tensor, n_fft: int, hop: int, center: bool,
                  normalized: bool, onesided: bool, length: int | None) -> torch.Tensor:
    """Fused inverse-STFT kernel on device fp32 spectra (..., bins, frames) in either memory order
    and the effective window (n_fft): the (..., out_len) signal (replaces trnfft/api.py:368-470
    after its argument handling).  Raises NotImplementedError where the plan refuses the shape
    (a hop too short for the kernel's frame tile, two-sided spectra at other n_fft)."""
    flags = ((_lib.STFT_ONESIDED if onesided else 0) | (_lib.STFT_CENTER if center else 0)
             | (_lib.STFT_NORMALIZED if normalized else 0))
    dev = re.device
    frames = re.shape[-1]
    lead = re.shape[:-2]
    batch = re.numel() // (re.shape[-2] * frames)
    re, im, fm = stft_planes(re.reshape(batch, re.shape[-2], frames), im.reshape(batch, im.shape[-2], frames))
    if fm:
        flags |= _lib.STFT_FRAMES_MAJOR
    plan = native_plan(_lib.KIND_STFT, n_fft, True, dev.index, hop=hop, flags=flags)
    win = win.contiguous()
    out_len = ctypes.c_int64()
    lib = _lib.lib()
    req = -1 if length is None else int(length)
    _lib.check(lib.tfa_istft_length(plan.handle, frames, req, ctypes.byref(out_len)), "tfa_istft_length")
    out = torch.empty(*lead, out_len.value, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.tfa_istft_execute(plan.handle, batch, frames, ptr(re), ptr(im), ptr(win), ptr(out), req,
                                   stream_handle(dev))
    _lib.check(rc, "tfa_istft_execute")
    return out


def stft_planes(re: torch.Tensor, im: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, bool]:
    """(..., bins, frames) spectrum planes as contiguous buffers for the STFT kernels, without a
    copy where possible: the planes themselves when both are contiguous (the reference's layout,
    trnfft/complex.py:29-33), (..., frames, bins) buffers (frames_major True) when both planes are
    transposed views of such tensors (torch.stft's memory order, and ``stft(...,
    frames_major=True)``), else contiguous copies."""
    if re.is_contiguous() and im.is_contiguous():
        return re, im, False
    rt, it = re.transpose(-2, -1), im.transpose(-2, -1)
    if rt.is_contiguous() and it.is_contiguous():
        return rt, it, True
    return re.contiguous(), im.contiguous(), False


def execute_stft(x: torch.Tensor, win: torch.Tensor, n_fft: int, hop: int, center: bool, normalized: bool,
                 onesided: bool, num_frames: int, frames_major: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused STFT kernel on device-resident fp32 x (..., L) and window (n_fft): (re, im) planes of
    shape (..., bins, frames) (replaces trnfft/api.py:291-365 after its argument handling).  By
    default the planes are contiguous, the reference's layout (its ComplexTensor makes the
    transposed planes contiguous, trnfft/complex.py:29-33); with ``frames_major`` they are
    transposed views of (..., frames, bins) buffers (torch.stft's memory order), which the kernel
    writes as one contiguous run per tile."""
    flags = (_lib.STFT_CENTER if center else 0) | (_lib.STFT_NORMALIZED if normalized else 0)
    flags |= (_lib.STFT_ONESIDED if onesided else 0) | (_lib.STFT_FRAMES_MAJOR if frames_major else 0)
    dev = x.device
    x = x.contiguous()
    win = win.contiguous()
    plan = native_plan(_lib.KIND_STFT, n_fft, False, dev.index, hop=hop, flags=flags)
    bins = n_fft // 2 + 1 if onesided else n_fft
    lead = x.shape[:-1]
    batch = 1
    for d in lead:
        batch *= d
    shape = (*lead, num_frames, bins) if frames_major else (*lead, bins, num_frames)
    out_re = torch.empty(*shape, dtype=torch.float32, device=dev)
    out_im = torch.empty_like(out_re)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_stft_execute(
            plan.handle, batch, x.shape[-1], ptr(x), ptr(win), ptr(out_re), ptr(out_im), stream_handle(dev)
        )
    _lib.check(rc, "tfa_stft_execute")
    if frames_major:
        return out_re.transpose(-2, -1), out_im.transpose(-2, -1)
    return out_re, out_im


def execute_stft_backward(g_re: torch.Tensor, g_im: torch.Tensor, win: torch.Tensor, n_fft: int, hop: int,
                          center: bool, normalized: bool, padded_len: int) -> torch.Tensor | None:
    """Gradient of the onesided fused STFT with respect to its padded signal, (b, padded_len),
    from the output gradient planes (b, bins, frames): one fused kernel on the forward plan (per
    frame the adjoint of the transform -- the r2c adjoint, or the adjoint Bluestein chain for
    n_fft that is not a power of two -- window, overlap-add; replaces the autograd of
    trnfft/api.py:310-349's frame gather, window and per-frame transform).  None when the kernel's
    frame tile refuses the hop (the caller composes).  The gradient planes may be in either
    layout (stft_planes)."""
    g_re, g_im, fm = stft_planes(g_re, g_im)
    flags = _lib.STFT_ONESIDED | (_lib.STFT_CENTER if center else 0) | (_lib.STFT_NORMALIZED if normalized else 0)
    flags |= _lib.STFT_FRAMES_MAJOR if fm else 0
    dev = g_re.device
    plan = native_plan(_lib.KIND_STFT, n_fft, False, dev.index, hop=hop, flags=flags)
    win = win.contiguous()
    b, frames = g_re.shape[0], (g_re.shape[-2] if fm else g_re.shape[-1])
    out = torch.empty(b, padded_len, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_stft_backward_execute(plan.handle, b, frames, ptr(g_re), ptr(g_im), ptr(win), ptr(out),
                                                  padded_len, stream_handle(dev))
    if rc == _lib.TFA_ERR_UNSUPPORTED:
        return None
    _lib.check(rc, "tfa_stft_backward_execute")
    return out


def strided_ok(n: int, stride: int) -> bool:
    if stride < 1 or n < 2:
        return False
    if (n & (n - 1)) == 0:
        return n <= _STRIDED_MAX_N or (n <= _STRIDED_FS_MAX_N and stride >= _strided_fs_min_stride(n))
    return n <= _STRIDED_BLUE_MAX_N


def _fft_via_gemm(x: ComplexTensor, inverse: bool) -> ComplexTensor:
    """X = x @ W with the exact DFT matrix, on the matrix-core DFT-GEMM kernel (n <= 256)."""
    re, im = x.real, x.imag
    n = re.shape[-1]
    dev = target_device(re, im)
    out_dev = re.device
    re = to_device_f32(re, dev)
    im = to_device_f32(im, dev)
    batch = re.numel() // n
    plan = native_plan(_lib.KIND_DFT_GEMM, n, inverse, dev.index)
    out_re = torch.empty_like(re)
    out_im = torch.empty_like(re)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_execute(
            plan.handle, batch, ptr(re), ptr(im), ptr(out_re), ptr(out_im), ptr(None), stream_handle(dev)
        )
    _lib.check(rc, "tfa_execute(dft_gemm)")
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)
