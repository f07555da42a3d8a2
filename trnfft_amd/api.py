"""Public torch.fft-style API on the HIP backend (surface of trnfft/api.py:22-538).

Every transform runs on the library's HIP kernels.  Tensors on the CPU are moved to the current
GPU and the result is returned on the input's device.  All helpers allocate on the input's
device (the reference's helpers allocate on the CPU, trnfft/api.py:55-56,487-488,536).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .complex import ComplexTensor
from .dispatch import _require_hip, target_device, to_device_f32
from . import autograd as _ag
from . import fft_core as _fc
from .fft_core import fft2_ok, fft_core, real_ok, strided_ok
from .plan import native_plan
from .precision import _resolve


def _is_real_tensor(x) -> bool:
    return isinstance(x, torch.Tensor) and not torch.is_complex(x)


def fft(input: torch.Tensor | ComplexTensor, n: int | None = None) -> ComplexTensor:
    """1-D discrete Fourier transform along the last dimension (trnfft/api.py:22-27)."""
    if _is_real_tensor(input):
        x = input if n is None else _resize_real(input, n)
        return _real_1d(x, inverse=False)
    x = _to_complex(input)
    if n is not None:
        x = _resize_last(x, n)
    return fft_core(x, inverse=False)


def ifft(input: torch.Tensor | ComplexTensor, n: int | None = None) -> ComplexTensor:
    """1-D inverse discrete Fourier transform, scaled 1/n (trnfft/api.py:30-35)."""
    if _is_real_tensor(input):
        x = input if n is None else _resize_real(input, n)
        return _real_1d(x, inverse=True)
    x = _to_complex(input)
    if n is not None:
        x = _resize_last(x, n)
    return fft_core(x, inverse=True)


def _real_1d(x: torch.Tensor, inverse: bool) -> ComplexTensor:
    # real input: the kernels read only the real plane (imaginary part zero, no zeros tensor)
    _resolve(None)
    if x.shape[-1] == 1:
        return ComplexTensor(x.clone())
    _require_hip("fft")
    return _ag.c2c(x, None, inverse)


def rfft(input: torch.Tensor, n: int | None = None) -> ComplexTensor:
    """FFT of a real signal, bins 0..n//2 (trnfft/api.py:38-46)."""
    if n is not None:
        input = _resize_real(input, n)
    n = input.shape[-1]
    if real_ok(n):
        _resolve(None)
        _require_hip("rfft")
        return _ag.r2c(input)
    result = _real_1d(input, inverse=False)
    half = n // 2 + 1
    return ComplexTensor(result.real[..., :half], result.imag[..., :half])


def irfft(input: ComplexTensor, n: int | None = None) -> torch.Tensor:
    """Inverse of rfft via the Hermitian-completed spectrum (trnfft/api.py:49-68)."""
    if n is None:
        n = 2 * (input.shape[-1] - 1)
    if n == 2 * (input.shape[-1] - 1) and real_ok(n):
        _resolve(None)
        _require_hip("irfft")
        return _ag.c2r(input.real, input.imag, n)
    dev = input.real.device
    full_re = torch.zeros(*input.shape[:-1], n, dtype=input.dtype, device=dev)
    full_im = torch.zeros(*input.shape[:-1], n, dtype=input.dtype, device=dev)
    half = input.shape[-1]
    full_re[..., :half] = input.real[..., :n]
    full_im[..., :half] = input.imag[..., :n]
    if n > 1:
        num_neg = n - half
        full_re[..., half:] = torch.flip(input.real[..., 1 : 1 + num_neg], dims=[-1])
        full_im[..., half:] = -torch.flip(input.imag[..., 1 : 1 + num_neg], dims=[-1])
    result = fft_core(ComplexTensor._wrap(full_re, full_im), inverse=True)
    return result.real


def hfft(input: ComplexTensor, n: int | None = None) -> torch.Tensor:
    """FFT of a Hermitian signal given one-sided (trnfft/api.py:71-86): irfft(conj(x), n) * n."""
    if n is None:
        n = 2 * (input.shape[-1] - 1)
    conj_input = ComplexTensor(input.real, -input.imag)
    return irfft(conj_input, n=n) * n


def ihfft(input: torch.Tensor, n: int | None = None) -> ComplexTensor:
    """One-sided inverse of a real signal (trnfft/api.py:89-102): conj(rfft(x, n)) / n."""
    n_actual = input.shape[-1] if n is None else n
    result = rfft(input, n=n_actual)
    return ComplexTensor(result.real / n_actual, -result.imag / n_actual)


def fft2(input: torch.Tensor | ComplexTensor, s: tuple[int, int] | None = None) -> ComplexTensor:
    """2-D FFT over the last two dimensions (trnfft/api.py:105-108)."""
    s_arg = None if s is None else tuple(s)
    return fftn(input, s=s_arg, dim=(-2, -1))


def _norm_dims(ndim: int, s, dim):
    if dim is None:
        dim = tuple(range(-len(s), 0)) if s is not None else tuple(range(-ndim, 0))
    return tuple(d % ndim for d in dim)


def fftn(
    input: torch.Tensor | ComplexTensor,
    s: tuple[int, ...] | None = None,
    dim: tuple[int, ...] | None = None,
) -> ComplexTensor:
    """N-D FFT along `dim` (default all), one axis at a time in the given order (trnfft/api.py:111-139)."""
    return _fftn(input, s, dim, inverse=False)


def ifftn(
    input: torch.Tensor | ComplexTensor,
    s: tuple[int, ...] | None = None,
    dim: tuple[int, ...] | None = None,
) -> ComplexTensor:
    """N-D inverse FFT (trnfft/api.py:142-167)."""
    return _fftn(input, s, dim, inverse=True)


def _fftn(input, s, dim, inverse: bool) -> ComplexTensor:
    ndim = input.dim() if isinstance(input, torch.Tensor) else len(input.shape)
    dim = _norm_dims(ndim, s, dim)
    if s is not None:
        assert len(s) == len(dim), f"len(s)={len(s)} must match len(dim)={len(dim)}"
    real_in = _is_real_tensor(input)
    x = input if real_in else _to_complex(input)
    if s is not None:
        for size, d in zip(s, dim):
            x = _resize_dim_real(x, d, size) if real_in else _resize_dim(x, d, size)
    if ndim >= 2 and sorted(dim) == [ndim - 2, ndim - 1] and fft2_ok(x.shape[-2], x.shape[-1], real_in):
        # both trailing axes at once: the 2-D kernels where they measured faster than the two
        # single-axis passes (the 1-D transforms of the two axes commute; only rounding differs
        # from the reference's dim -2 then dim -1 order)
        _resolve(None)
        _require_hip("fft2")
        if real_in:
            return _ag.fft2(x, None, inverse)
        return _ag.fft2(x.real, x.imag, inverse)
    order = list(dim)
    if real_in and (ndim - 1) in order:
        # real input: transform the contiguous last axis first (it reads only the real plane);
        # the axes' 1-D transforms commute, so only rounding differs from the given order
        order.remove(ndim - 1)
        order.insert(0, ndim - 1)
    for d in order:
        x = _fft_along_dim(x, d, inverse=inverse)
    return x


def rfft2(input: torch.Tensor, s: tuple[int, int] | None = None) -> ComplexTensor:
    """2-D FFT of a real signal, Hermitian-halved on the last dim (trnfft/api.py:170-179)."""
    return rfftn(input, s=tuple(s) if s is not None else None, dim=(-2, -1))


def rfftn(
    input: torch.Tensor,
    s: tuple[int, ...] | None = None,
    dim: tuple[int, ...] | None = None,
) -> ComplexTensor:
    """N-D FFT of a real signal (trnfft/api.py:182-225): rfft on the last axis of `dim`, then c2c."""
    assert not torch.is_complex(input), "rfftn requires real input"
    ndim = input.dim()
    dim = _norm_dims(ndim, s, dim)
    last_dim, other_dims = dim[-1], dim[:-1]
    n_last = s[-1] if s is not None else None
    if last_dim == ndim - 1:
        x = rfft(input, n=n_last)
    else:
        x = rfft(input.transpose(last_dim, -1).contiguous(), n=n_last).transpose(last_dim, -1)
    if s is not None:
        for size, d in zip(s[:-1], other_dims):
            x = _resize_dim(x, d, size)
    for d in other_dims:
        x = _fft_along_dim(x, d, inverse=False)
    return x


def irfft2(input: ComplexTensor, s: tuple[int, int] | None = None) -> torch.Tensor:
    """Inverse of rfft2 (trnfft/api.py:228-239)."""
    return irfftn(input, s=tuple(s) if s is not None else None, dim=(-2, -1))


def irfftn(
    input: ComplexTensor,
    s: tuple[int, ...] | None = None,
    dim: tuple[int, ...] | None = None,
) -> torch.Tensor:
    """Inverse of rfftn (trnfft/api.py:242-288): c2c inverse on the other axes, then irfft."""
    ndim = input.real.dim()
    dim = _norm_dims(ndim, s, dim)
    last_dim, other_dims = dim[-1], dim[:-1]
    x = input
    if s is not None:
        for size, d in zip(s[:-1], other_dims):
            x = _resize_dim(x, d, size)
        n_last = s[-1]
    else:
        n_last = 2 * (x.shape[last_dim] - 1)
    for d in other_dims:
        x = _fft_along_dim(x, d, inverse=True)
    if last_dim == ndim - 1:
        return irfft(x, n=n_last)
    x_t = ComplexTensor(
        x.real.transpose(last_dim, -1).contiguous(),
        x.imag.transpose(last_dim, -1).contiguous(),
    )
    return irfft(x_t, n=n_last).transpose(last_dim, -1).contiguous()


def stft_num_frames(length: int, n_fft: int, hop_length: int, center: bool = True) -> int:
    padded = length + 2 * (n_fft // 2) if center else length
    return 1 + (padded - n_fft) // hop_length


_default_windows: dict[tuple, torch.Tensor] = {}


def _effective_window(window: torch.Tensor | None, n_fft: int, win_length: int, dtype, device=None) -> torch.Tensor:
    if window is None:
        # default periodic Hann (torch.hann_window, as the reference), built once per device so
        # later calls (including ones under HIP-graph capture) make no host-to-device copy
        key = (win_length, n_fft, dtype, str(device))
        cached = _default_windows.get(key)
        if cached is not None:
            return cached
        w = _effective_window(torch.hann_window(win_length, dtype=dtype), n_fft, win_length, dtype)
        w = w.to(device) if device is not None else w
        _default_windows[key] = w
        return w
    if win_length < n_fft:
        padded = torch.zeros(n_fft, dtype=window.dtype, device=window.device)
        offset = (n_fft - win_length) // 2
        padded[offset : offset + win_length] = window
        window = padded
    return window


# longest non-power-of-two n_fft of the fused per-frame Bluestein STFT (4096-point convolution:
# n + n/2 <= 4096 onesided, 2n - 1 <= 4096 two-sided)
_STFT_BLUE_MAX_N = {True: 2731, False: 2048}


def _fused_stft_ok(n_fft: int, onesided: bool = True) -> bool:
    """Whether the fused STFT kernel takes this n_fft: a power of two in [16, 4096] (two real
    frames per transform), or any other n_fft from 9 up to 2731 (onesided) or 2048 (two-sided)
    (one Bluestein transform per frame).  Both are differentiable: the signal gradient is one
    fused adjoint kernel where its tile allows, the composed adjoint otherwise."""
    if n_fft & (n_fft - 1) == 0:
        return 16 <= n_fft <= 4096
    return 9 <= n_fft <= _STFT_BLUE_MAX_N[bool(onesided)]


def stft(
    input: torch.Tensor,
    n_fft: int,
    hop_length: int | None = None,
    win_length: int | None = None,
    window: torch.Tensor | None = None,
    center: bool = True,
    pad_mode: str = "reflect",
    normalized: bool = False,
    onesided: bool = True,
    *,
    frames_major: bool = False,
) -> ComplexTensor:
    """Short-time Fourier transform, output (..., freq, time) (trnfft/api.py:291-365).

    The result planes are contiguous (..., freq, time) tensors, as the reference returns them (its
    ComplexTensor makes the transposed planes contiguous, trnfft/complex.py:29-33).
    ``frames_major=True`` (not in the reference) returns transposed views of (..., time, freq)
    buffers instead -- torch.stft's memory order, which the fused kernel writes as one contiguous
    run per frame tile -- for callers that accept strided planes; ``istft`` reads either.

    Power-of-two n_fft in [16, 4096], and other n_fft from 9 to 2731 (2048 two-sided), run as
    one fused kernel that reads the raw waveform (framing, padding, window, transform -- one
    Bluestein chain per frame for non-power-of-two n_fft -- and the (freq, time) transpose in one
    pass); with a pad_mode other than "reflect" the signal is padded on the device first (the
    reference's F.pad) and the fused kernel frames the padded signal.  Other n_fft keep the
    reference's composition on the device: pad, frame gather, window, then the transform kernels
    (Bluestein for non-power-of-two n_fft) and the onesided slice.
    """
    if hop_length is None:
        hop_length = n_fft // 4
    if win_length is None:
        win_length = n_fft
    _resolve(None)
    _require_hip("stft")
    dev = target_device(input)
    win = _effective_window(window, n_fft, win_length, input.dtype, dev)
    out_dev = input.device
    x = to_device_f32(input, dev)
    win = to_device_f32(win, dev)
    fused = _fused_stft_ok(n_fft, onesided)
    if center and pad_mode == "reflect" and fused:
        length = x.shape[-1]
        if length <= n_fft // 2:
            raise ValueError(f"reflect padding of {n_fft // 2} needs more than {n_fft // 2} samples; got {length}")
        num_frames = stft_num_frames(length, n_fft, hop_length, center)
        out = _ag.stft(x, win, n_fft, hop_length, True, normalized, onesided, num_frames, frames_major)
        out_re, out_im = out.real, out.imag
        if x.dim() == 2 and x.shape[0] == 1:
            # the reference squeezes a (1, L) signal to 1-D after padding (trnfft/api.py:313-315),
            # so its result has no batch axis; keep that shape for drop-in compatibility
            out_re, out_im = out_re[0], out_im[0]
        out = ComplexTensor._wrap(out_re, out_im)
        return out if out_dev == dev else out.to(out_dev)
    if center:
        # trnfft/api.py:310-315, on the device: F.pad needs a 2-D+ input; (1, L') is squeezed back
        pad_amount = n_fft // 2
        x = x.unsqueeze(0) if x.dim() == 1 else x
        x = torch.nn.functional.pad(x, (pad_amount, pad_amount), mode=pad_mode)
        x = x.squeeze(0) if x.dim() == 2 and x.shape[0] == 1 else x
    padded_length = x.shape[-1]
    num_frames = 1 + (padded_length - n_fft) // hop_length
    if num_frames < 0:
        raise ValueError(f"signal of {padded_length} samples (after padding) is shorter than n_fft={n_fft}")
    bins = n_fft // 2 + 1 if onesided else n_fft
    if num_frames == 0:
        empty = torch.empty(*x.shape[:-1], bins, 0, dtype=torch.float32, device=dev)
        out = ComplexTensor._wrap(empty, empty.clone())
        return out if out_dev == dev else out.to(out_dev)
    if fused:
        # the padded signal through the fused kernel (no centre padding of its own)
        out = _ag.stft(x.contiguous(), win, n_fft, hop_length, False, normalized, onesided, num_frames,
                       frames_major)
        return out if out_dev == dev else out.to(out_dev)
    # trnfft/api.py:321-363 on the device: frame gather, window, transform of real frames,
    # onesided slice, (freq, time) transpose, normalisation
    # (the frame gather as a strided view: the same elements as the reference's index tensor,
    # and a cheap adjoint under autograd)
    frames = (x.unfold(-1, n_fft, hop_length)[..., :num_frames, :] * win).contiguous()  # (..., T, n_fft)
    spec = rfft(frames) if onesided else _real_1d(frames, inverse=False)
    # (..., T, bins) -> (..., bins, T): the reference's transpose, made contiguous by its
    # ComplexTensor (views of the (..., T, bins) buffers with frames_major)
    out_re, out_im = spec.real.transpose(-2, -1), spec.imag.transpose(-2, -1)
    if normalized:
        scale = 1.0 / math.sqrt(n_fft)
        out_re, out_im = out_re * scale, out_im * scale
    if not frames_major:
        out_re, out_im = out_re.contiguous(), out_im.contiguous()
    out = ComplexTensor._wrap(out_re, out_im)
    return out if out_dev == dev else out.to(out_dev)


def istft(
    input: ComplexTensor,
    n_fft: int,
    hop_length: int | None = None,
    win_length: int | None = None,
    window: torch.Tensor | None = None,
    center: bool = True,
    normalized: bool = False,
    onesided: bool = True,
    length: int | None = None,
) -> torch.Tensor:
    """Inverse STFT by overlap-add with window-sum normalisation (trnfft/api.py:368-470).

    One fused kernel (completion, inverse transform -- two frames per transform for power-of-two
    n_fft in [16, 4096], onesided or two-sided spectra; one inverse Bluestein chain per frame for
    other n_fft in [9, 2048], onesided -- window, overlap-add, envelope division, trim), whose
    spectra gradient at power-of-two n_fft is the fused forward STFT of the envelope-divided
    gradient; for window gradients, gradients at other n_fft, two-sided spectra at other n_fft or
    hops too short for the kernel's frame tile, the same steps run as a composition of the
    differentiable kernels.
    """
    if hop_length is None:
        hop_length = n_fft // 4
    if win_length is None:
        win_length = n_fft
    fused = _istft_fused(input, n_fft, hop_length, win_length, window, center, normalized, onesided, length)
    if fused is not None:
        return fused
    dev = input.real.device
    win = _effective_window(
        window.to(dev) if window is not None else None, n_fft, win_length, input.dtype
    ).to(dev)
    spec_re = input.real.transpose(-2, -1)
    spec_im = input.imag.transpose(-2, -1)
    if normalized:
        scale = math.sqrt(n_fft)
        spec_re, spec_im = spec_re * scale, spec_im * scale
    if onesided:
        bins = spec_re.shape[-1]
        full_re = torch.zeros(*spec_re.shape[:-1], n_fft, dtype=spec_re.dtype, device=dev)
        full_im = torch.zeros_like(full_re)
        full_re[..., :bins] = spec_re
        full_im[..., :bins] = spec_im
        if n_fft > 1:
            num_neg = n_fft - bins
            full_re[..., bins:] = torch.flip(spec_re[..., 1 : 1 + num_neg], dims=[-1])
            full_im[..., bins:] = -torch.flip(spec_im[..., 1 : 1 + num_neg], dims=[-1])
        spec_re, spec_im = full_re, full_im
    num_frames = spec_re.shape[-2]
    frames = fft_core(ComplexTensor(spec_re, spec_im), inverse=True).real  # (..., T, n_fft)
    expected_len = n_fft + (num_frames - 1) * hop_length
    batch_shape = frames.shape[:-2]
    flat = frames.reshape(-1, num_frames, n_fft)
    pos = (torch.arange(num_frames, device=dev).unsqueeze(1) * hop_length + torch.arange(n_fft, device=dev)).reshape(-1)
    output = torch.zeros(flat.shape[0], expected_len, dtype=frames.dtype, device=dev)
    raw = torch.zeros_like(output)
    output.index_add_(1, pos, (flat * win).reshape(flat.shape[0], -1))
    raw.index_add_(1, pos, flat.reshape(flat.shape[0], -1))
    window_sum = torch.zeros(expected_len, dtype=frames.dtype, device=dev)
    window_sum.index_add_(0, pos, (win**2).repeat(num_frames))
    mask = window_sum > 1e-8
    output = torch.where(mask, output / torch.where(mask, window_sum, torch.ones_like(window_sum)), raw)
    output = output.reshape(*batch_shape, expected_len)
    if center:
        pad_amount = n_fft // 2
        output = output[..., pad_amount:]
        if output.shape[-1] > pad_amount:
            output = output[..., :-pad_amount] if length is None else output
    if length is not None:
        cur = output.shape[-1]
        if cur > length:
            output = output[..., :length]
        elif cur < length:
            pad = torch.zeros(*batch_shape, length - cur, dtype=output.dtype, device=dev)
            output = torch.cat([output, pad], dim=-1)
    return output.contiguous()


def _istft_fused(spec, n_fft, hop, win_length, window, center, normalized, onesided, length):
    """The fused inverse-STFT kernel (differentiable in the spectra at power-of-two n_fft), or None
    when its preconditions do not hold."""
    from .dispatch import to_device_f32_strided

    re, im = spec.real, spec.imag
    # power-of-two n_fft in [16, 4096] (two frames per inverse transform; onesided or two-sided
    # spectra), other n_fft in [9, 2048] (one inverse Bluestein chain per frame, onesided)
    pow2 = n_fft & (n_fft - 1) == 0
    bins = n_fft // 2 + 1 if onesided else n_fft
    if ((not onesided and not pow2) or (pow2 and not 16 <= n_fft <= 4096) or (not pow2 and not 9 <= n_fft <= 2048)
            or re.dim() < 2 or re.shape[-2] != bins or re.shape[-1] < 1):
        return None
    # a window that needs a gradient, and gradients through the Bluestein chains, take the composition
    if _ag._grad_on(window) or (_ag._grad_on(re, im) and not pow2):
        return None
    _resolve(None)
    _require_hip("istft")
    dev = target_device(re, im)
    out_dev = re.device
    # either memory order of the (..., bins, frames) planes is taken without a copy
    re = to_device_f32_strided(re, dev)
    im = to_device_f32_strided(im, dev)
    win = _effective_window(window.to(dev) if window is not None else None, n_fft, win_length, torch.float32, dev)
    win = to_device_f32(win, dev)
    try:
        out = _ag.istft(re, im, win, n_fft, hop, center, normalized, onesided, length,
                        win_length if window is None else None)
    except NotImplementedError:
        return None  # hop too small for the kernel's frame tile
    return out if out_dev == dev else out.to(out_dev)


# --- Helpers ---------------------------------------------------------------------------------


def _to_complex(x) -> ComplexTensor:
    if isinstance(x, ComplexTensor):
        return x
    return ComplexTensor(x)


def _resize_last(x: ComplexTensor, n: int) -> ComplexTensor:
    current = x.shape[-1]
    if current == n:
        return x
    if current < n:
        pad = torch.zeros(*x.shape[:-1], n - current, dtype=x.dtype, device=x.device)
        return ComplexTensor(torch.cat([x.real, pad], dim=-1), torch.cat([x.imag, pad], dim=-1))
    return ComplexTensor(x.real[..., :n], x.imag[..., :n])


def _resize_real(x: torch.Tensor, n: int) -> torch.Tensor:
    current = x.shape[-1]
    if current == n:
        return x
    if current < n:
        pad = torch.zeros(*x.shape[:-1], n - current, dtype=x.dtype, device=x.device)
        return torch.cat([x, pad], dim=-1)
    return x[..., :n]


def _resize_dim(x: ComplexTensor, dim: int, n: int) -> ComplexTensor:
    ndim = len(x.shape)
    dim = dim % ndim
    if dim != ndim - 1:
        x = x.transpose(dim, -1)
    x = _resize_last(x, n)
    if dim != ndim - 1:
        x = x.transpose(dim, -1)
    return x


def _resize_dim_real(x: torch.Tensor, dim: int, n: int) -> torch.Tensor:
    return _resize_real(x.transpose(dim, -1), n).transpose(dim, -1).contiguous()


def _fft_along_dim(x, dim: int, inverse: bool) -> ComplexTensor:
    """1-D FFT along `dim` of a ComplexTensor or real tensor (trnfft/api.py:496-516).

    The last axis runs the contiguous kernels; another axis runs the strided kernels in place of
    the reference's transpose / FFT / transpose-back copies (power-of-two n <= 4096, other
    n <= 2048, and power-of-two n <= 2^24 over at least 4 or 8 trailing columns); the remaining
    shapes keep the transpose round trip.
    """
    real_in = _is_real_tensor(x)
    shape = tuple(x.shape)
    ndim = len(shape)
    dim = dim % ndim
    n = shape[dim]
    if dim == ndim - 1:
        if real_in:
            return _real_1d(x, inverse)
        return fft_core(x, inverse=inverse)
    stride = 1
    for s_ in shape[dim + 1 :]:
        stride *= s_
    if strided_ok(n, stride):
        _resolve(None)
        _require_hip("fftn")
        if real_in:
            return _ag.c2c_strided(x, None, dim, inverse)
        return _ag.c2c_strided(x.real, x.imag, dim, inverse)
    if real_in:
        moved = x.transpose(dim, -1).contiguous()
        res = _real_1d(moved, inverse)
    else:
        res = fft_core(x.transpose(dim, -1), inverse=inverse)
    return res.transpose(dim, -1)
