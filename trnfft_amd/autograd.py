"""Autograd for the HIP path (the role of trnfft/nki/autograd.py:1-205).

The reference's pytorch path is differentiable because it is made of torch ops; its NKI kernels
are wrapped in ``torch.autograd.Function`` classes whose backward emits the analytic adjoint
(trnfft/nki/autograd.py:125-155 complex linear, :92-112 complex GEMM, :167-205 FFT).  Here every
native launch that can sit on a training path is wrapped the same way, and the backward runs on
the same native kernels:

* c2c, any length, last axis / strided axis / both trailing axes (forward F, unnormalised):
      dx = n * F^-1(dy);   inverse (F^-1, scaled 1/n):  dx = F(dy) / n
  (trnfft/nki/autograd.py:190-203); for real input the gradient is the real part.
* r2c (rfft, bins 0..n/2):  dx_j = Re sum_k dy_k e^{+2 pi i j k / n} = n * c2r(dy'), where dy'
  halves bins 1..n/2-1 (c2r doubles them back and drops Im of bins 0 and n/2, whose real parts
  are the only ones that reach a real signal).
* c2r (irfft):  dX = r2c(dy) / n with bins 1..n/2-1 doubled (they appear twice in the
  Hermitian-completed spectrum); bins 0 and n/2 get no imaginary gradient.
* STFT: per-frame adjoint of the onesided (c2r as above) or two-sided (c2c) transform, times
  the window, overlap-added back onto the padded signal (torch fold), then the reflect-pad
  adjoint folds the padded edges back into the signal.  The window gradient, when asked for,
  is the frame-by-frame correlation of the padded signal with the unwindowed frame gradient.
* complex GEMM C = A B:            dA = dC B^H,  dB = A^H dC
  complex linear Y = X W^T + b:    dX = dY conj(W),  dW = dY^T conj(X),  db = sum over rows of dY
  each product one tfa_complex_gemm_ex launch (the reference runs eight real matmuls).

Second derivatives: every transform and product here is linear in each operand, so its adjoint
is again one of these operations.  Under ``create_graph=True`` (grad mode on inside backward) each
backward builds its adjoint from the differentiable wrappers of this module (c2c of the opposite
direction, c2r for r2c and r2c for c2r with the same bin weights, complex products of conjugated /
transposed operands, and torch ops for the STFT's framing, window and padding adjoints), so the
gradient can be differentiated again; an ordinary backward keeps the direct kernel calls.
"""

from __future__ import annotations

import collections
import functools
import math

import torch
import torch.nn.functional as F

from . import _lib
from . import fft_core as _fc
from .complex import ComplexTensor


def _grad_on(*ts) -> bool:
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in ts)


def _c(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous()


# ---------------------------------------------------------------------------------------------
# c2c: last axis, strided axis, both trailing axes
# ---------------------------------------------------------------------------------------------


class _C2CFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, re, im, inverse: bool, mode: str, dim: int):
        ctx.inverse, ctx.mode, ctx.dim, ctx.real_in = inverse, mode, dim, im is None
        if mode == "last":
            ctx.size = re.shape[-1]
            y = _fc.execute_1d(re, im, inverse)
        elif mode == "strided":
            ctx.size = re.shape[dim]
            y = _fc.execute_strided(re, im, dim, inverse)
        else:  # "fft2"
            ctx.size = re.shape[-1] * re.shape[-2]
            y = _fc.execute_fft2(re, im, inverse)
        return y.real, y.imag

    @staticmethod
    def backward(ctx, g_re, g_im):
        adj = not ctx.inverse
        if torch.is_grad_enabled():  # create_graph: the adjoint transform is recorded too
            s = 1.0 / ctx.size if ctx.inverse else float(ctx.size)
            if ctx.mode == "fft2":
                y = _fft2_any(g_re, g_im, adj)
            else:
                y = _c2c(g_re, g_im, adj, ctx.mode, ctx.dim)
            return y.real * s, None if ctx.real_in else y.imag * s, None, None, None
        g_re, g_im = _c(g_re), _c(g_im)
        if ctx.mode == "last":
            g = _fc.execute_1d(g_re, g_im, adj)
        elif ctx.mode == "strided":
            g = _fc.execute_strided(g_re, g_im, ctx.dim, adj)
        else:
            g = _fc.execute_fft2_any(g_re, g_im, adj)
        s = 1.0 / ctx.size if ctx.inverse else float(ctx.size)
        d_re = g.real.mul_(s)
        d_im = None if ctx.real_in else g.imag.mul_(s)
        return d_re, d_im, None, None, None


def _c2c(re, im, inverse, mode, dim=-1) -> ComplexTensor:
    if _grad_on(re, im):
        y_re, y_im = _C2CFn.apply(re, im, inverse, mode, dim)
        return ComplexTensor._wrap(y_re, y_im)
    if mode == "last":
        return _fc.execute_1d(re, im, inverse)
    if mode == "strided":
        return _fc.execute_strided(re, im, dim, inverse)
    return _fc.execute_fft2(re, im, inverse)


def _fft2_any(re, im, inverse) -> ComplexTensor:
    """Differentiable transform over the two trailing axes by the route execute_fft2_any takes."""
    if _fc.fft2_ok(re.shape[-2], re.shape[-1], im is None):
        return _c2c(re, im, inverse, "fft2")
    y = _c2c(re, im, inverse, "strided", re.dim() - 2)
    return _c2c(y.real, y.imag, inverse, "last")


def c2c(re: torch.Tensor, im: torch.Tensor | None, inverse: bool) -> ComplexTensor:
    """Last-axis transform (im None: real input), differentiable."""
    return _c2c(re, im, inverse, "last")


def c2c_strided(re: torch.Tensor, im: torch.Tensor | None, dim: int, inverse: bool) -> ComplexTensor:
    """Transform along axis `dim` in place of a transpose round trip, differentiable."""
    return _c2c(re, im, inverse, "strided", dim)


def fft2(re: torch.Tensor, im: torch.Tensor | None, inverse: bool) -> ComplexTensor:
    """Transform over the two trailing axes, differentiable."""
    return _c2c(re, im, inverse, "fft2")


# ---------------------------------------------------------------------------------------------
# real rows: r2c / c2r
# ---------------------------------------------------------------------------------------------


def _bin_weights(g: torch.Tensor, n: int, inner: float, edge: float) -> torch.Tensor:
    """(n/2 + 1) weights: `inner` for bins 1..n/2-1, `edge` for bins 0 and n/2."""
    w = torch.full((g.shape[-1],), inner, dtype=g.dtype, device=g.device)
    w[0] = edge
    w[n // 2] = edge
    return w


def _r2c_adjoint(g_re: torch.Tensor, g_im: torch.Tensor, n: int) -> torch.Tensor:
    h = n // 2
    g_re, g_im = g_re.clone(), g_im.clone()
    g_re[..., 1:h] *= 0.5
    g_im[..., 1:h] *= 0.5
    return _fc.execute_c2r(g_re, g_im, n).mul_(float(n))


def _c2r_adjoint(g: torch.Tensor, n: int):
    h = n // 2
    y = _fc.execute_r2c(_c(g))
    d_re, d_im = y.real.mul_(1.0 / n), y.imag.mul_(1.0 / n)
    d_re[..., 1:h] *= 2.0
    d_im[..., 1:h] *= 2.0
    d_im[..., 0] = 0.0
    d_im[..., h] = 0.0
    return d_re, d_im


class _R2CFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.n = x.shape[-1]
        y = _fc.execute_r2c(x)
        return y.real, y.imag

    @staticmethod
    def backward(ctx, g_re, g_im):
        if torch.is_grad_enabled():  # create_graph: the same adjoint through the differentiable c2r
            w = _bin_weights(g_re, ctx.n, 0.5, 1.0)
            return c2r(g_re * w, g_im * w, ctx.n) * float(ctx.n)
        return _r2c_adjoint(g_re, g_im, ctx.n)


class _C2RFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, re, im, n: int):
        ctx.n = n
        return _fc.execute_c2r(re, im, n)

    @staticmethod
    def backward(ctx, g):
        if torch.is_grad_enabled():  # create_graph: the same adjoint through the differentiable r2c
            y = r2c(g)
            return (y.real * _bin_weights(y.real, ctx.n, 2.0 / ctx.n, 1.0 / ctx.n),
                    y.imag * _bin_weights(y.imag, ctx.n, 2.0 / ctx.n, 0.0), None)
        d_re, d_im = _c2r_adjoint(g, ctx.n)
        return d_re, d_im, None


def r2c(x: torch.Tensor) -> ComplexTensor:
    if _grad_on(x):
        y_re, y_im = _R2CFn.apply(x)
        return ComplexTensor._wrap(y_re, y_im)
    return _fc.execute_r2c(x)


def c2r(re: torch.Tensor, im: torch.Tensor, n: int) -> torch.Tensor:
    if _grad_on(re, im):
        return _C2RFn.apply(re, im, n)
    return _fc.execute_c2r(re, im, n)


# ---------------------------------------------------------------------------------------------
# STFT
# ---------------------------------------------------------------------------------------------


class _StftFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, win, n_fft, hop, center, normalized, onesided, num_frames, frames_major):
        ctx.save_for_backward(x, win)
        ctx.cfg = (n_fft, hop, center, normalized, onesided, num_frames)
        return _fc.execute_stft(x, win, n_fft, hop, center, normalized, onesided, num_frames, frames_major)

    @staticmethod
    def backward(ctx, g_re, g_im):
        x, win = ctx.saved_tensors
        n_fft, hop, center, normalized, onesided, frames = ctx.cfg
        length = x.shape[-1]
        lead = x.shape[:-1]
        b = x.numel() // length
        bins = g_re.shape[-2]
        pad = n_fft // 2 if center else 0
        if torch.is_grad_enabled():  # create_graph: the composed adjoint, recorded
            return _stft_adjoint_recorded(ctx, x, win, g_re, g_im)
        if onesided and ctx.needs_input_grad[0] and not ctx.needs_input_grad[1] and g_re.is_cuda:
            # no window gradient: one fused kernel (per-frame transform adjoint, window, overlap-add)
            d_xp = _fc.execute_stft_backward(g_re.reshape(b, bins, frames), g_im.reshape(b, bins, frames), win,
                                             n_fft, hop, center, normalized, length + 2 * pad)
            if d_xp is not None:
                return (_unpad_reflect(d_xp, pad, length).reshape(*lead, length), None, None, None, None, None, None, None,
                        None)
        # (..., bins, frames) -> (b, frames, bins): one spectrum per row
        gr = g_re.reshape(b, bins, frames).transpose(1, 2).contiguous()
        gi = g_im.reshape(b, bins, frames).transpose(1, 2).contiguous()
        if onesided and n_fft & (n_fft - 1) == 0:
            fg = _r2c_adjoint(gr, gi, n_fft)  # (b, frames, n_fft)
        else:
            if bins < n_fft:
                # onesided, n_fft not a power of two: the adjoint of keeping bins < n_fft/2 + 1 of
                # the complex transform is zero-filling the rest before its adjoint
                gr = F.pad(gr, (0, n_fft - bins))
                gi = F.pad(gi, (0, n_fft - bins))
            fg = _fc.execute_1d(gr, gi, True).real.mul_(float(n_fft))
        if normalized:
            fg.mul_(1.0 / math.sqrt(n_fft))
        if center:
            xp = F.pad(x.reshape(b, 1, length), (pad, pad), mode="reflect").reshape(b, -1)
        else:
            xp = x.reshape(b, length)
        lp = xp.shape[-1]
        d_win = None
        if ctx.needs_input_grad[1]:
            fr = xp.unfold(-1, n_fft, hop)[:, :frames]  # (b, frames, n_fft)
            d_win = (fr * fg).sum(dim=(0, 1))
        d_x = None
        if ctx.needs_input_grad[0]:
            fg.mul_(win)
            d_xp = F.fold(fg.transpose(1, 2), output_size=(1, lp), kernel_size=(1, n_fft), stride=(1, hop))
            d_xp = d_xp.reshape(b, lp)
            d_x = _unpad_reflect(d_xp, pad, length).reshape(*lead, length)
        return d_x, d_win, None, None, None, None, None, None, None


def _stft_adjoint_recorded(ctx, x, win, g_re, g_im):
    """The STFT backward's composed adjoint (the same steps as the direct path) from differentiable
    operations only, so that the gradients it returns can be differentiated again."""
    n_fft, hop, center, normalized, onesided, frames = ctx.cfg
    length = x.shape[-1]
    lead = x.shape[:-1]
    b = x.numel() // length
    bins = g_re.shape[-2]
    pad = n_fft // 2 if center else 0
    gr = g_re.reshape(b, bins, frames).transpose(1, 2).contiguous()
    gi = g_im.reshape(b, bins, frames).transpose(1, 2).contiguous()
    if onesided and n_fft & (n_fft - 1) == 0:
        w = _bin_weights(gr, n_fft, 0.5, 1.0)
        fg = c2r(gr * w, gi * w, n_fft) * float(n_fft)
    else:
        if bins < n_fft:
            gr = F.pad(gr, (0, n_fft - bins))
            gi = F.pad(gi, (0, n_fft - bins))
        fg = c2c(gr, gi, True).real * float(n_fft)
    if normalized:
        fg = fg * (1.0 / math.sqrt(n_fft))
    if center:
        xp = F.pad(x.reshape(b, 1, length), (pad, pad), mode="reflect").reshape(b, -1)
    else:
        xp = x.reshape(b, length)
    lp = xp.shape[-1]
    d_win = d_x = None
    if ctx.needs_input_grad[1]:
        d_win = (xp.unfold(-1, n_fft, hop)[:, :frames] * fg).sum(dim=(0, 1))
    if ctx.needs_input_grad[0]:
        d_xp = F.fold((fg * win).transpose(1, 2), output_size=(1, lp), kernel_size=(1, n_fft), stride=(1, hop))
        d_xp = d_xp.reshape(b, lp)
        d_x = d_xp[:, pad : pad + length]
        if pad:  # the reflected edges folded back, out of place
            d_x = (d_x + F.pad(d_xp[:, :pad].flip(-1), (1, length - 1 - pad))
                   + F.pad(d_xp[:, pad + length :].flip(-1), (length - 1 - pad, 1)))
        d_x = d_x.reshape(*lead, length)
    return d_x, d_win, None, None, None, None, None, None, None


def _unpad_reflect(d_xp: torch.Tensor, pad: int, length: int) -> torch.Tensor:
    """Adjoint of the reflect padding x_pad[i] = x[pad - i] (i < pad), x_pad[pad + j] = x[j],
    x_pad[pad + L + i] = x[L - 2 - i]: the kept span, with the reflected edges folded back in
    place (a view of d_xp's rows; pad = 0 is the plain prefix)."""
    d_x = d_xp[:, pad : pad + length]
    if pad:
        d_x[:, 1 : pad + 1] += d_xp[:, :pad].flip(-1)
        d_x[:, length - 1 - pad : length - 1] += d_xp[:, pad + length :].flip(-1)
    return d_x


def stft(x, win, n_fft, hop, center, normalized, onesided, num_frames, frames_major=False) -> ComplexTensor:
    """Fused STFT kernel on device fp32 x (..., L), window (n_fft); differentiable in x and window.
    Contiguous (..., bins, frames) planes, or with ``frames_major`` transposed views of
    (..., frames, bins) buffers."""
    if _grad_on(x, win):
        y_re, y_im = _StftFn.apply(x, win, n_fft, hop, center, normalized, onesided, num_frames, frames_major)
    else:
        y_re, y_im = _fc.execute_stft(x, win, n_fft, hop, center, normalized, onesided, num_frames, frames_major)
    return ComplexTensor._wrap(y_re, y_im)


# ---------------------------------------------------------------------------------------------
# inverse STFT (power-of-two n_fft, fused kernel forward)
# ---------------------------------------------------------------------------------------------


@functools.lru_cache(maxsize=8)
def _default_window_envelope(n_fft: int, win_length: int, hop: int, frames: int) -> torch.Tensor:
    """Window-square envelope (fp32, host) of the default window (periodic Hann of win_length,
    centred in n_fft) over `frames` frames: it depends on the shape only, so the gradient of a
    call with the default window reads it (and its raw-sum test) without building it on the
    device or synchronising with it."""
    w = torch.zeros(n_fft, dtype=torch.float32)
    off = (n_fft - win_length) // 2
    w[off:off + win_length] = torch.hann_window(win_length, dtype=torch.float32)
    pos = (torch.arange(frames).unsqueeze(1) * hop + torch.arange(n_fft)).reshape(-1)
    return torch.zeros(n_fft + (frames - 1) * hop, dtype=torch.float32).index_add_(0, pos, (w * w).repeat(frames))


_default_inv_env: "collections.OrderedDict" = collections.OrderedDict()  # key -> device 1/env (0 where env <= 1e-8)
_DEFAULT_INV_ENV_KEEP = 8


def _default_window_inv_env(n_fft, win_length, hop, frames, dev):
    key = (n_fft, win_length, hop, frames, str(dev))
    inv = _default_inv_env.get(key)
    if inv is None:
        env = _default_window_envelope(n_fft, win_length, hop, frames)
        inv = torch.where(env > 1e-8, 1.0 / env.clamp_min(1e-30), torch.zeros_like(env)).to(dev)
        _default_inv_env[key] = inv
        while len(_default_inv_env) > _DEFAULT_INV_ENV_KEEP:
            _default_inv_env.popitem(last=False)
    else:
        _default_inv_env.move_to_end(key)
    return inv


def _pad_product(g2, scale, start, total, rec):
    """(rows, total) = zero-padded g2 * scale, g2 (rows, m) placed at column start: one product
    written into the padded buffer (only the pads are cleared); F.pad when recording a graph."""
    m = g2.shape[-1]
    if rec:
        return F.pad(g2 * scale, (start, total - start - m))
    out = torch.empty(g2.shape[0], total, dtype=g2.dtype, device=g2.device)
    out[:, :start].zero_()
    out[:, start + m:].zero_()
    torch.mul(g2, scale, out=out[:, start:start + m])
    return out


def _istft_adjoint(g, win, n_fft, hop, center, normalized, onesided, frames, length, default_win):
    """Gradient of the inverse STFT (trnfft/api.py:368-470) with respect to its spectra.  The
    forward keeps samples [start, start + m) of y[s] = sum_t f_t(s - t hop) w(s - t hop) / env[s]
    (the raw sum of the frames where env[s] <= 1e-8), f_t the real frames of the spectra X_t.  So
    the frame gradient is w[j] u1[t hop + j] + u2[t hop + j] with u1 = g / env (env > 1e-8) and
    u2 = g (elsewhere), g zero-padded back to the untrimmed length: a windowed frame gather and a
    forward transform, i.e. the STFT without centring, then the adjoint of the frames' completion
    -- onesided (c2r): r2c / n with bins 1..n/2-1 doubled and no imaginary gradient at 0 and n/2;
    two-sided (real part of the inverse c2c): the full forward transform / n -- and sqrt(n) when
    normalized.  The interior factor is folded into the transform's window, the edge bins fixed
    after it.  Built from the differentiable stft under grad mode (create_graph).
    default_win: (win_length) of the default window, whose raw-sum test runs on the host."""
    rec = torch.is_grad_enabled()
    dev = g.device
    lead = g.shape[:-1]
    out_len = g.shape[-1]
    expected = n_fft + (frames - 1) * hop
    start = n_fft // 2 if center else 0
    cur = expected - start
    if start and cur > start and length is None:
        cur -= start
    m = min(cur, out_len)
    if default_win is not None:
        inv = _default_window_inv_env(n_fft, default_win, hop, frames, dev)
        env_h = _default_window_envelope(n_fft, default_win, hop, frames)
        raw_kept = bool((env_h[start:start + m] <= 1e-8).any())
        mask = inv > 0 if raw_kept else None
    else:
        pos = (torch.arange(frames, device=dev).unsqueeze(1) * hop + torch.arange(n_fft, device=dev)).reshape(-1)
        env = torch.zeros(expected, dtype=torch.float32, device=dev).index_add(0, pos, (win**2).repeat(frames))
        mask = env > 1e-8
        inv = torch.where(mask, 1.0 / torch.where(mask, env, torch.ones_like(env)), torch.zeros_like(env))
        raw_kept = bool((~mask[start:start + m]).any())  # (one device synchronisation)
    g2 = g.reshape(-1, out_len)[:, :m]
    u1 = _pad_product(g2, inv[start:start + m], start, expected, rec)  # the trim's adjoint, / env
    sc = (math.sqrt(n_fft) if normalized else 1.0) / n_fft
    f = 2.0 * sc if onesided else sc  # the interior bins' factor, on the window
    stft_fn = stft if rec else (lambda *a: ComplexTensor._wrap(*_fc.execute_stft(*a)))
    spec = stft_fn(u1, win * f, n_fft, hop, False, False, onesided, frames)
    s_re, s_im = spec.real, spec.imag
    if raw_kept:  # the raw-sum samples inside the kept range: the same transform, window of ones
        u2 = _pad_product(g2, (~mask[start:start + m]).to(g2.dtype), start, expected, rec)
        raw = stft_fn(u2, torch.full_like(win, f), n_fft, hop, False, False, onesided, frames)
        s_re, s_im = s_re + raw.real, s_im + raw.imag
    if onesided:  # bins 0 and n/2 count once (real part) and carry no imaginary gradient
        h = n_fft // 2
        if rec:
            wr = _bin_weights(s_re.transpose(-2, -1), n_fft, 1.0, 0.5).unsqueeze(-1)
            wi = _bin_weights(s_im.transpose(-2, -1), n_fft, 1.0, 0.0).unsqueeze(-1)
            s_re, s_im = s_re * wr, s_im * wi
        elif h:  # rows 0 and h in one strided op each
            s_re[..., 0::h, :] *= 0.5
            s_im[..., 0::h, :] = 0.0
        else:
            s_re *= 0.5
            s_im.zero_()
    bins = s_re.shape[-2]
    return s_re.reshape(*lead, bins, frames), s_im.reshape(*lead, bins, frames)


class _IstftFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, re, im, win, n_fft, hop, center, normalized, onesided, length, default_win):
        ctx.save_for_backward(win)
        ctx.cfg = (n_fft, hop, center, normalized, onesided, re.shape[-1], length, default_win)
        return _fc.execute_istft(re, im, win, n_fft, hop, center, normalized, onesided, length)

    @staticmethod
    def backward(ctx, g):
        (win,) = ctx.saved_tensors
        n_fft, hop, center, normalized, onesided, frames, length, default_win = ctx.cfg
        d_re, d_im = _istft_adjoint(g if torch.is_grad_enabled() else g.contiguous(), win, n_fft, hop, center,
                                    normalized, onesided, frames, length, default_win)
        return d_re, d_im, None, None, None, None, None, None, None, None


def istft(re, im, win, n_fft, hop, center, normalized, onesided, length, default_win=None) -> torch.Tensor:
    """Fused inverse-STFT kernel on device fp32 spectra and the effective window; differentiable in
    the spectra (power-of-two n_fft; the window is taken as a constant).  default_win: the
    win_length of the default (periodic Hann) window when no window was given, else None."""
    if _grad_on(re, im):
        return _IstftFn.apply(re, im, win, n_fft, hop, center, normalized, onesided, length, default_win)
    return _fc.execute_istft(re, im, win, n_fft, hop, center, normalized, onesided, length)


# ---------------------------------------------------------------------------------------------
# complex GEMM / linear
# ---------------------------------------------------------------------------------------------


class _ComplexGEMMFn(torch.autograd.Function):
    """C = A @ op(B) (+ bias), op(B) = B or B^T; A (m, k) 2-D."""

    @staticmethod
    def forward(ctx, a_re, a_im, b_re, b_im, bias_re, bias_im, b_trans: bool, what: str):
        from .dispatch import gemm_ex

        ctx.save_for_backward(a_re, a_im, b_re, b_im)
        ctx.b_trans, ctx.has_bias = b_trans, bias_re is not None
        return gemm_ex(a_re, a_im, _lib.OP_N, b_re, b_im, _lib.OP_T if b_trans else _lib.OP_N, 1.0,
                       bias_re, bias_im, what=what)

    @staticmethod
    def backward(ctx, g_re, g_im):
        from .dispatch import gemm_ex

        a_re, a_im, b_re, b_im = ctx.saved_tensors
        need = ctx.needs_input_grad
        da_re = da_im = db_re = db_im = dbias_re = dbias_im = None
        if torch.is_grad_enabled():  # create_graph: the adjoint products through the differentiable gemm
            if need[0] or need[1]:  # dA = dC op(B)^H
                da_re, da_im = gemm(g_re, g_im, b_re, -b_im, not ctx.b_trans)
            if need[2] or need[3]:
                if ctx.b_trans:  # B = dC^T conj(A)
                    db_re, db_im = gemm(g_re.t().contiguous(), g_im.t().contiguous(), a_re, -a_im, False)
                else:  # B = A^H dC
                    db_re, db_im = gemm(a_re.t().contiguous(), (-a_im).t().contiguous(), g_re, g_im, False)
            if ctx.has_bias and (need[4] or need[5]):
                dbias_re, dbias_im = g_re.sum(0), g_im.sum(0)
            return da_re, da_im, db_re, db_im, dbias_re, dbias_im, None, None
        g_re, g_im = _c(g_re), _c(g_im)
        if need[0] or need[1]:
            # dA = dC op(B)^H: op(B) = B -> B^H (OP_C of B); op(B) = B^T (linear) -> conj(B) (OP_R)
            da_re, da_im = gemm_ex(g_re, g_im, _lib.OP_N, b_re, b_im, _lib.OP_R if ctx.b_trans else _lib.OP_C,
                                   what="complex_gemm backward dA")
        if need[2] or need[3]:
            if ctx.b_trans:
                # B^T = A^H dC  ->  B = dC^T conj(A)
                db_re, db_im = gemm_ex(g_re, g_im, _lib.OP_T, a_re, a_im, _lib.OP_R, what="complex_gemm backward dB")
            else:
                db_re, db_im = gemm_ex(a_re, a_im, _lib.OP_C, g_re, g_im, _lib.OP_N, what="complex_gemm backward dB")
        if ctx.has_bias and (need[4] or need[5]):
            dbias_re, dbias_im = g_re.sum(0), g_im.sum(0)
        return da_re, da_im, db_re, db_im, dbias_re, dbias_im, None, None


def gemm(a_re, a_im, b_re, b_im, b_trans: bool, bias_re=None, bias_im=None, what="complex_gemm"):
    """(c_re, c_im) = A @ op(B) (+ bias) for 2-D device fp32 planes; differentiable."""
    if _grad_on(a_re, a_im, b_re, b_im, bias_re, bias_im):
        return _ComplexGEMMFn.apply(a_re, a_im, b_re, b_im, bias_re, bias_im, b_trans, what)
    from .dispatch import gemm_ex

    return gemm_ex(a_re, a_im, _lib.OP_N, b_re, b_im, _lib.OP_T if b_trans else _lib.OP_N, 1.0, bias_re, bias_im,
                   what=what)


class _ComplexBMMFn(torch.autograd.Function):
    """C_b = A_b @ B_b for b < batch; A (batch or 1, m, k), B (batch or 1, k, n) (1: shared)."""

    @staticmethod
    def forward(ctx, a_re, a_im, b_re, b_im, batch: int):
        from .dispatch import gemm_batched

        ctx.save_for_backward(a_re, a_im, b_re, b_im)
        ctx.batch = batch
        return gemm_batched(a_re, a_im, _lib.OP_N, b_re, b_im, _lib.OP_N, batch)

    @staticmethod
    def backward(ctx, g_re, g_im):
        from .dispatch import gemm_batched, gemm_ex

        a_re, a_im, b_re, b_im = ctx.saved_tensors
        batch = ctx.batch
        need = ctx.needs_input_grad
        da_re = da_im = db_re = db_im = None
        if torch.is_grad_enabled():  # create_graph: the adjoint products through the differentiable bmm
            if need[0] or need[1]:  # dA_b = dC_b B_b^H
                da_re, da_im = bmm(g_re, g_im, b_re.transpose(1, 2).contiguous(), (-b_im).transpose(1, 2).contiguous(),
                                   batch)
                if a_re.shape[0] == 1 and batch > 1:
                    da_re, da_im = da_re.sum(0, keepdim=True), da_im.sum(0, keepdim=True)
            if need[2] or need[3]:  # dB_b = A_b^H dC_b
                db_re, db_im = bmm(a_re.transpose(1, 2).contiguous(), (-a_im).transpose(1, 2).contiguous(), g_re, g_im,
                                   batch)
                if b_re.shape[0] == 1 and batch > 1:
                    db_re, db_im = db_re.sum(0, keepdim=True), db_im.sum(0, keepdim=True)
            return da_re, da_im, db_re, db_im, None
        g_re, g_im = _c(g_re), _c(g_im)
        if need[0] or need[1]:
            # dA_b = dC_b B_b^H, summed over the batch when A is shared
            da_re, da_im = gemm_batched(g_re, g_im, _lib.OP_N, b_re, b_im, _lib.OP_C, batch,
                                        what="complex_matmul backward dA")
            if a_re.shape[0] == 1 and batch > 1:
                da_re, da_im = da_re.sum(0, keepdim=True), da_im.sum(0, keepdim=True)
        if need[2] or need[3]:
            # dB_b = A_b^H dC_b, summed over the batch when B is shared
            if b_re.shape[0] == batch or batch == 1:
                db_re, db_im = gemm_batched(a_re, a_im, _lib.OP_C, g_re, g_im, _lib.OP_N, batch,
                                            what="complex_matmul backward dB")
            elif a_re.shape[0] == batch:
                # sum_b A_b^H dC_b = A_flat^H dC_flat with the batch stacked along the rows
                m, k = a_re.shape[1:]
                db_re, db_im = gemm_ex(a_re.reshape(batch * m, k), a_im.reshape(batch * m, k), _lib.OP_C,
                                       g_re.reshape(batch * m, -1), g_im.reshape(batch * m, -1), _lib.OP_N,
                                       what="complex_matmul backward dB")
                db_re, db_im = db_re.unsqueeze(0), db_im.unsqueeze(0)
            else:
                db_re, db_im = gemm_batched(a_re, a_im, _lib.OP_C, g_re.sum(0, keepdim=True),
                                            g_im.sum(0, keepdim=True), _lib.OP_N, 1, what="complex_matmul backward dB")
        return da_re, da_im, db_re, db_im, None


def bmm(a_re, a_im, b_re, b_im, batch: int):
    """(c_re, c_im) = batched A @ B, (batch, m, n); differentiable."""
    if _grad_on(a_re, a_im, b_re, b_im):
        return _ComplexBMMFn.apply(a_re, a_im, b_re, b_im, batch)
    from .dispatch import gemm_batched

    return gemm_batched(a_re, a_im, _lib.OP_N, b_re, b_im, _lib.OP_N, batch)


def fft_autograd(x_real: torch.Tensor, x_imag: torch.Tensor, inverse: bool, precision: str = "fast"):
    """(y_re, y_im) of the last-axis transform, differentiable (trnfft/nki/autograd.py:204-205)."""
    y = c2c(x_real, x_imag, inverse)
    return y.real, y.imag


def complex_gemm_autograd(a_real, a_imag, b_real, b_imag):
    """C = A @ B, differentiable (trnfft/nki/autograd.py:115-116)."""
    return gemm(a_real, a_imag, b_real, b_imag, False)


def complex_linear_autograd(x_real, x_imag, w_real, w_imag):
    """Y = X @ W^T, differentiable (trnfft/nki/autograd.py:158-159)."""
    return gemm(x_real, x_imag, w_real, w_imag, True, what="complex_linear")
