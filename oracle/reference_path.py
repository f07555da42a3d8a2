"""CPU restatement of trnfft's pytorch-backend FFT path (test infrastructure only).

Every function works on CPU torch tensors (split real/imag planes, fp32 unless stated) and
follows the cited reference lines operation by operation, so that fp32 rounding matches the
reference's own CPU result.  Where the reference loops in Python over positions of identical
work (the per-k butterfly loop), the loop is vectorised over k; ``cooley_tukey_loop`` keeps
the literal loop and the tests check both forms agree bit for bit.
"""

from __future__ import annotations

import math
import time

import numpy as np
import torch

__all__ = [
    "padded_length",
    "bit_reverse_indices",
    "bit_reverse_indices_loop",
    "cooley_tukey",
    "cooley_tukey_loop",
    "LiteralLoopTiming",
    "bluestein",
    "reference_chirp",
    "fft_core",
    "fft",
    "ifft",
    "rfft",
    "irfft",
    "fftn",
    "ifftn",
    "fft2",
    "stft",
    "istft",
    "stft_num_frames",
    "complex_linear",
    "complex_matmul",
    "dft_gemm",
    "stage_parallel_fft",
    "factorize",
]


def padded_length(n: int) -> int:
    """Bluestein padded length, trnfft/plan.py:42: ``1 << (2n-2).bit_length()``."""
    return 1 << (2 * n - 2).bit_length()


def bit_reverse_indices_loop(n: int, bits: int) -> torch.Tensor:
    """Literal restatement of trnfft/fft_core.py:1379-1389 (scalar loop; small n only)."""
    result = torch.zeros(n, dtype=torch.long)
    for i in range(n):
        rev = 0
        val = i
        for _ in range(bits):
            rev = (rev << 1) | (val & 1)
            val >>= 1
        result[i] = rev
    return result


def bit_reverse_indices(n: int, bits: int) -> torch.Tensor:
    """Same permutation as trnfft/fft_core.py:1379-1389, computed with array ops."""
    idx = np.arange(n, dtype=np.int64)
    rev = np.zeros(n, dtype=np.int64)
    for b in range(bits):
        rev |= ((idx >> b) & 1) << (bits - 1 - b)
    return torch.from_numpy(rev)


def _twiddles(half: int, m: int, sign: float, dtype) -> tuple[torch.Tensor, torch.Tensor]:
    # trnfft/fft_core.py:86-88: angles = sign * 2.0 * math.pi * arange(half) / m in `dtype`
    angles = sign * 2.0 * math.pi * torch.arange(half, dtype=dtype) / m
    return torch.cos(angles), torch.sin(angles)


def cooley_tukey(re: torch.Tensor, im: torch.Tensor, inverse: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Radix-2 DIT of trnfft/fft_core.py:53-117 (pytorch branch), vectorised over k.

    Stage s works on groups of m = 2^(s+1): element k of the even half and of the odd half of
    every group form one butterfly with twiddle tw[k].  The reference's loop over k performs the
    same fp32 operations (t*o products, difference/sum, then e+p and e-p) on every group; here
    all k are processed at once through a (..., n/m, m) view.
    """
    if _LITERAL_LOOP is not None:
        return _LITERAL_LOOP.run(re, im, inverse)
    n = re.shape[-1]
    log2n = int(math.log2(n))
    assert 1 << log2n == n, f"Not power of 2: {n}"
    sign = 1.0 if inverse else -1.0
    indices = bit_reverse_indices(n, log2n)
    re = re[..., indices].clone()
    im = im[..., indices].clone()
    lead = re.shape[:-1]
    for s in range(log2n):
        m = 1 << (s + 1)
        half = m >> 1
        tw_re, tw_im = _twiddles(half, m, sign, re.dtype)
        r = re.reshape(*lead, n // m, m)
        i = im.reshape(*lead, n // m, m)
        e_re, o_re = r[..., :half], r[..., half:]
        e_im, o_im = i[..., :half], i[..., half:]
        prod_re = tw_re * o_re - tw_im * o_im
        prod_im = tw_re * o_im + tw_im * o_re
        new_re = torch.cat([e_re + prod_re, e_re - prod_re], dim=-1)
        new_im = torch.cat([e_im + prod_im, e_im - prod_im], dim=-1)
        re = new_re.reshape(*lead, n)
        im = new_im.reshape(*lead, n)
    if inverse:
        scale = 1.0 / n
        re = re * scale
        im = im * scale
    return re.contiguous(), im.contiguous()


def cooley_tukey_loop(
    re: torch.Tensor, im: torch.Tensor, inverse: bool, k_limit: int | None = None, stage_log: list | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """Literal restatement of trnfft/fft_core.py:67-117 with its per-k Python loop.

    Used to pin ``cooley_tukey`` (bit equality on small sizes) and as the CPU baseline, since
    this loop is where the reference's pytorch path spends its time.

    Timing sample only: with ``k_limit`` each stage runs just its first ``k_limit`` butterfly
    positions (the result is then NOT a transform) and appends (positions run, positions in the
    stage, seconds) to ``stage_log``.  Every position of a stage does the same work on tensors
    of the same size, so the stage's full time is its measured time x positions / run.
    """
    n = re.shape[-1]
    log2n = int(math.log2(n))
    assert 1 << log2n == n, f"Not power of 2: {n}"
    sign = 1.0 if inverse else -1.0
    indices = bit_reverse_indices(n, log2n)
    re = re[..., indices].clone()
    im = im[..., indices].clone()
    for s in range(log2n):
        m = 1 << (s + 1)
        half = m >> 1
        tw_re, tw_im = _twiddles(half, m, sign, re.dtype)
        run = half if k_limit is None else min(half, k_limit)
        t_stage = time.perf_counter()
        for k in range(run):
            even_idx = list(range(k, n, m))
            odd_idx = list(range(k + half, n, m))
            e_re = re[..., even_idx]
            e_im = im[..., even_idx]
            o_re = re[..., odd_idx]
            o_im = im[..., odd_idx]
            t_re = tw_re[k]
            t_im = tw_im[k]
            prod_re = t_re * o_re - t_im * o_im
            prod_im = t_re * o_im + t_im * o_re
            re[..., even_idx] = e_re + prod_re
            im[..., even_idx] = e_im + prod_im
            re[..., odd_idx] = e_re - prod_re
            im[..., odd_idx] = e_im - prod_im
        if stage_log is not None:
            stage_log.append((run, half, time.perf_counter() - t_stage))
    if inverse:
        scale = 1.0 / n
        re = re * scale
        im = im * scale
    return re, im


class LiteralLoopTiming:
    """Timing context (CPU baseline only): inside it every power-of-two transform that
    ``cooley_tukey`` would do (through fft_core, bluestein, fftn, stft, ...) runs the literal
    per-k loop of trnfft/fft_core.py:67-117 instead, capped at ``k_limit`` positions per stage.

    ``seconds`` = measured wall time of the timed region + the time of the skipped positions
    (each capped stage's measured time x (positions / run - 1)).  With ``k_limit=None`` nothing
    is skipped and the outputs are the reference's; with a cap the outputs are meaningless.
    """

    def __init__(self, k_limit: int | None = None):
        self.k_limit = k_limit
        self.skipped_s = 0.0
        self.positions_run = 0
        self.positions_total = 0
        self._t0 = 0.0
        self.seconds = 0.0

    def run(self, re, im, inverse):
        log: list = []
        out = cooley_tukey_loop(re, im, inverse, k_limit=self.k_limit, stage_log=log)
        for run, half, sec in log:
            self.positions_run += run
            self.positions_total += half
            if run < half:
                self.skipped_s += sec * (half / run - 1.0)
        return out

    def __enter__(self):
        global _LITERAL_LOOP
        if _LITERAL_LOOP is not None:
            raise RuntimeError("LiteralLoopTiming does not nest")
        _LITERAL_LOOP = self
        self._t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        global _LITERAL_LOOP
        self.seconds = time.perf_counter() - self._t0 + self.skipped_s
        _LITERAL_LOOP = None
        return False


_LITERAL_LOOP: LiteralLoopTiming | None = None


def _cmul(ar, ai, br, bi):
    # ComplexTensor.__mul__, trnfft/complex.py:84-89 (same operation order)
    return ar * br - ai * bi, ar * bi + ai * br


def reference_chirp(n: int, inverse: bool, dtype=torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """Chirp of trnfft/fft_core.py:1316-1320: exp(sign*i*pi*k^2/n) with the angle in `dtype`."""
    sign = 1.0 if inverse else -1.0
    k = torch.arange(n, dtype=dtype)
    chirp_angles = sign * math.pi * k * k / n
    return torch.cos(chirp_angles), torch.sin(chirp_angles)


def bluestein(re: torch.Tensor, im: torch.Tensor, inverse: bool, padded_n: int | None = None):
    """Bluestein chirp-z of trnfft/fft_core.py:1285-1376 ("fast" precision)."""
    n = re.shape[-1]
    m = padded_n if padded_n is not None else padded_length(n)
    chirp_re, chirp_im = reference_chirp(n, inverse, re.dtype)
    # step 1: y = x * chirp
    y_re, y_im = _cmul(re, im, chirp_re, chirp_im)
    # step 2: zero-pad to m
    batch_shape = re.shape[:-1]
    y_pad_re = torch.zeros(*batch_shape, m, dtype=re.dtype)
    y_pad_im = torch.zeros(*batch_shape, m, dtype=re.dtype)
    y_pad_re[..., :n] = y_re
    y_pad_im[..., :n] = y_im
    # step 3: h = conj(chirp), circularly wrapped (the loop at :1342-1344 vectorised)
    h_re = torch.zeros(m, dtype=re.dtype)
    h_im = torch.zeros(m, dtype=re.dtype)
    h_re[:n] = chirp_re
    h_im[:n] = -chirp_im
    if n > 1:
        h_re[m - n + 1 :] = torch.flip(chirp_re[1:], dims=[0])
        h_im[m - n + 1 :] = -torch.flip(chirp_im[1:], dims=[0])
    if len(batch_shape) > 0:
        h_re, h_im = h_re.unsqueeze(0), h_im.unsqueeze(0)
    # step 4: circular convolution via three power-of-two FFTs
    Y_re, Y_im = cooley_tukey(y_pad_re, y_pad_im, False)
    H_re, H_im = cooley_tukey(h_re, h_im, False)
    p_re, p_im = _cmul(Y_re, Y_im, H_re, H_im)
    c_re, c_im = cooley_tukey(p_re, p_im, True)
    # step 5: slice and multiply by the chirp
    r_re, r_im = _cmul(c_re[..., :n], c_im[..., :n], chirp_re, chirp_im)
    if inverse:
        scale = 1.0 / n
        r_re, r_im = r_re * scale, r_im * scale
    return r_re.contiguous(), r_im.contiguous()


def fft_core(re: torch.Tensor, im: torch.Tensor, inverse: bool = False):
    """trnfft/fft_core.py:22-50 for precision "fast": n==1 clone, pow2 radix-2, else Bluestein."""
    n = re.shape[-1]
    if n == 1:
        return re.clone(), im.clone()
    if n & (n - 1) == 0:
        return cooley_tukey(re, im, inverse)
    return bluestein(re, im, inverse, padded_n=padded_length(n))


def _as_pair(x):
    if isinstance(x, tuple):
        re, im = x
        return re.contiguous(), im.contiguous()
    if torch.is_complex(x):
        return x.real.contiguous(), x.imag.contiguous()
    return x.contiguous(), torch.zeros_like(x)


def _resize_last(re, im, n):
    # trnfft/api.py:482-493
    cur = re.shape[-1]
    if cur == n:
        return re, im
    if cur < n:
        pad = torch.zeros(*re.shape[:-1], n - cur, dtype=re.dtype)
        return torch.cat([re, pad], dim=-1), torch.cat([im, pad], dim=-1)
    return re[..., :n].contiguous(), im[..., :n].contiguous()


def fft(x, n: int | None = None):
    """trnfft/api.py:22-27."""
    re, im = _as_pair(x)
    if n is not None:
        re, im = _resize_last(re, im, n)
    return fft_core(re, im, False)


def ifft(x, n: int | None = None):
    """trnfft/api.py:30-35."""
    re, im = _as_pair(x)
    if n is not None:
        re, im = _resize_last(re, im, n)
    return fft_core(re, im, True)


def rfft(x: torch.Tensor, n: int | None = None):
    """trnfft/api.py:38-46: full c2c of the real input, sliced to n//2+1."""
    if n is not None:
        cur = x.shape[-1]
        if cur < n:
            x = torch.cat([x, torch.zeros(*x.shape[:-1], n - cur, dtype=x.dtype)], dim=-1)
        elif cur > n:
            x = x[..., :n]
    n = x.shape[-1]
    re, im = fft_core(x.contiguous(), torch.zeros_like(x), False)
    half = n // 2 + 1
    return re[..., :half].contiguous(), im[..., :half].contiguous()


def irfft(x, n: int | None = None) -> torch.Tensor:
    """trnfft/api.py:49-68: Hermitian reconstruction, inverse c2c, real part."""
    re, im = x
    if n is None:
        n = 2 * (re.shape[-1] - 1)
    full_re = torch.zeros(*re.shape[:-1], n, dtype=re.dtype)
    full_im = torch.zeros(*re.shape[:-1], n, dtype=re.dtype)
    half = re.shape[-1]
    full_re[..., :half] = re
    full_im[..., :half] = im
    if n > 1:
        num_neg = n - half
        full_re[..., half:] = torch.flip(re[..., 1 : 1 + num_neg], dims=[-1])
        full_im[..., half:] = -torch.flip(im[..., 1 : 1 + num_neg], dims=[-1])
    out_re, _ = fft_core(full_re, full_im, True)
    return out_re


def _fft_along_dim(re, im, dim, inverse):
    # trnfft/api.py:496-516 (transpose copy, flatten, fft_core, reshape, transpose back)
    ndim = re.dim()
    dim = dim % ndim
    if dim != ndim - 1:
        re = re.transpose(dim, -1).contiguous()
        im = im.transpose(dim, -1).contiguous()
    shape = re.shape
    n = shape[-1]
    r, i = fft_core(re.reshape(-1, n), im.reshape(-1, n), inverse)
    re, im = r.reshape(shape), i.reshape(shape)
    if dim != ndim - 1:
        re = re.transpose(dim, -1).contiguous()
        im = im.transpose(dim, -1).contiguous()
    return re, im


def fftn(x, dim=None, inverse: bool = False):
    """trnfft/api.py:111-139 (and ifftn :142-167) without the s= resize."""
    re, im = _as_pair(x)
    ndim = re.dim()
    if dim is None:
        dim = tuple(range(-ndim, 0))
    dim = tuple(d % ndim for d in dim)
    for d in dim:
        re, im = _fft_along_dim(re, im, d, inverse)
    return re, im


def ifftn(x, dim=None):
    return fftn(x, dim=dim, inverse=True)


def fft2(x):
    """trnfft/api.py:105-108: fftn over (-2, -1), dim -2 first."""
    return fftn(x, dim=(-2, -1))


def stft_num_frames(length: int, n_fft: int, hop_length: int, center: bool = True) -> int:
    padded = length + 2 * (n_fft // 2) if center else length
    return 1 + (padded - n_fft) // hop_length


def stft(
    x: torch.Tensor,
    n_fft: int,
    hop_length: int | None = None,
    win_length: int | None = None,
    window: torch.Tensor | None = None,
    center: bool = True,
    pad_mode: str = "reflect",
    normalized: bool = False,
    onesided: bool = True,
):
    """trnfft/api.py:291-365; frames go through fft_core (multi_core_fft disabled)."""
    if hop_length is None:
        hop_length = n_fft // 4
    if win_length is None:
        win_length = n_fft
    if window is None:
        window = torch.hann_window(win_length, dtype=x.dtype)
    if center:
        pad_amount = n_fft // 2
        x = x.unsqueeze(0) if x.dim() == 1 else x
        x = torch.nn.functional.pad(x, (pad_amount, pad_amount), mode=pad_mode)
        x = x.squeeze(0) if x.dim() == 2 and x.shape[0] == 1 else x
    padded_length = x.shape[-1]
    num_frames = 1 + (padded_length - n_fft) // hop_length
    frame_idx = torch.arange(n_fft).unsqueeze(0) + torch.arange(num_frames).unsqueeze(1) * hop_length
    frames = x[..., frame_idx]
    if win_length < n_fft:
        padded_window = torch.zeros(n_fft, dtype=x.dtype)
        offset = (n_fft - win_length) // 2
        padded_window[offset : offset + win_length] = window
        frames = frames * padded_window
    else:
        frames = frames * window
    orig_shape = frames.shape
    f_re = frames.contiguous().reshape(-1, n_fft)
    r_re, r_im = fft_core(f_re, torch.zeros_like(f_re), False)
    r_re = r_re.reshape(orig_shape)
    r_im = r_im.reshape(orig_shape)
    if onesided:
        bins = n_fft // 2 + 1
        r_re, r_im = r_re[..., :bins], r_im[..., :bins]
    r_re = r_re.transpose(-2, -1)
    r_im = r_im.transpose(-2, -1)
    if normalized:
        scale = 1.0 / math.sqrt(n_fft)
        r_re, r_im = r_re * scale, r_im * scale
    return r_re.contiguous(), r_im.contiguous()


def istft(
    spec,
    n_fft: int,
    hop_length: int | None = None,
    win_length: int | None = None,
    window: torch.Tensor | None = None,
    center: bool = True,
    normalized: bool = False,
    onesided: bool = True,
    length: int | None = None,
) -> torch.Tensor:
    """trnfft/api.py:368-470 (overlap-add loops vectorised with index_add)."""
    s_re, s_im = spec
    if hop_length is None:
        hop_length = n_fft // 4
    if win_length is None:
        win_length = n_fft
    if window is None:
        window = torch.hann_window(win_length, dtype=s_re.dtype)
    if normalized:
        scale = math.sqrt(n_fft)
        s_re, s_im = s_re * scale, s_im * scale
    spec_re = s_re.transpose(-2, -1)
    spec_im = s_im.transpose(-2, -1)
    if onesided:
        bins = spec_re.shape[-1]
        full_re = torch.zeros(*spec_re.shape[:-1], n_fft, dtype=spec_re.dtype)
        full_im = torch.zeros(*spec_im.shape[:-1], n_fft, dtype=spec_im.dtype)
        full_re[..., :bins] = spec_re
        full_im[..., :bins] = spec_im
        if n_fft > 1:
            num_neg = n_fft - bins
            full_re[..., bins:] = torch.flip(spec_re[..., 1 : 1 + num_neg], dims=[-1])
            full_im[..., bins:] = -torch.flip(spec_im[..., 1 : 1 + num_neg], dims=[-1])
        spec_re, spec_im = full_re, full_im
    num_frames = spec_re.shape[-2]
    f_re, _ = fft_core(spec_re.contiguous().reshape(-1, n_fft), spec_im.contiguous().reshape(-1, n_fft), True)
    frames = f_re.reshape(*spec_re.shape[:-1], n_fft)
    if win_length < n_fft:
        padded = torch.zeros(n_fft, dtype=window.dtype)
        offset = (n_fft - win_length) // 2
        padded[offset : offset + win_length] = window
        window = padded
    expected_len = n_fft + (num_frames - 1) * hop_length
    batch_shape = frames.shape[:-2]
    output = torch.zeros(*batch_shape, expected_len, dtype=frames.dtype)
    window_sum = torch.zeros(expected_len, dtype=frames.dtype)
    raw_output = torch.zeros(*batch_shape, expected_len, dtype=frames.dtype)
    for t in range(num_frames):
        start = t * hop_length
        output[..., start : start + n_fft] += frames[..., t, :] * window
        window_sum[start : start + n_fft] += window**2
        raw_output[..., start : start + n_fft] += frames[..., t, :]
    mask = window_sum > 1e-8
    output[..., mask] = output[..., mask] / window_sum[mask]
    output[..., ~mask] = raw_output[..., ~mask]
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
            pad = torch.zeros(*batch_shape, length - cur, dtype=output.dtype)
            output = torch.cat([output, pad], dim=-1)
    return output


def complex_matmul(a, b):
    """trnfft/complex.py:142-150: four real matmuls."""
    ar, ai = a
    br, bi = b
    re = torch.matmul(ar, br) - torch.matmul(ai, bi)
    im = torch.matmul(ar, bi) + torch.matmul(ai, br)
    return re, im


def complex_linear(x, w_re, w_im, bias_re=None, bias_im=None):
    """ComplexLinear.forward pytorch branch, trnfft/nn.py:43-48 (y = x W^T + b)."""
    xr, xi = x
    lin = torch.nn.functional.linear
    re = lin(xr, w_re) - lin(xi, w_im)
    im = lin(xi, w_re) + lin(xr, w_im)
    if bias_re is not None:
        re = re + bias_re
        im = im + bias_im
    return re, im


def dft_gemm(re: torch.Tensor, im: torch.Tensor, inverse: bool, fp32_angles: bool = False):
    """DFT as one complex GEMM, trnfft/fft_core.py:221-251: X = x @ W.

    ``fp32_angles=True`` builds W exactly as the reference (angle 2*pi*k*j/n in fp32, :239-243);
    the default builds W from the exact integer phase (k*j mod n) in float64, the accurate DFT
    matrix used as the parity oracle for the HIP DFT-GEMM path (the reference's pytorch backend
    never takes this route: on CPU trnfft.fft runs cooley_tukey).
    """
    n = re.shape[-1]
    sign = 1.0 if inverse else -1.0
    if fp32_angles:
        k = torch.arange(n, dtype=re.dtype)
        kj = k.unsqueeze(1) * k.unsqueeze(0)
        angles = sign * 2.0 * math.pi * kj / n
        w_re, w_im = torch.cos(angles), torch.sin(angles)
        out = complex_matmul((re, im), (w_re, w_im))
    else:
        k = torch.arange(n, dtype=torch.int64)
        ph = (k.unsqueeze(1) * k.unsqueeze(0)) % n
        angles = sign * 2.0 * math.pi * ph.to(torch.float64) / n
        w_re, w_im = torch.cos(angles), torch.sin(angles)
        r, i = complex_matmul((re.double(), im.double()), (w_re, w_im))
        out = (r.to(re.dtype), i.to(re.dtype))
    if inverse:
        return out[0] * (1.0 / n), out[1] * (1.0 / n)
    return out


def factorize(n: int) -> tuple[int, int]:
    """trnfft/nki/multicore.py:134-148: largest divisor n1 <= sqrt(n), n2 = n // n1."""
    n1 = int(n**0.5)
    while n1 > 1 and n % n1 != 0:
        n1 -= 1
    if n1 <= 1:
        raise ValueError(f"n={n} has no non-trivial divisors (prime); row-column FFT not applicable")
    return n1, n // n1


def stage_parallel_fft(re: torch.Tensor, im: torch.Tensor, inverse: bool):
    """Row-column FFT of one transform, trnfft/nki/multicore.py:151-219 (shards run in order)."""
    n = re.shape[-1]
    n1, n2 = factorize(n)
    sign = 1.0 if inverse else -1.0
    x_re = re.reshape(n).float().reshape(n1, n2)
    x_im = im.reshape(n).float().reshape(n1, n2)
    c_re, c_im = fft_core(x_re.T.contiguous(), x_im.T.contiguous(), inverse)
    y_re, y_im = c_re.T.contiguous(), c_im.T.contiguous()
    k1 = torch.arange(n1, dtype=torch.float32).unsqueeze(1)
    l = torch.arange(n2, dtype=torch.float32).unsqueeze(0)  # noqa: E741
    angles = sign * 2.0 * math.pi * l * k1 / n
    tw_re, tw_im = torch.cos(angles), torch.sin(angles)
    z_re = y_re * tw_re - y_im * tw_im
    z_im = y_re * tw_im + y_im * tw_re
    r_re, r_im = fft_core(z_re.contiguous(), z_im.contiguous(), inverse)
    return r_re.T.contiguous().reshape(n), r_im.T.contiguous().reshape(n)
