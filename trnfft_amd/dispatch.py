"""Backend dispatch (interface of trnfft/nki/dispatch.py:50-102, with "hip" in place of "nki").

    "auto"    — HIP if the native library loads and a gfx950 GPU is visible
    "pytorch" — do not use this backend (the caller's own pytorch path runs instead)
    "hip"     — always HIP (RuntimeError at selection time if unavailable)

This package is the HIP dispatch target only: every compute entry point raises RuntimeError
when ``_use_hip()`` is False.  There is no CPU fallback inside it; trnfft keeps its own pytorch
path and consults ``_use_hip()`` before delegating here.

CPU inputs are moved to the current GPU and results moved back, as the reference's NKI path
does with its XLA device (trnfft/nki/dispatch.py:423-428, trnfft/nki/autograd.py:58-60).
"""

from __future__ import annotations

import ctypes
import functools

import torch

from . import _lib
from .complex import ComplexTensor
from .precision import _SUPPORTED as _SUPPORTED_PRECISION

HAS_HIP = _lib.library_present()
# the reference's flag (trnfft/nki/dispatch.py:17-24): this backend has no NKI path
HAS_NKI = False

_backend = "auto"


def set_backend(backend: str):
    """Set dispatch backend: 'auto', 'pytorch', or 'hip' (trnfft/nki/dispatch.py:53-59)."""
    global _backend
    assert backend in ("auto", "pytorch", "hip")
    if backend == "hip" and not _hip_ready():
        raise RuntimeError(
            "HIP backend requires libtrnfft_amd.so (python -m trnfft_amd.csrc.build) and a gfx950 GPU"
        )
    _backend = backend


def get_backend() -> str:
    return _backend


@functools.lru_cache(maxsize=1)
def _hip_ready() -> bool:
    if not HAS_HIP:
        return False
    try:
        _lib.lib()
    except OSError:
        return False
    if not torch.cuda.is_available():
        return False
    try:
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except Exception:
        return False
    return arch.startswith("gfx950")


def _use_hip() -> bool:
    if _backend == "hip":
        return True
    if _backend == "pytorch":
        return False
    return _hip_ready()


def hip_accepts(*tensors: torch.Tensor | None, precision: str = "fast") -> bool:
    """Whether a call should be routed to this backend at all.

    True only when the backend is selected and usable (``_use_hip()``), the caller's *resolved*
    precision mode is ``"fast"`` -- the caller resolves its per-call override against its own
    global first, as trnfft/precision.py:88-94 does for trnfft/fft_core.py:37-39 -- and every
    tensor given (signal planes, window, weights; None is skipped) is a real float32 tensor.
    The reference computes in its input's dtype (twiddles in ``re.dtype``, fft_core.py:84-88; the
    chirp in ``x.dtype``, :1317; the window in ``input.dtype``, api.py:307-308) and runs its
    "kahan"/"double" modes on its own path, so for anything else the caller keeps that path.
    Asked directly, this package raises for such calls (TypeError for other dtypes,
    NotImplementedError for other modes); it never computes them in fp32."""
    if precision not in _SUPPORTED_PRECISION:
        return False
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float32:
            return False
    return _use_hip()


def _require_hip(what: str) -> None:
    if not _use_hip():
        if _backend == "pytorch":
            raise RuntimeError(
                f"trnfft_amd.{what}: backend is 'pytorch'; the pytorch path belongs to trnfft itself "
                "(trnfft_amd only executes the HIP target)"
            )
        raise RuntimeError(
            f"trnfft_amd.{what}: HIP backend unavailable (needs libtrnfft_amd.so built for gfx950 and a "
            "visible gfx950 GPU); no CPU fallback exists in this package"
        )
    _lib.lib()


def target_device(*tensors: torch.Tensor) -> torch.device:
    """Device to run on: the inputs' GPU, or the current GPU for CPU inputs."""
    for t in tensors:
        if t is not None and t.is_cuda:
            return t.device
    return torch.device("cuda", torch.cuda.current_device())


def to_device_f32(t: torch.Tensor | None, dev: torch.device) -> torch.Tensor | None:
    """Contiguous fp32 copy of t on dev (no copy when it already is one)."""
    if t is None:
        return None
    if t.dtype != torch.float32:
        raise TypeError(f"the HIP backend computes in fp32; got {t.dtype}")
    return t.to(dev, non_blocking=False).contiguous()


def to_device_f32_strided(t: torch.Tensor | None, dev: torch.device) -> torch.Tensor | None:
    """fp32 t on dev with its strides kept (no copy when it already is there): for inputs a kernel
    takes in more than one memory order (the STFT spectra planes)."""
    if t is None:
        return None
    if t.dtype != torch.float32:
        raise TypeError(f"the HIP backend computes in fp32; got {t.dtype}")
    return t.to(dev, non_blocking=False)


def stream_handle(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def gemm_ex(a_re, a_im, a_op: int, b_re, b_im, b_op: int, alpha: float = 1.0, bias_re=None, bias_im=None,
            what: str = "complex_gemm"):
    """C = alpha * op(A) @ op(B) (+ bias) on the MFMA kernel for 2-D device fp32 planes; returns
    (c_re, c_im).  op: _lib.OP_N (X), OP_T (X^T), OP_C (conj(X)^T), OP_R (conj(X))."""
    dev = a_re.device
    a_re, a_im, b_re, b_im = (t.contiguous() for t in (a_re, a_im, b_re, b_im))
    at = a_op in (_lib.OP_T, _lib.OP_C)
    bt = b_op in (_lib.OP_T, _lib.OP_C)
    m, k = (a_re.shape[1], a_re.shape[0]) if at else a_re.shape
    kb, n = (b_re.shape[1], b_re.shape[0]) if bt else b_re.shape
    if kb != k:
        raise ValueError(f"{what}: inner dimensions differ ({k} vs {kb})")
    c_re = torch.empty(m, n, device=dev, dtype=torch.float32)
    c_im = torch.empty(m, n, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_complex_gemm_ex(
            m, n, k, ptr(a_re), ptr(a_im), a_re.shape[1], a_op, ptr(b_re), ptr(b_im), b_re.shape[1], b_op,
            float(alpha), ptr(bias_re), ptr(bias_im), ptr(c_re), ptr(c_im), n, stream_handle(dev),
        )
    _lib.check(rc, what)
    return c_re, c_im


def gemm_batched(a_re, a_im, a_op: int, b_re, b_im, b_op: int, batch: int, alpha: float = 1.0,
                 what: str = "complex_matmul"):
    """C_b = alpha * op(A_b) @ op(B_b) for b < batch on the MFMA kernel; A and B are 3-D device fp32
    planes whose first axis is `batch` or 1 (1: the matrix is shared by every product).  Returns
    (c_re, c_im) of shape (batch, m, n)."""
    dev = a_re.device
    a_re, a_im, b_re, b_im = (t.contiguous() for t in (a_re, a_im, b_re, b_im))
    at = a_op in (_lib.OP_T, _lib.OP_C)
    bt = b_op in (_lib.OP_T, _lib.OP_C)
    m, k = (a_re.shape[2], a_re.shape[1]) if at else a_re.shape[1:]
    kb, n = (b_re.shape[2], b_re.shape[1]) if bt else b_re.shape[1:]
    if kb != k:
        raise RuntimeError(f"{what}: inner dimensions differ ({k} vs {kb})")
    sa = 0 if a_re.shape[0] == 1 else a_re.shape[1] * a_re.shape[2]
    sb = 0 if b_re.shape[0] == 1 else b_re.shape[1] * b_re.shape[2]
    c_re = torch.empty(batch, m, n, device=dev, dtype=torch.float32)
    c_im = torch.empty(batch, m, n, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        rc = _lib.lib().tfa_complex_gemm_batched(
            batch, m, n, k, ptr(a_re), ptr(a_im), a_re.shape[2], sa, a_op, ptr(b_re), ptr(b_im), b_re.shape[2], sb,
            b_op, float(alpha), ptr(None), ptr(None), ptr(c_re), ptr(c_im), n, m * n, stream_handle(dev),
        )
    _lib.check(rc, what)
    return c_re, c_im


def _gemm(a_re, a_im, b_re, b_im, b_trans: bool, bias_re=None, bias_im=None, what="complex_gemm"):
    """op(B) = B or B^T; A's leading dimensions are batch rows.  Differentiable (the adjoint
    products run on the same kernel)."""
    from . import autograd as _ag

    _require_hip(what)
    dev = target_device(a_re, b_re)
    out_dev = a_re.device
    a_re, a_im = to_device_f32(a_re, dev), to_device_f32(a_im, dev)
    b_re, b_im = to_device_f32(b_re, dev), to_device_f32(b_im, dev)
    bias_re, bias_im = to_device_f32(bias_re, dev), to_device_f32(bias_im, dev)
    if b_re.dim() != 2:
        raise ValueError(f"{what}: expects a 2-D right operand")
    lead = a_re.shape[:-1]
    k = a_re.shape[-1]
    c_re, c_im = _ag.gemm(a_re.reshape(-1, k), a_im.reshape(-1, k), b_re, b_im, b_trans, bias_re, bias_im, what)
    out = ComplexTensor._wrap(c_re.reshape(*lead, c_re.shape[-1]), c_im.reshape(*lead, c_im.shape[-1]))
    return out if out_dev == dev else out.to(out_dev)


def complex_matmul(a: ComplexTensor, b: ComplexTensor) -> ComplexTensor:
    """A @ B with torch.matmul's shape rules (trnfft/complex.py:142-150 runs four torch.matmul):
    1-D operands are promoted and the added axis removed, a 2-D right operand makes A's leading
    axes rows of one GEMM, and batched operands broadcast over their leading axes and run as one
    strided-batched launch.  Every product runs on the MFMA kernel."""
    ar, ai, br, bi = a.real, a.imag, b.real, b.imag
    if ar.dim() == 0 or br.dim() == 0:
        raise RuntimeError("complex_matmul: both arguments need to be at least 1-D")
    pre, post = ar.dim() == 1, br.dim() == 1
    if pre:
        ar, ai = ar.unsqueeze(0), ai.unsqueeze(0)
    if post:
        br, bi = br.unsqueeze(-1), bi.unsqueeze(-1)
    if ar.shape[-1] != br.shape[-2]:
        raise RuntimeError(
            f"complex_matmul: shapes {tuple(a.real.shape)} and {tuple(b.real.shape)} cannot be multiplied"
        )
    if br.dim() == 2:
        out = _gemm(ar, ai, br, bi, False, what="complex_matmul")
        re, im = out.real, out.imag
    else:
        re, im = _bmm(ar, ai, br, bi)
    if post:
        re, im = re.squeeze(-1), im.squeeze(-1)
    if pre:
        d = -1 if post else -2
        re, im = re.squeeze(d), im.squeeze(d)
    return ComplexTensor._wrap(re, im)


def _bmm(a_re, a_im, b_re, b_im):
    """Broadcast batched product of (..., m, k) and (..., k, n) planes (b at least 3-D)."""
    from . import autograd as _ag

    _require_hip("complex_matmul")
    dev = target_device(a_re, b_re)
    out_dev = a_re.device
    a_re, a_im = to_device_f32(a_re, dev), to_device_f32(a_im, dev)
    b_re, b_im = to_device_f32(b_re, dev), to_device_f32(b_im, dev)
    m, k = a_re.shape[-2:]
    n = b_re.shape[-1]
    bshape = torch.broadcast_shapes(a_re.shape[:-2], b_re.shape[:-2])
    batch = 1
    for d in bshape:
        batch *= d

    def batched(x_re, x_im, rows, cols):
        # a matrix shared by the whole batch keeps a batch axis of 1 (stride 0 in the launch);
        # otherwise the operand is broadcast to the full batch
        own = 1
        for d in x_re.shape[:-2]:
            own *= d
        if own == 1:
            return x_re.reshape(1, rows, cols), x_im.reshape(1, rows, cols)
        return (x_re.expand(*bshape, rows, cols).reshape(batch, rows, cols),
                x_im.expand(*bshape, rows, cols).reshape(batch, rows, cols))

    if batch == 0 or m == 0 or n == 0:
        z = torch.zeros(*bshape, m, n, device=dev, dtype=torch.float32)
        re, im = z, z.clone()
    else:
        a3 = batched(a_re, a_im, m, k)
        b3 = batched(b_re, b_im, k, n)
        c_re, c_im = _ag.bmm(a3[0], a3[1], b3[0], b3[1], batch)
        re, im = c_re.reshape(*bshape, m, n), c_im.reshape(*bshape, m, n)
    if out_dev != dev:
        re, im = re.to(out_dev), im.to(out_dev)
    return re, im


def complex_gemm(a: ComplexTensor, b: ComplexTensor) -> ComplexTensor:
    """C = A @ B on the MFMA complex GEMM (trnfft/nki/dispatch.py:74-84)."""
    if a.real.dim() != 2 or b.real.dim() != 2:
        raise ValueError("complex_gemm expects 2-D operands")
    return _gemm(a.real, a.imag, b.real, b.imag, False)


def complex_linear(
    x: ComplexTensor,
    w_real: torch.Tensor,
    w_imag: torch.Tensor,
    bias_real: torch.Tensor | None = None,
    bias_imag: torch.Tensor | None = None,
) -> ComplexTensor:
    """y = x @ W^T (+ bias) with W (out, in) (trnfft/nki/dispatch.py:91-102, trnfft/nn.py:46-48)."""
    return _gemm(x.real, x.imag, w_real, w_imag, True, bias_real, bias_imag, what="complex_linear")
