"""trnfft_amd — MI355X (gfx950) HIP backend for trnfft's FFT hot path.

Same surface as trnfft (trnfft/__init__.py:13-68): torch.fft-style transforms on the split
re/im ComplexTensor, plan caching, backend and precision selection, ComplexLinear.  Every
transform executes on hand-written HIP kernels through the C ABI in include/trnfft_amd.h;
there is no CPU fallback.
"""

__version__ = "0.1.0"

from .api import (
    fft,
    fft2,
    fftn,
    hfft,
    ifft,
    ifftn,
    ihfft,
    irfft,
    irfft2,
    irfftn,
    istft,
    rfft,
    rfft2,
    rfftn,
    stft,
)
from .complex import ComplexTensor, complex_matmul
from .dispatch import HAS_HIP, HAS_NKI, complex_gemm, complex_linear, get_backend, hip_accepts, set_backend
from .plan import FFTAlgorithm, FFTPlan, clear_plan_cache, create_plan
from .precision import get_precision, set_ozaki_product_precision_verified, set_precision

__all__ = [
    "fft",
    "ifft",
    "rfft",
    "hfft",
    "ihfft",
    "irfft",
    "fft2",
    "fftn",
    "ifftn",
    "rfft2",
    "irfft2",
    "rfftn",
    "irfftn",
    "stft",
    "istft",
    "ComplexTensor",
    "complex_matmul",
    "complex_gemm",
    "complex_linear",
    "create_plan",
    "clear_plan_cache",
    "FFTPlan",
    "FFTAlgorithm",
    "HAS_HIP",
    "HAS_NKI",
    "set_backend",
    "get_backend",
    "hip_accepts",
    "set_precision",
    "set_ozaki_product_precision_verified",
    "get_precision",
]
