"""Precision-mode selection, interface of trnfft/precision.py:70-94.

The HIP backend executes the reference's default ``"fast"`` mode (straight fp32).  The other
modes the reference accepts are Trainium precision experiments (bf16/Ozaki GEMMs, Kahan
butterflies, fp64 host Bluestein); they are valid values here too, but asking the HIP backend to
run them raises NotImplementedError instead of silently computing in fp32.
"""

from __future__ import annotations

_VALID = ("fast", "kahan", "double", "bf16", "bf16_refined", "ozaki", "ozaki_hq")
_SUPPORTED = ("fast",)

_precision: str = "fast"


def set_precision(mode: str) -> None:
    """Set the global precision mode (trnfft/precision.py:75-80)."""
    global _precision
    if mode not in _VALID:
        raise ValueError(f"precision mode must be one of {_VALID}; got {mode!r}")
    _precision = mode


def get_precision() -> str:
    return _precision


_ozaki_product_precision_verified = False


def set_ozaki_product_precision_verified(verified: bool = True) -> None:
    """Interface of trnfft/fft_core.py:186-197 (declares that the matrix units multiply bf16
    pairs at fp32 precision, enabling the reference's "ozaki" modes).  Recorded for callers that
    set it; the Ozaki modes themselves are Trainium experiments that this backend does not run
    (``_resolve`` raises NotImplementedError for them either way)."""
    global _ozaki_product_precision_verified
    _ozaki_product_precision_verified = bool(verified)


def _resolve(precision) -> str:
    """Per-call override against the global (trnfft/precision.py:88-94), restricted to "fast"."""
    if precision is None:
        precision = _precision
    elif precision not in _VALID:
        raise ValueError(f"precision must be one of {_VALID} or None; got {precision!r}")
    if precision not in _SUPPORTED:
        raise NotImplementedError(
            f"precision={precision!r} is a Trainium-specific mode; the HIP backend runs 'fast' (fp32) only"
        )
    return precision
