"""FFT plans: the reference's algorithm choice plus the device-side plans that own the tables.

``FFTPlan`` / ``create_plan`` / ``clear_plan_cache`` keep trnfft's interface and keying
(trnfft/plan.py:14-50): power-of-two n -> COOLEY_TUKEY, anything else -> BLUESTEIN with
``padded_n = 1 << (2n-2).bit_length()``.  Unlike the reference, which caches only that choice
and rebuilds twiddles, bit reversal, chirp and filter spectrum on every call
(trnfft/fft_core.py:75,86-88,1316-1345), the native plan built here owns all device tables and
is cached per (kind, n, direction, device, extra) for the life of the process.
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from enum import Enum, auto

from . import _lib


class FFTAlgorithm(Enum):
    COOLEY_TUKEY = auto()
    BLUESTEIN = auto()


@dataclass(frozen=True)
class FFTPlan:
    n: int
    algorithm: FFTAlgorithm
    inverse: bool
    padded_n: int | None = None  # For Bluestein

    @property
    def is_power_of_2(self) -> bool:
        return self.algorithm == FFTAlgorithm.COOLEY_TUKEY


_plan_cache: dict[tuple, FFTPlan] = {}
_native_cache: dict[tuple, NativePlan] = {}
_lock = threading.Lock()


def create_plan(n: int, inverse: bool = False) -> FFTPlan:
    """Algorithm choice for length n, cached by (n, inverse) (trnfft/plan.py:34-46)."""
    key = (n, inverse)
    plan = _plan_cache.get(key)
    if plan is not None:
        return plan
    if n & (n - 1) == 0:
        plan = FFTPlan(n=n, algorithm=FFTAlgorithm.COOLEY_TUKEY, inverse=inverse)
    else:
        m = 1 << (2 * n - 2).bit_length()
        plan = FFTPlan(n=n, algorithm=FFTAlgorithm.BLUESTEIN, inverse=inverse, padded_n=m)
    with _lock:
        _plan_cache[key] = plan
    return plan


def clear_plan_cache():
    """Drop every cached plan, releasing the native plans' device tables."""
    with _lock:
        _plan_cache.clear()
        natives = list(_native_cache.values())
        _native_cache.clear()
    for p in natives:
        p.destroy()


class NativePlan:
    """Owner of one ``tfa_plan`` (device tables) created on a given device."""

    __slots__ = ("handle", "kind", "n", "inverse", "device", "padded_n", "hop", "flags", "n2")

    def __init__(self, kind: int, n: int, inverse: bool, device: int, hop: int = 0, flags: int = 0, n2: int = 0):
        import torch

        self.kind, self.n, self.inverse, self.device = kind, n, inverse, device
        self.hop, self.flags, self.n2 = hop, flags, n2
        desc = _lib.PlanDesc(kind=kind, inverse=int(bool(inverse)), n=n, hop=hop, flags=flags, reserved=0, n2=n2)
        handle = ctypes.c_void_p()
        lib = _lib.lib()
        with torch.cuda.device(device):
            _lib.check(lib.tfa_plan_create(ctypes.byref(handle), ctypes.byref(desc)), "tfa_plan_create")
        self.handle = handle
        self.padded_n = int(lib.tfa_plan_padded_n(handle))

    def workspace_bytes(self, batch: int) -> int:
        out = ctypes.c_size_t()
        _lib.check(_lib.lib().tfa_plan_workspace_size(self.handle, batch, ctypes.byref(out)), "tfa_plan_workspace_size")
        return int(out.value)

    def destroy(self) -> None:
        if self.handle:
            _lib.lib().tfa_plan_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:  # interpreter shutdown
            pass


def native_plan(kind: int, n: int, inverse: bool, device: int, hop: int = 0, flags: int = 0, n2: int = 0) -> NativePlan:
    key = (kind, n, bool(inverse), device, hop, flags, n2)
    p = _native_cache.get(key)
    if p is not None:
        return p
    with _lock:
        p = _native_cache.get(key)
        if p is None:
            p = NativePlan(kind, n, inverse, device, hop, flags, n2)
            _native_cache[key] = p
    return p
