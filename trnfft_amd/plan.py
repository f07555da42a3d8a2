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
from collections import OrderedDict
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
_lock = threading.Lock()

# Native plans kept alive by the cache (least recently used evicted first).  Plans own device
# tables (up to ~130 MB for the longest Bluestein lengths); a plan leaves memory only when the
# last Python reference to it is gone, so a call that fetched a plan keeps it valid until it
# returns, whatever another thread does to the cache meanwhile.  A plan used under HIP-graph
# capture is retained by the native library itself until the process exits (tfa_plan_destroy
# does not free a captured plan's tables), so replays stay valid after an eviction or a clear.
NATIVE_CACHE_MAX = 64


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
    """Drop every cached plan (trnfft/plan.py:49-50).  Native plans release their device tables
    once no caller still holds them (captured plans stay with the native library)."""
    with _lock:
        _plan_cache.clear()
        _native_cache.clear()


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


class _LruCache:
    """Bounded key -> plan map; the least recently used entry is dropped past `limit`."""

    def __init__(self, limit: int):
        self.limit = limit
        self._d: OrderedDict = OrderedDict()

    def get(self, key):
        p = self._d.get(key)
        if p is not None:
            self._d.move_to_end(key)
        return p

    def put(self, key, plan) -> None:
        self._d[key] = plan
        self._d.move_to_end(key)
        while len(self._d) > self.limit:
            self._d.popitem(last=False)

    def clear(self) -> None:
        self._d.clear()

    def __len__(self) -> int:
        return len(self._d)

    def __contains__(self, key) -> bool:
        return key in self._d


_native_cache = _LruCache(NATIVE_CACHE_MAX)


def native_plan(kind: int, n: int, inverse: bool, device: int, hop: int = 0, flags: int = 0, n2: int = 0,
                _factory=None) -> NativePlan:
    """The cached native plan for this key, created on first use.  The returned object keeps the
    plan alive for as long as the caller holds it."""
    key = (kind, n, bool(inverse), device, hop, flags, n2)
    with _lock:
        p = _native_cache.get(key)
        if p is None:
            p = (_factory or NativePlan)(kind, n, inverse, device, hop, flags, n2)
            _native_cache.put(key, p)
    return p
