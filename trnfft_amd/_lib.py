"""ctypes binding of libtrnfft_amd.so (the C ABI declared in include/trnfft_amd.h).

The library is built in-tree by ``trnfft_amd.csrc.build`` (or ``__graft_entry__.build()``).
Nothing here falls back to another implementation: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtrnfft_amd.so")

TFA_OK = 0
TFA_ERR_INVALID = -1
TFA_ERR_UNSUPPORTED = -2
TFA_ERR_HIP = -3

KIND_C2C = 0
KIND_BLUESTEIN = 1
KIND_DFT_GEMM = 2
KIND_STFT = 3
KIND_FFT2 = 4
KIND_REAL = 5

# operand ops of tfa_complex_gemm_ex
OP_N, OP_T, OP_C, OP_R = 0, 1, 2, 3

STFT_CENTER = 1
STFT_NORMALIZED = 2
STFT_ONESIDED = 4
STFT_FRAMES_MAJOR = 8

# every symbol include/trnfft_amd.h declares
EXPORTS = (
    "tfa_plan_create",
    "tfa_plan_destroy",
    "tfa_plan_workspace_size",
    "tfa_plan_padded_n",
    "tfa_execute",
    "tfa_execute_noalloc",
    "tfa_execute_strided",
    "tfa_strided_workspace_size",
    "tfa_execute_strided_ws",
    "tfa_stft_frames",
    "tfa_stft_execute",
    "tfa_istft_length",
    "tfa_istft_execute",
    "tfa_stft_backward_execute",
    "tfa_complex_gemm",
    "tfa_complex_gemm_ex",
    "tfa_complex_gemm_batched",
    "tfa_last_error",
    "tfa_abi_version",
)


class PlanDesc(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("inverse", ctypes.c_int32),
        ("n", ctypes.c_int64),
        ("hop", ctypes.c_int64),
        ("flags", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("n2", ctypes.c_int64),
    ]


_lib = None
_lock = threading.Lock()
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def _declare(lib: ctypes.CDLL) -> None:
    lib.tfa_plan_create.argtypes = [ctypes.POINTER(_vp), ctypes.POINTER(PlanDesc)]
    lib.tfa_plan_create.restype = ctypes.c_int
    lib.tfa_plan_destroy.argtypes = [_vp]
    lib.tfa_plan_destroy.restype = None
    lib.tfa_plan_workspace_size.argtypes = [_vp, _i64, ctypes.POINTER(ctypes.c_size_t)]
    lib.tfa_plan_workspace_size.restype = ctypes.c_int
    lib.tfa_plan_padded_n.argtypes = [_vp]
    lib.tfa_plan_padded_n.restype = _i64
    lib.tfa_execute.argtypes = [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.tfa_execute.restype = ctypes.c_int
    lib.tfa_execute_strided.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp]
    lib.tfa_execute_strided.restype = ctypes.c_int
    lib.tfa_strided_workspace_size.argtypes = [_vp, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)]
    lib.tfa_strided_workspace_size.restype = ctypes.c_int
    lib.tfa_execute_strided_ws.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.tfa_execute_strided_ws.restype = ctypes.c_int
    lib.tfa_stft_frames.argtypes = [_vp, _i64, ctypes.POINTER(_i64)]
    lib.tfa_stft_frames.restype = ctypes.c_int
    lib.tfa_stft_execute.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp]
    lib.tfa_stft_execute.restype = ctypes.c_int
    lib.tfa_istft_length.argtypes = [_vp, _i64, _i64, ctypes.POINTER(_i64)]
    lib.tfa_istft_length.restype = ctypes.c_int
    lib.tfa_istft_execute.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _vp]
    lib.tfa_istft_execute.restype = ctypes.c_int
    lib.tfa_stft_backward_execute.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _vp]
    lib.tfa_stft_backward_execute.restype = ctypes.c_int
    lib.tfa_complex_gemm.argtypes = [_i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _vp]
    lib.tfa_complex_gemm.restype = ctypes.c_int
    lib.tfa_complex_gemm_ex.argtypes = [_i64, _i64, _i64, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i32, ctypes.c_float,
                                        _vp, _vp, _vp, _vp, _i64, _vp]
    lib.tfa_complex_gemm_ex.restype = ctypes.c_int
    lib.tfa_complex_gemm_batched.argtypes = [_i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i32, _vp, _vp, _i64, _i64,
                                             _i32, ctypes.c_float, _vp, _vp, _vp, _vp, _i64, _i64, _vp]
    lib.tfa_complex_gemm_batched.restype = ctypes.c_int
    lib.tfa_execute_noalloc.argtypes = [_vp, _i64, _vp, _vp, _vp, _vp, _vp]
    lib.tfa_execute_noalloc.restype = ctypes.c_int
    lib.tfa_last_error.argtypes = []
    lib.tfa_last_error.restype = ctypes.c_char_p
    lib.tfa_abi_version.argtypes = []
    lib.tfa_abi_version.restype = _i32


def library_present() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library; raises RuntimeError when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"trnfft_amd native library not built ({LIB_PATH}); run "
                    "`python -m trnfft_amd.csrc.build` (hipcc, gfx950)"
                )
            handle = ctypes.CDLL(LIB_PATH)
            _declare(handle)
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Map a C status to the exception the reference raises for the same condition."""
    if rc == TFA_OK:
        return
    msg = lib().tfa_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if rc == TFA_ERR_INVALID:
        raise ValueError(text)
    if rc == TFA_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)
