"""ctypes binding of ``libkda_hip.so`` (C ABI declared in include/kda_hip.h).

The library is loaded lazily on first use and never replaced by anything else:
if it is missing or was built for another ABI version, every call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkda_hip.so"
ABI_VERSION = 14

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

STATUS_OK = 0
STATUS_BAD_SHAPE = 2
STATUS_UNSUPPORTED = 4
STATUS_TOO_LARGE = 7

BWD_SCRATCH_BYTES = 64 << 20    # KDA_BWD_SCRATCH_BYTES: the static buffer of kda_chunkwise_bwd_noalloc

_i64x3 = ctypes.c_int64 * 3


class KdaFwdArgs(ctypes.Structure):
    """Mirror of ``struct kda_fwd_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64),
        ("K", ctypes.c_int64), ("V", ctypes.c_int64),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("g", ctypes.c_void_p), ("beta", ctypes.c_void_p),
        ("q_stride", _i64x3), ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("g_stride", _i64x3), ("beta_stride", _i64x3),
        ("qkv_dtype", ctypes.c_int32), ("g_dtype", ctypes.c_int32), ("beta_dtype", ctypes.c_int32),
        ("state_in", ctypes.c_void_p), ("state_in_dtype", ctypes.c_int32),
        ("state_out", ctypes.c_void_p), ("state_out_dtype", ctypes.c_int32),
        ("o", ctypes.c_void_p),
        ("scale", ctypes.c_float),
        ("clamp_fp16_out", ctypes.c_int32),
        ("chunk_size", ctypes.c_int64),
    ]


class KdaGateArgs(ctypes.Structure):
    """Mirror of ``struct kda_gate_args`` (include/kda_hip.h)."""

    _fields_ = [("a_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p)]


class KdaOutEpilogue(ctypes.Structure):
    """Mirror of ``struct kda_out_epilogue`` (include/kda_hip.h)."""

    _fields_ = [("gate", ctypes.c_void_p), ("gate_stride", ctypes.c_int64 * 2),
                ("weight", ctypes.c_void_p), ("eps", ctypes.c_float)]


class KdaBwdArgs(ctypes.Structure):
    """Mirror of ``struct kda_bwd_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64),
        ("K", ctypes.c_int64), ("V", ctypes.c_int64),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("g", ctypes.c_void_p), ("beta", ctypes.c_void_p), ("ckpt", ctypes.c_void_p),
        ("d_o", ctypes.c_void_p), ("d_state_out", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dg", ctypes.c_void_p),
        ("dbeta", ctypes.c_void_p), ("dv", ctypes.c_void_p), ("d_state_in", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("scale", ctypes.c_float), ("io_dtype", ctypes.c_int32),
    ]


_ptr3 = ctypes.c_void_p * 3


class KdaPrepArgs(ctypes.Structure):
    """Mirror of ``struct kda_prep_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64),
        ("K", ctypes.c_int64), ("V", ctypes.c_int64), ("conv_size", ctypes.c_int64),
        ("x", _ptr3), ("x_stride", (ctypes.c_int64 * 2) * 3),
        ("conv_w", _ptr3), ("conv_b", _ptr3), ("w_dtype", ctypes.c_int32),
        ("hist_in", _ptr3), ("hist_out", _ptr3),
        ("gk", ctypes.c_void_p), ("gk_stride", ctypes.c_int64 * 2),
        ("a_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p), ("p_dtype", ctypes.c_int32),
        ("beta_logit", ctypes.c_void_p), ("beta_stride", ctypes.c_int64 * 2),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("g", ctypes.c_void_p), ("beta", ctypes.c_void_p),
        ("l2_eps", ctypes.c_float), ("x_dtype", ctypes.c_int32),
    ]


class KdaOutputArgs(ctypes.Structure):
    """Mirror of ``struct kda_output_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64), ("V", ctypes.c_int64),
        ("o", ctypes.c_void_p), ("o_stride", ctypes.c_int64 * 3),
        ("gate", ctypes.c_void_p), ("gate_stride", ctypes.c_int64 * 2),
        ("weight", ctypes.c_void_p), ("w_dtype", ctypes.c_int32),
        ("y", ctypes.c_void_p), ("eps", ctypes.c_float), ("x_dtype", ctypes.c_int32),
    ]


class KdaPrepBwdArgs(ctypes.Structure):
    """Mirror of ``struct kda_prep_bwd_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64),
        ("K", ctypes.c_int64), ("V", ctypes.c_int64), ("conv_size", ctypes.c_int64),
        ("x", _ptr3), ("x_stride", (ctypes.c_int64 * 2) * 3),
        ("conv_w", _ptr3), ("conv_b", _ptr3), ("w_dtype", ctypes.c_int32),
        ("dy", _ptr3), ("dx", _ptr3), ("dw", _ptr3), ("db", _ptr3),
        ("gk", ctypes.c_void_p), ("gk_stride", ctypes.c_int64 * 2),
        ("a_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p), ("p_dtype", ctypes.c_int32),
        ("beta_logit", ctypes.c_void_p), ("beta_stride", ctypes.c_int64 * 2),
        ("dg", ctypes.c_void_p), ("dbeta", ctypes.c_void_p),
        ("dgk", ctypes.c_void_p), ("dbeta_logit", ctypes.c_void_p),
        ("da_log", ctypes.c_void_p), ("ddt_bias", ctypes.c_void_p),
        ("l2_eps", ctypes.c_float), ("x_dtype", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
    ]


class KdaOutputBwdArgs(ctypes.Structure):
    """Mirror of ``struct kda_output_bwd_args`` (include/kda_hip.h)."""

    _fields_ = [
        ("B", ctypes.c_int64), ("T", ctypes.c_int64), ("H", ctypes.c_int64), ("V", ctypes.c_int64),
        ("o", ctypes.c_void_p), ("o_stride", ctypes.c_int64 * 3),
        ("gate", ctypes.c_void_p), ("gate_stride", ctypes.c_int64 * 2),
        ("weight", ctypes.c_void_p), ("w_dtype", ctypes.c_int32),
        ("dy", ctypes.c_void_p), ("d_o", ctypes.c_void_p), ("dgate", ctypes.c_void_p),
        ("dweight", ctypes.c_void_p), ("eps", ctypes.c_float), ("x_dtype", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
    ]


EXPORTED_SYMBOLS = ("kda_chunkwise_fwd", "kda_recurrent_fwd", "kda_chunkwise_fwd_ckpt",
                    "kda_chunkwise_gated_fwd", "kda_recurrent_gated_fwd", "kda_chunkwise_fused_fwd",
                    "kda_chunkwise_long_fwd", "kda_chunkwise_long_workspace_size",
                    "kda_chunkwise_bwd",
                    "kda_chunkwise_bwd_workspace_size", "kda_chunkwise_bwd_noalloc",
                    "kda_prep_fwd", "kda_output_fwd", "kda_prep_bwd", "kda_prep_bwd_workspace_size",
                    "kda_output_bwd", "kda_output_bwd_workspace_size", "kda_status_str", "kda_abi_version")

_lib = None
_lock = threading.Lock()


class NativeLibraryError(RuntimeError):
    """libkda_hip.so is missing, unloadable or of the wrong ABI version."""


def load() -> ctypes.CDLL:
    """Load (once) and return the native library, raising if it is unusable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"{LIB_PATH} not found: build it with __graft_entry__.build() "
                "(hipcc, gfx950) before using the HIP KDA kernels")
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name in EXPORTED_SYMBOLS:
            if not hasattr(lib, name):
                raise NativeLibraryError(f"{LIB_PATH} does not export {name}")
        lib.kda_chunkwise_fwd.argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.c_void_p]
        lib.kda_chunkwise_fwd.restype = ctypes.c_int
        lib.kda_recurrent_fwd.argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.c_void_p]
        lib.kda_recurrent_fwd.restype = ctypes.c_int
        for name in ("kda_chunkwise_gated_fwd", "kda_recurrent_gated_fwd"):
            getattr(lib, name).argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.POINTER(KdaGateArgs), ctypes.c_void_p]
            getattr(lib, name).restype = ctypes.c_int
        lib.kda_chunkwise_long_fwd.argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.c_int64, ctypes.c_void_p,
                                               ctypes.c_void_p]
        lib.kda_chunkwise_long_fwd.restype = ctypes.c_int
        lib.kda_chunkwise_long_workspace_size.argtypes = [ctypes.c_int64] * 6
        lib.kda_chunkwise_long_workspace_size.restype = ctypes.c_size_t
        lib.kda_chunkwise_fused_fwd.argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.POINTER(KdaGateArgs),
                                                ctypes.POINTER(KdaOutEpilogue), ctypes.c_void_p]
        lib.kda_chunkwise_fused_fwd.restype = ctypes.c_int
        lib.kda_chunkwise_fwd_ckpt.argtypes = [ctypes.POINTER(KdaFwdArgs), ctypes.c_void_p, ctypes.c_void_p]
        lib.kda_chunkwise_fwd_ckpt.restype = ctypes.c_int
        lib.kda_chunkwise_bwd.argtypes = [ctypes.POINTER(KdaBwdArgs), ctypes.c_void_p]
        lib.kda_chunkwise_bwd.restype = ctypes.c_int
        lib.kda_chunkwise_bwd_noalloc.argtypes = [ctypes.POINTER(KdaBwdArgs), ctypes.c_void_p]
        lib.kda_chunkwise_bwd_noalloc.restype = ctypes.c_int
        lib.kda_chunkwise_bwd_workspace_size.argtypes = [ctypes.c_int64] * 5
        lib.kda_chunkwise_bwd_workspace_size.restype = ctypes.c_size_t
        lib.kda_prep_fwd.argtypes = [ctypes.POINTER(KdaPrepArgs), ctypes.c_void_p]
        lib.kda_prep_fwd.restype = ctypes.c_int
        lib.kda_output_fwd.argtypes = [ctypes.POINTER(KdaOutputArgs), ctypes.c_void_p]
        lib.kda_output_fwd.restype = ctypes.c_int
        lib.kda_prep_bwd.argtypes = [ctypes.POINTER(KdaPrepBwdArgs), ctypes.c_void_p]
        lib.kda_prep_bwd.restype = ctypes.c_int
        lib.kda_prep_bwd_workspace_size.argtypes = [ctypes.c_int64] * 6
        lib.kda_prep_bwd_workspace_size.restype = ctypes.c_size_t
        lib.kda_output_bwd.argtypes = [ctypes.POINTER(KdaOutputBwdArgs), ctypes.c_void_p]
        lib.kda_output_bwd.restype = ctypes.c_int
        lib.kda_output_bwd_workspace_size.argtypes = [ctypes.c_int64] * 4
        lib.kda_output_bwd_workspace_size.restype = ctypes.c_size_t
        lib.kda_status_str.argtypes = [ctypes.c_int]
        lib.kda_status_str.restype = ctypes.c_char_p
        lib.kda_abi_version.argtypes = []
        lib.kda_abi_version.restype = ctypes.c_int
        version = lib.kda_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(
                f"{LIB_PATH} has ABI version {version}, this wrapper expects {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def status_str(code: int) -> str:
    return load().kda_status_str(int(code)).decode()
