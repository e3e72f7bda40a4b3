"""ctypes binding of libkfhip.so (include/kfhip.h).

The library is loaded once; a missing library is an error, never a silent
fallback: every op of this package runs on the HIP kernels or raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_char_p, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent.parent / "libkfhip.so"

# status codes / enums of include/kfhip.h
KF_OK = 0
KF_F32, KF_BF16 = 0, 1
KF_I8, KF_I16 = 2, 3  # lookup-table element types
KF_KIND_CHEB, KF_KIND_BSPLINE, KF_KIND_RATIONAL = 0, 1, 2
KF_MAP_IDENTITY, KF_MAP_TANH, KF_MAP_TANH_SQ = 0, 1, 2
KF_OP_F, KF_OP_G, KF_OP_P = 0, 1, 2
KF_OP_F_BASE, KF_OP_P_BASE, KF_OP_G_BASE, KF_OP_G_BIAS = 3, 4, 5, 6
KF_MAX_K, KF_MAX_NT = 16, 24
KF_EWORKSPACE = -2
KF_NOALLOC_SCRATCH_BYTES = 64 << 20

EXPORTS = (
    "kf_workspace_bytes",
    "kf_F",
    "kf_F_noalloc",
    "kf_G",
    "kf_P",
    "kf_features",
    "kf_edge_derivative",
    "kf_bspline_interval",
    "kf_rational_workspace_bytes",
    "kf_rational_param_grad",
    "kf_rational_bwd_workspace_bytes",
    "kf_rational_bwd",
    "kf_column_sums_workspace_bytes",
    "kf_column_sums",
    "kf_silu_taylor",
    "kf_probe_mfma",
    "kf_lut_forward",
    "kf_base_fused",
    "kf_F_base",
    "kf_F_bias",
    "kf_G_bias",
    "kf_P_base",
    "kf_G_base",
    "kf_last_error",
    "kf_version",
)


class KfBasis(ctypes.Structure):
    _fields_ = [
        ("kind", c_int32),
        ("size", c_int32),
        ("order", c_int32),
        ("n_t", c_int32),
        ("input_map", c_int32),
        ("spline_k", c_int32),
        ("n_knots", c_int32),
        ("num_deg", c_int32),
        ("den_deg", c_int32),
        ("group_size", c_int32),
        ("fold", c_void_p),
        ("knots", c_void_p),
        ("knots_cmp", c_void_p),
        ("num", c_void_p),
        ("den", c_void_p),
        ("knots_uniform", c_void_p),
    ]


_lock = threading.Lock()
_lib = None


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """The loaded library (raises if it is missing or incomplete)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(f"{p} is missing: build it with `python -m kanforge_amd.build` (needs hipcc)")
        lib = ctypes.CDLL(str(p))
        for name in EXPORTS:
            if not hasattr(lib, name):
                raise RuntimeError(f"{p} does not export {name}")
        P = ctypes.POINTER(KfBasis)
        lib.kf_workspace_bytes.argtypes = [c_int, P, c_int, c_int64, c_int64, c_int64]
        lib.kf_workspace_bytes.restype = c_size_t
        lib.kf_F.argtypes = [P, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        lib.kf_F_noalloc.argtypes = [P, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        lib.kf_G.argtypes = [P, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        lib.kf_P.argtypes = [P, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        lib.kf_features.argtypes = [P, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p]
        lib.kf_edge_derivative.argtypes = [P, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        lib.kf_bspline_interval.argtypes = [c_int64, c_int64, c_void_p, c_void_p, c_int32, c_void_p, c_void_p]
        lib.kf_rational_workspace_bytes.argtypes = [P, c_int64, c_int64]
        lib.kf_rational_workspace_bytes.restype = c_size_t
        lib.kf_rational_param_grad.argtypes = [P, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        for name in ("kf_F", "kf_F_noalloc", "kf_G", "kf_P", "kf_features", "kf_edge_derivative", "kf_bspline_interval", "kf_rational_param_grad"):
            getattr(lib, name).restype = c_int
        lib.kf_probe_mfma.argtypes = [c_int, c_int, c_int, c_void_p, c_void_p]
        lib.kf_rational_bwd_workspace_bytes.argtypes = [P, c_int, c_int64, c_int64, c_int64]
        lib.kf_rational_bwd_workspace_bytes.restype = c_size_t
        lib.kf_rational_bwd.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 7 + [c_void_p, c_size_t, c_void_p]
        lib.kf_rational_bwd.restype = c_int
        lib.kf_column_sums_workspace_bytes.argtypes = [c_int64, c_int64]
        lib.kf_column_sums_workspace_bytes.restype = c_size_t
        lib.kf_column_sums.argtypes = [c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        lib.kf_column_sums.restype = c_int
        lib.kf_silu_taylor.argtypes = [c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6
        lib.kf_silu_taylor.restype = c_int
        lib.kf_lut_forward.argtypes = [c_int, c_int64, c_int64, c_int64, c_int64] + [c_void_p] * 10
        lib.kf_probe_mfma.restype = c_int
        lib.kf_lut_forward.restype = c_int
        lib.kf_base_fused.argtypes = [c_int, P, c_int, c_int64, c_int64, c_int64]
        lib.kf_F_base.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6 + [c_size_t, c_void_p]
        lib.kf_P_base.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6 + [c_size_t, c_void_p]
        lib.kf_G_base.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6 + [c_size_t, c_void_p]
        lib.kf_F_bias.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6 + [c_size_t, c_void_p]
        lib.kf_G_bias.argtypes = [P, c_int, c_int64, c_int64, c_int64] + [c_void_p] * 6 + [c_size_t, c_void_p]
        for name in ("kf_base_fused", "kf_F_base", "kf_P_base", "kf_G_base", "kf_F_bias", "kf_G_bias"):
            getattr(lib, name).restype = c_int
        lib.kf_last_error.argtypes = []
        lib.kf_last_error.restype = c_char_p
        lib.kf_version.argtypes = []
        lib.kf_version.restype = c_char_p
        if path is None:
            _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError with the library's message when rc != 0."""
    if rc != KF_OK:
        msg = load().kf_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
