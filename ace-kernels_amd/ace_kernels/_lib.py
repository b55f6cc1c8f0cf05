"""ctypes binding of ``libace_hip.so`` (the C-ABI declared in ``include/ace_hip.h``).

The library is the only implementation of the loss in this package: if it is
missing or fails to load, every call raises -- there is no fallback path.
Build it with ``python ace-kernels_amd/build.py``.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache
from pathlib import Path

LIB_PATH = Path(os.environ.get("ACE_HIP_LIB", Path(__file__).resolve().with_name("libace_hip.so")))

ABI_VERSION = 9

# enums of include/ace_hip.h
F32, BF16, F16, F64 = 0, 1, 2, 3
TARGET_LABELS_I64, TARGET_ONEHOT_F32, TARGET_ONEHOT_F64 = 0, 1, 2
HARD, SOFT = 0, 1
ACT_NONE, ACT_SOFTMAX, ACT_SIGMOID = 0, 1, 2
RED_MEAN, RED_SUM, RED_NONE = 0, 1, 2

# every symbol include/ace_hip.h declares
EXPORTS = (
    "ace_abi_version",
    "ace_error_string",
    "ace_workspace_bytes",
    "ace_workspace_reset_bytes",
    "ace_forward",
    "ace_backward",
    "ace_set_launch_events",
    "ace_set_test_hooks",
    "ace_read_bytes_scratch",
    "ace_read_bytes",
    "ace_probabilities",
    "ace_set_timeline",
    "ace_workspace_bytes_levels",
    "ace_forward_levels",
    "ace_backward_levels",
    "ace_forward_noalloc",
    "ace_forward_f64",
    "ace_backward_f64",
)

# ace_forward_noalloc's scratch (ACE_NOALLOC_SCRATCH_BYTES) and its error code
NOALLOC_SCRATCH_BYTES = 1 << 20
EINVAL, EUNSUPPORTED, ESCRATCH = 1, 2, 4

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t


class AceFwdLevel(ctypes.Structure):
    """struct AceFwdLevel of include/ace_hip.h."""

    _fields_ = [("x", _p), ("target", _p), ("voxels", _i64), ("coef", _p), ("diff", _p),
                ("jac", _p), ("per_class", _p), ("loss", _p)]


class AceBwdLevel(ctypes.Structure):
    """struct AceBwdLevel of include/ace_hip.h."""

    _fields_ = [("x", _p), ("target", _p), ("voxels", _i64), ("coef", _p), ("diff", _p),
                ("jac", _p), ("grad_output", _p), ("dx", _p)]


class AceLibraryError(RuntimeError):
    """libace_hip.so is missing, stale, or returned an error code."""


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise AceLibraryError(
            f"{LIB_PATH} not found: the HIP extension is not built "
            "(run `python ace-kernels_amd/build.py`)"
        )
    # the process's HIP runtime is torch's; load it first so the library binds to it
    import torch  # noqa: F401

    handle = ctypes.CDLL(str(LIB_PATH))
    handle.ace_abi_version.restype = _i
    handle.ace_abi_version.argtypes = []
    handle.ace_error_string.restype = ctypes.c_char_p
    handle.ace_error_string.argtypes = [_i]
    for name in ("ace_workspace_bytes", "ace_workspace_reset_bytes"):
        fn = getattr(handle, name)
        fn.restype = _sz
        fn.argtypes = [_i64, _i64, _i64, _i, _i, _i, _i, _i]
    handle.ace_forward.restype = _i
    handle.ace_forward.argtypes = [
        _p, _i, _p, _i,            # x, dtype, target, kind
        _i64, _i64, _i64,          # B, C, N
        _i, _i, _i,                # K, binning, activation
        _i, _i, _i, _i,            # include_bg, ignore_empty, reduction, right
        _f, _p, _p, _p,            # empty_weight, class_weight, bin_table, centre_table
        _p, _sz,                   # workspace, bytes
        _p, _p, _p, _p, _p, _p,    # coef, diff, jac, per_class, loss, stats
        _p,                        # stream
    ]
    handle.ace_forward_noalloc.restype = _i
    handle.ace_forward_noalloc.argtypes = [
        _p, _i, _p, _i,            # x, dtype, target, kind
        _i64, _i64, _i64,          # B, C, N
        _i, _i, _i,                # K, binning, activation
        _i, _i, _i, _i,            # include_bg, ignore_empty, reduction, right
        _f, _p, _p, _p,            # empty_weight, class_weight, bin_table, centre_table
        _p, _p, _p, _p, _p, _p,    # coef, diff, jac, per_class, loss, stats
        _p,                        # stream
    ]
    _d = ctypes.c_double
    handle.ace_forward_f64.restype = _i
    handle.ace_forward_f64.argtypes = [
        _p, _p, _i,                # x, target, kind
        _i64, _i64, _i64,          # B, C, N
        _i, _i, _i,                # K, binning, activation
        _i, _i, _i, _i,            # include_bg, ignore_empty, reduction, right
        _d, _p, _p, _p,            # empty_weight, class_weight, bin_table, centre_table
        _p, _sz,                   # workspace, bytes
        _p, _p, _p, _p, _p, _p,    # coef, diff, jac, per_class, loss, stats
        _p,                        # stream
    ]
    handle.ace_backward_f64.restype = _i
    handle.ace_backward_f64.argtypes = [
        _p, _p, _i,
        _i64, _i64, _i64,
        _i, _i, _i, _i, _i,        # K, binning, activation, include_bg, right
        _p, _p,                    # bin_table, centre_table
        _p, _p, _p,                # coef, diff, jac
        _p, _i,                    # grad_output, per_class
        _p, _p,                    # dx, stream
    ]
    handle.ace_backward.restype = _i
    handle.ace_backward.argtypes = [
        _p, _i, _p, _i,
        _i64, _i64, _i64,
        _i, _i, _i, _i, _i,        # K, binning, activation, include_bg, right
        _p, _p,                    # bin_table, centre_table
        _p, _p, _p,                # coef, diff, jac
        _p, _i,                    # grad_output, per_class
        _p, _p,                    # dx, stream
    ]
    handle.ace_workspace_bytes_levels.restype = _sz
    handle.ace_workspace_bytes_levels.argtypes = [_i, ctypes.POINTER(_i64), _i64, _i64, _i, _i, _i, _i]
    handle.ace_forward_levels.restype = _i
    handle.ace_forward_levels.argtypes = [
        _i, ctypes.POINTER(AceFwdLevel), _i,   # levels, per-level pointers, dtype
        _i64, _i64, _i, _i, _i,                # B, C, K, binning, include_bg
        _i, _i, _i, _f,                        # ignore_empty, reduction, right, empty_weight
        _p, _p, _p,                            # class_weight, bin_table, centre_table
        _p, _sz, _p,                           # workspace, bytes, stream
    ]
    handle.ace_backward_levels.restype = _i
    handle.ace_backward_levels.argtypes = [
        _i, ctypes.POINTER(AceBwdLevel), _i,
        _i64, _i64, _i, _i, _i, _i, _i,        # B, C, K, binning, include_bg, right, per_class
        _p, _p, _p,                            # bin_table, centre_table, stream
    ]
    handle.ace_set_launch_events.restype = _i
    handle.ace_set_launch_events.argtypes = [_p, _p]
    handle.ace_set_test_hooks.restype = _i
    handle.ace_set_test_hooks.argtypes = [_i, _i]
    handle.ace_read_bytes_scratch.restype = _sz
    handle.ace_read_bytes_scratch.argtypes = []
    handle.ace_read_bytes.restype = _i
    handle.ace_read_bytes.argtypes = [_p, _sz, _p, _sz, _p, _p]
    handle.ace_probabilities.restype = _i
    handle.ace_probabilities.argtypes = [_p, _i, _i64, _i64, _i64, _i, _p, _p]
    handle.ace_set_timeline.restype = _i
    handle.ace_set_timeline.argtypes = [_p]
    version = handle.ace_abi_version()
    if version != ABI_VERSION:
        raise AceLibraryError(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}: rebuild it")
    return handle


@lru_cache(maxsize=1)
def autograd():
    """``ace_kernels._ace_autograd`` (the loss call and its backward node in
    C++, ``csrc/ace_autograd.cpp``), wired to this process's
    ``libace_hip.so``: it calls the entry points of the library ``lib()``
    loaded.  Raises ``AceLibraryError`` when the module is not built."""
    handle = lib()
    try:
        from ace_kernels import _ace_autograd as mod
    except ImportError as e:
        raise AceLibraryError(
            f"ace_kernels/_ace_autograd.so failed to load ({e}): "
            "run `python ace-kernels_amd/build.py`"
        ) from e

    def addr(fn) -> int:
        return int(ctypes.cast(fn, ctypes.c_void_p).value)

    mod.set_entry_points(addr(handle.ace_forward), addr(handle.ace_backward),
                         addr(handle.ace_forward_levels), addr(handle.ace_backward_levels),
                         addr(handle.ace_error_string))
    return mod


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().ace_error_string(rc).decode()
        raise AceLibraryError(f"{what} failed with code {rc}: {msg}")
