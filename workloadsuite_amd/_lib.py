"""ctypes binding of libssd.so (include/ssd.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already loaded (both resolve the SONAME libamdhip64.so.7): device
pointers and streams are then shared with torch's allocator and streams.
There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- must precede the CDLL, see module docstring

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libssd.so")

SSD_ABI_VERSION = 8
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
STATE_SPLIT_BF16, STATE_SPLIT_F16 = 3, 4  # f32 states as 16-bit (hi, lo) pairs
STATE_F16S = 5  # f32 states as f16 rows with a power-of-two scale per row
STATE_F16S_LOCAL = 6  # local states as f16 rows, a scale per row and 16-column tile packed into the item's first rows

# Every symbol include/ssd.h declares.
EXPORTS = (
    "ssd_abi_version",
    "ssd_strerror",
    "ssd_check_dims",
    "ssd_workspace_bytes",
    "ssd_chunk_prep_bytes",
    "ssd_chunk_prep",
    "ssd_chunk_cumsum",
    "ssd_chunk_state",
    "ssd_state_passing",
    "ssd_chunk_state_passing",
    "ssd_chunk_scan",
    "ssd_forward_chunk",
    "ssd_forward",
    "ssd_decode_step",
    "ssd_layer_prep",
    "ssd_layer_workspace_bytes",
    "ssd_layer_forward",
    "ssd_forward_noalloc",
)


class SSDDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in
                ("batch", "seqlen", "nheads", "headdim", "dstate", "ngroups", "chunk")]


class SSDEpilogue(ctypes.Structure):
    _fields_ = [("D", ctypes.c_void_p), ("z", ctypes.c_void_p), ("z_strides", ctypes.c_int64 * 4)]


class SSDLayerParams(ctypes.Structure):
    _fields_ = [("conv_kernel", ctypes.c_int64), ("conv_w", ctypes.c_void_p), ("conv_b", ctypes.c_void_p),
                ("dt_bias", ctypes.c_void_p), ("A_log", ctypes.c_void_p), ("D", ctypes.c_void_p)]


_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_dims_p = ctypes.POINTER(SSDDims)
_epi_p = ctypes.POINTER(SSDEpilogue)
_prm_p = ctypes.POINTER(SSDLayerParams)
_int = ctypes.c_int

_SIGNATURES = {
    "ssd_abi_version": (_int, []),
    "ssd_strerror": (ctypes.c_char_p, [_int]),
    "ssd_check_dims": (_int, [_dims_p, _int]),
    "ssd_workspace_bytes": (ctypes.c_size_t, [_dims_p, _int]),
    "ssd_chunk_cumsum": (_int, [_dims_p, _vp, _i64p, _vp, _vp, _vp]),
    "ssd_chunk_prep_bytes": (ctypes.c_size_t, [_dims_p]),
    "ssd_chunk_prep": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, ctypes.c_size_t, _vp]),
    "ssd_chunk_state": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _int, _vp, _vp]),
    "ssd_state_passing": (_int, [_dims_p, _vp, _int, _vp, _vp, _vp, _vp, _vp]),
    "ssd_chunk_state_passing": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _vp, _vp,
                                       _vp, _int, _vp, _vp, _vp]),
    "ssd_chunk_scan": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                              _vp, _vp, _int, _vp, _vp, _i64p, _vp, _epi_p, _vp]),
    "ssd_forward_chunk": (ctypes.c_int64, [_dims_p, _int, _int]),
    "ssd_forward": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                           _vp, _vp, _i64p, _vp, _vp, ctypes.c_size_t, _int, _vp]),
    "ssd_decode_step": (_int, [_dims_p, _int, _vp, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _i64p,
                                _vp, _i64p, _epi_p, _vp]),
    "ssd_layer_prep": (_int, [_dims_p, _int, _prm_p, _vp, _i64p, _vp, _i64p, _vp, _vp, _vp, _vp, _vp]),
    "ssd_layer_workspace_bytes": (ctypes.c_size_t, [_dims_p, _int]),
    "ssd_layer_forward": (_int, [_dims_p, _int, _prm_p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                 _vp, _i64p, _vp, _i64p, _vp, ctypes.c_size_t, _vp]),
    "ssd_forward_noalloc": (_int, [_dims_p, _int, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
                                   _vp, _vp, _i64p, _vp, _int, _vp]),
}

_LIB = None


class SSDError(RuntimeError):
    """A nonzero status from libssd (negative: invalid argument; positive: HIP error)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libssd status {status}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load libssd.so once; raises if it is missing or its ABI does not match."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m workloadsuite_amd.build` "
                "(there is no CPU fallback for the SSD forward)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.ssd_abi_version() != SSD_ABI_VERSION:
            raise RuntimeError(f"libssd ABI {lib.ssd_abi_version()} != expected {SSD_ABI_VERSION}")
        _LIB = lib
    return _LIB


def check(status: int) -> None:
    if status != 0:
        raise SSDError(status, load().ssd_strerror(status).decode())


def dims(batch, seqlen, nheads, headdim, dstate, ngroups, chunk) -> SSDDims:
    return SSDDims(batch, seqlen, nheads, headdim, dstate, ngroups, chunk)


def strides(t) -> ctypes.Array:
    s = t.stride()
    return (ctypes.c_int64 * len(s))(*s)
