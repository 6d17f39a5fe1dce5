"""ctypes binding of libpasa_amd.so (the C ABI declared in include/pasa.h).

The library is built in-tree by ``pasa_amd.build``.  There is no fallback: if
the shared object is missing or fails to load, every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("PASA_AMD_LIB", Path(__file__).resolve().parent / "libpasa_amd.so"))

# pasa_dtype_t
DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

# pasa_status_t
STATUS = {
    0: "PASA_OK",
    -1: "PASA_ERR_NULL_POINTER",
    -2: "PASA_ERR_BAD_SHAPE",
    -3: "PASA_ERR_HEAD_DIM",
    -4: "PASA_ERR_BLOCK_SIZE",
    -5: "PASA_ERR_NUM_SELECTED",
    -6: "PASA_ERR_OVERFLOW",
    -7: "PASA_ERR_DTYPE",
    -8: "PASA_ERR_WORKSPACE",
    -9: "PASA_ERR_BAD_ARG",
    -10: "PASA_ERR_TEXT_SEGMENT",
    -11: "PASA_ERR_LAUNCH",
    -12: "PASA_ERR_GROUP_SIZE",
    -13: "PASA_ERR_TOO_MANY_BLOCKS",
}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_dbl = ctypes.c_double
_sz = ctypes.c_size_t

class Placement(ctypes.Structure):
    """pasa_placement_t: the token-major view of frame-major slices."""
    _fields_ = [("num_frame", ctypes.c_int64), ("frame_size", ctypes.c_int64),
                ("head_is_temporal", ctypes.c_void_p), ("heads", ctypes.c_int64)]


_pl = ctypes.POINTER(Placement)

# name -> (restype, argtypes); mirrors include/pasa.h exactly.
SIGNATURES = {
    "pasa_abi_version": (_int, []),
    "pasa_status_string": (ctypes.c_char_p, [_int]),
    "pasa_last_error": (ctypes.c_char_p, []),
    "pasa_num_selected": (_i64, [_dbl, _i64]),
    "pasa_permute": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _int,
                            _vp, _int, _vp]),
    "pasa_block_stats": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                _i64, _int, _vp]),
    "pasa_block_stats_ws": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _int, _vp, _sz, _vp]),
    "pasa_block_stats_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "pasa_select": (_int, [_vp, _vp, _vp, _vp, _dbl, _dbl, _int, _vp, _vp, _vp, _vp, _sz, _i64, _i64,
                           _i64, _vp]),
    "pasa_select_workspace_bytes": (_sz, [_i64, _i64]),
    "pasa_select_from_scores": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp]),
    "pasa_sparse_attn": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _dbl, _i64, _i64, _i64,
                                _i64, _i64, _i64, _i64, _i64, _int, _int, _vp, _sz, _vp]),
    "pasa_sparse_attn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "pasa_sparse_attn_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _dbl, _i64, _i64, _i64,
                                        _i64, _i64, _i64, _i64, _i64, _int, _int, _vp]),
    "pasa_pack_phase2": (_int, [_vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "pasa_sparse_attn_packed": (_int, [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _dbl, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _i64, _i64, _int, _int, _vp]),
    "pasa_block_stats_placed": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _pl, _int, _vp, _sz, _vp]),
    "pasa_sparse_attn_packed_placed": (_int, [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _dbl, _i64, _i64, _i64,
                                              _i64, _i64, _i64, _i64, _i64, _int, _pl, _int, _vp]),
    "pasa_dense_attn": (_int, [_vp, _vp, _vp, _vp, _dbl, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "pasa_qkv_prologue": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int,
                                 _i64, _i64, _int, _int, _dbl, _vp, _vp, _int, _i64, _int, _vp]),
    "pasa_row_ops": (_int, [_vp, _int, _vp, _int, _vp, _vp, _int, _int, _vp, _vp, _int, _vp, _vp, _vp, _int,
                            _i64, _i64, _i64, _i64, _dbl, _vp]),
}

ABI_VERSION = 11

# Size of the static device array behind pasa_sparse_attn_noalloc (PASA_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20


class PasaError(RuntimeError):
    """A negative status returned by the C ABI."""

    def __init__(self, fn: str, status: int, message: str):
        self.fn = fn
        self.status = status
        self.code = STATUS.get(status, str(status))
        super().__init__(f"{fn} -> {self.code} ({status}): {message}")


_LIB = None


def load() -> ctypes.CDLL:
    """Load the library (once) and bind every entry point; raises if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m pasa_amd.build` "
            "(there is no CPU fallback for the PISA kernels)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.pasa_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(fn: str, status: int) -> None:
    if status != 0:
        msg = load().pasa_last_error().decode(errors="replace")
        raise PasaError(fn, status, msg)


def call(fn: str, *args) -> int:
    """Call an int-returning entry point and raise PasaError on a negative status."""
    rc = getattr(load(), fn)(*args)
    check(fn, rc)
    return rc
