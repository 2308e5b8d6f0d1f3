"""ctypes binding of libqmm4.so (the C ABI in include/qmm4.h).

There is no fallback: if the library is missing or fails to load, every call raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqmm4.so")

QMM4_OK = 0
QMM4_ERR_INVALID = -22
QMM4_ERR_UNSUPPORTED = -95
QMM4_ERR_NOMEM = -12
QMM4_ERR_HIP = -5
QMM4_ERR_CAPTURE = -16

QMM4_EPILOGUE_NONE = 0
QMM4_EPILOGUE_SILU_MUL = 1

# Size of qmm4_affine_bf16_noalloc's static device array per GPU (QMM4_NOALLOC_SCRATCH_BYTES).
QMM4_NOALLOC_SCRATCH_BYTES = 136 * 1024 * 1024

# name -> (restype, argtypes); the symbols include/qmm4.h declares.
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
SIGNATURES = {
    "qmm4_affine_bf16": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _vp]),
    "qmm4_affine_bf16_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _vp]),
    "qmm4_gate_up_silu_bf16": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _vp]),
    "dequant4_affine_bf16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _vp]),
    "qmm4_add_rms_norm_bf16": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]),
    "qmm4_add_rms_norm_qmm_bf16": (_int, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _i64, _i64, _i64, _int, _int, _int, _int, _vp]),
    "qmm4_last_error": (ctypes.c_char_p, []),
    "qmm4_abi_version": (_int, []),
}

_lib = None


class LibraryNotBuilt(RuntimeError):
    pass


def load():
    """Load libqmm4.so once and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(
            f"{LIB_PATH} not found: build it with `python -m mlx_tree_spec_amd.build` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().qmm4_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Map a C return code onto the Python exception the reference's callers would see."""
    if rc == QMM4_OK:
        return
    msg = f"[{what}] {last_error()}"
    if rc == QMM4_ERR_INVALID:
        raise ValueError(msg)
    if rc == QMM4_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == QMM4_ERR_NOMEM:
        raise MemoryError(msg)
    raise RuntimeError(f"{msg} (code {rc})")
