"""ctypes binding of oracle/qmm4_cpu.c — TEST INFRASTRUCTURE (test reference and timed CPU baseline).

Loads the AVX-512 build where the host CPU has AVX-512 F/BW/VL, else the AVX2 build. Both are
built by `make -C oracle` (also run by __graft_entry__.build()).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def _has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512vl", "avx512dq"} <= fl
    except OSError:
        pass
    return False


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib_path() -> str:
    return os.path.join(_HERE, "libqmm4_oracle_v4.so" if _has_avx512() else "libqmm4_oracle_v3.so")


def load():
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run `make -C oracle`")
        lib = ctypes.CDLL(path)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        i64 = ctypes.c_int64
        lib.qmm4_oracle_qmm.argtypes = [u16p, u32p, u16p, u16p, u16p, i64, i64, i64, ctypes.c_int]
        lib.qmm4_oracle_qmm.restype = ctypes.c_int
        lib.qmm4_oracle_qmm_f32.argtypes = [u16p, u32p, u16p, u16p, ctypes.POINTER(ctypes.c_float), i64, i64,
                                             i64, ctypes.c_int]
        lib.qmm4_oracle_qmm_f32.restype = ctypes.c_int
        lib.qmm4_oracle_dequant.argtypes = [u32p, u16p, u16p, u16p, i64, i64, ctypes.c_int]
        lib.qmm4_oracle_dequant.restype = ctypes.c_int
        lib.qmm4_oracle_num_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _p(a, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


def num_threads() -> int:
    return int(load().qmm4_oracle_num_threads())


def qmm(x, w, s, b, n_threads: int = 0) -> np.ndarray:
    """bf16 bits [M, N] of y = x @ dequant(w).T (fp32 accumulation)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.uint16)
    rc = load().qmm4_oracle_qmm(_p(x, ctypes.c_uint16), _p(w, ctypes.c_uint32), _p(s, ctypes.c_uint16),
                                _p(b, ctypes.c_uint16), _p(y, ctypes.c_uint16), m, n, k, n_threads)
    if rc != 0:
        raise ValueError(f"qmm4_oracle_qmm returned {rc}")
    return y


def qmm_f32(x, w, s, b, n_threads: int = 0) -> np.ndarray:
    """fp32 [M, N] of y = x @ dequant(w).T (fp32 accumulation, not rounded to bf16)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    rc = load().qmm4_oracle_qmm_f32(_p(x, ctypes.c_uint16), _p(w, ctypes.c_uint32), _p(s, ctypes.c_uint16),
                                    _p(b, ctypes.c_uint16), _p(y, ctypes.c_float), m, n, k, n_threads)
    if rc != 0:
        raise ValueError(f"qmm4_oracle_qmm_f32 returned {rc}")
    return y


def dequant(w, s, b, n_threads: int = 0) -> np.ndarray:
    """bf16 bits [N, K] of the dequantized weight."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    n, kw = w.shape
    out = np.empty((n, kw * 8), dtype=np.uint16)
    rc = load().qmm4_oracle_dequant(_p(w, ctypes.c_uint32), _p(s, ctypes.c_uint16), _p(b, ctypes.c_uint16),
                                    _p(out, ctypes.c_uint16), n, kw * 8, n_threads)
    if rc != 0:
        raise ValueError(f"qmm4_oracle_dequant returned {rc}")
    return out
