"""ctypes access to oracle/lib/liboracle_codec.so, the C restatement of the
codecs in oracle/codec.py (same rules, fast enough for full expert stacks).
Test infrastructure only."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "lib" / "liboracle_codec.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def nf4_quantize(w_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w.shape
    codes = np.empty((rows, cols // 2), dtype=np.uint8)
    absmax = np.empty((rows, cols // 64), dtype=np.uint16)
    _load().oracle_nf4_quantize(_p(w), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(codes),
                                _p(absmax))
    return codes, absmax


def nf4_dequantize(codes: np.ndarray, absmax: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    a = np.ascontiguousarray(absmax, dtype=np.uint16)
    rows, half = c.shape
    out = np.empty((rows, half * 2), dtype=np.uint16)
    _load().oracle_nf4_dequantize(_p(c), _p(a), ctypes.c_int64(rows), ctypes.c_int64(half * 2),
                                  _p(out))
    return out


def int8_quantize(w_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty(rows, dtype=np.uint16)
    _load().oracle_int8_quantize(_p(w), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(q), _p(s))
    return q, s


def int8_dequantize(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    qq = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(scale, dtype=np.uint16)
    rows, cols = qq.shape
    out = np.empty((rows, cols), dtype=np.uint16)
    _load().oracle_int8_dequantize(_p(qq), _p(s), ctypes.c_int64(rows), ctypes.c_int64(cols),
                                   _p(out))
    return out
