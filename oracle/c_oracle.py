"""ctypes loader of the C oracle (liboracle_q4q8.so) — TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_q4q8.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < (HERE / "q4q8_oracle.c").stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB))
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_q8_1_n_blocks.restype = i64
        L.oracle_q8_1_n_blocks.argtypes = [vp]
        L.oracle_quantize_q8_1.restype = ctypes.c_int
        L.oracle_quantize_q8_1.argtypes = [vp, vp, vp]
        L.oracle_parse_q8_1.restype = None
        L.oracle_parse_q8_1.argtypes = [vp, vp, vp, vp, i64]
        L.oracle_block_sums.restype = ctypes.c_int
        L.oracle_block_sums.argtypes = [vp, vp, vp, i64, i64, i64]
        L.oracle_matmul.restype = ctypes.c_int
        L.oracle_matmul.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_int]
        L.oracle_quantize_q4_0.restype = ctypes.c_int
        L.oracle_quantize_q4_0.argtypes = [vp, vp, i64, i64]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def dims4(dims):
    return np.array((list(dims) + [1, 1, 1])[:4], dtype=np.int64)


def quantize_q8_1(x: np.ndarray, dims) -> np.ndarray:
    """x: float32 buffer with dim0 fastest (any contiguous array; raw memory order is used)."""
    d = dims4(dims)
    flat = np.ascontiguousarray(np.ravel(np.asarray(x, dtype=np.float32), order="K"))
    out = np.zeros(int(lib().oracle_q8_1_n_blocks(_p(d))) * 144, dtype=np.uint8)
    rc = lib().oracle_quantize_q8_1(_p(flat), _p(out), _p(d))
    if rc:
        raise ValueError(f"oracle_quantize_q8_1 rejected dims {dims}")
    return out


def parse_q8_1(raw: np.ndarray, n_blocks: int):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    qs = np.empty((n_blocks, 128), np.int8)
    d = np.empty((n_blocks, 4), np.float32)
    s = np.empty((n_blocks, 4), np.float32)
    lib().oracle_parse_q8_1(_p(raw), _p(qs), _p(d), _p(s), n_blocks)
    return qs, d, s


def block_sums(w: np.ndarray, xq: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
    out = np.empty((M, N, K // 32), np.int32)
    rc = lib().oracle_block_sums(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(xq)), _p(out), K, N, M)
    if rc:
        raise ValueError("bad K")
    return out


def matmul(w: np.ndarray, xq: np.ndarray, K: int, N: int, M: int, mode: int = 0) -> np.ndarray:
    """mode 0: fp64 evaluation; mode 1: fp32 in the reference kernel's sequential order."""
    out = np.empty((M, N), np.float32)
    rc = lib().oracle_matmul(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(xq)), _p(out), K, N, M, mode)
    if rc:
        raise ValueError("bad K")
    return out


def quantize_q4_0(wf: np.ndarray) -> np.ndarray:
    wf = np.ascontiguousarray(wf, dtype=np.float32)
    N, K = wf.shape
    out = np.empty(N * (K // 32) * 18, np.uint8)
    if lib().oracle_quantize_q4_0(_p(wf), _p(out), N, K):
        raise ValueError("bad K")
    return out


def f32_to_f16_bits(v: float) -> int:
    return int(lib().oracle_f32_to_f16(ctypes.c_float(v)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(h))
