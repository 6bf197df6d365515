"""ctypes binding of the C ABI (include/jjjetson_ops_amd.h) for device tensors.

These wrappers take torch device tensors (HIP memory) and launch on torch's
current stream, so ``torch.cuda.Event`` timing brackets exactly the kernels.
The shared library must have been built (``python -m jjjetson_ops_amd.build``);
loading fails loudly otherwise — there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libjjjetson_ops_amd.so")

JJO_OK = 0
JJO_ERR_INVALID_ARG = 1
JJO_ERR_HIP = 2
JJO_ERR_NO_DEVICE = 3

ALGO_AUTO = 0
ALGO_GEMV = 1
ALGO_MFMA = 2
ALGO_SKINNY = 3

QK = 32
QSUPER = 128
Q8_BLOCK_BYTES = 144
Q4_BLOCK_BYTES = 18

# Every symbol include/jjjetson_ops_amd.h declares.
EXPORTED_SYMBOLS = (
    "jjo_last_error",
    "jjo_version",
    "q8_1_output_bytes",
    "q8_1",
    "q8_1_device",
    "parse_q8_1_output",
    "mat_mul_q4_0_q8_1",
    "mat_mul_q4_0_q8_1_device",
    "mat_mul_q4_0_q8_1_f32_device",
    "mat_mul_q4_0_q8_1_device_algo",
    "mat_mul_q4_0_q8_1_block_sums_device",
    "mat_mul_q4_0_q8_1_grouped_device",
)


class JJOError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where}: status {code}: {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m jjjetson_ops_amd.build` "
                "(there is no CPU fallback for this path)")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64p, i32, i64 = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int64
        L.jjo_last_error.restype = ctypes.c_char_p
        L.jjo_last_error.argtypes = []
        L.jjo_version.restype = ctypes.c_char_p
        L.jjo_version.argtypes = []
        L.q8_1_output_bytes.restype = i64
        L.q8_1_output_bytes.argtypes = [i64p, i32]
        L.q8_1.restype = i32
        L.q8_1.argtypes = [vp, vp, i64p, i32]
        L.q8_1_device.restype = i32
        L.q8_1_device.argtypes = [vp, vp, i64p, i32, vp]
        L.parse_q8_1_output.restype = None
        L.parse_q8_1_output.argtypes = [vp, vp, vp, vp, i64]
        L.mat_mul_q4_0_q8_1.restype = i32
        L.mat_mul_q4_0_q8_1.argtypes = [vp, vp, vp, vp, i64p, i32, i32, i32]
        L.mat_mul_q4_0_q8_1_device.restype = i32
        L.mat_mul_q4_0_q8_1_device.argtypes = [vp, vp, vp, i32, i32, i32, vp]
        L.mat_mul_q4_0_q8_1_f32_device.restype = i32
        L.mat_mul_q4_0_q8_1_f32_device.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp]
        L.mat_mul_q4_0_q8_1_device_algo.restype = i32
        L.mat_mul_q4_0_q8_1_device_algo.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp]
        L.mat_mul_q4_0_q8_1_block_sums_device.restype = i32
        L.mat_mul_q4_0_q8_1_block_sums_device.argtypes = [vp, vp, vp, i32, i32, i32, vp]
        L.mat_mul_q4_0_q8_1_grouped_device.restype = i32
        L.mat_mul_q4_0_q8_1_grouped_device.argtypes = [vp, vp, vp, i32, vp, vp, i32, i32, i32, vp]
        _lib = L
    return _lib


def _check(rc: int, where: str) -> None:
    if rc != JJO_OK:
        raise JJOError(rc, where, lib().jjo_last_error().decode(errors="replace"))


def _dims(dims) -> tuple:
    d = (ctypes.c_int64 * len(dims))(*[int(v) for v in dims])
    return d, len(dims)


def version() -> str:
    return lib().jjo_version().decode()


def q8_1_output_bytes(dims) -> int:
    d, n = _dims(dims)
    return int(lib().q8_1_output_bytes(d, n))


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    return ctypes.c_void_p(stream.cuda_stream)


def _dev(t, name: str):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def quantize_q8_1(x, out, dims=None, stream=None) -> None:
    """Device quantize: x fp32 (dim0 = K fastest), out uint8 of q8_1_output_bytes(dims)."""
    import torch
    if x.dtype != torch.float32 or out.dtype != torch.uint8:
        raise ValueError("x must be float32 and out uint8")
    if dims is None:
        dims = [x.shape[-1], x.numel() // x.shape[-1]]
    need = q8_1_output_bytes(dims)
    if need < 0:
        raise ValueError(f"invalid dims {dims}")
    if out.numel() < need or x.numel() < int(__import__("math").prod(dims)):
        raise ValueError("buffer too small for dims")
    d, n = _dims(dims)
    _check(lib().q8_1_device(_dev(x, "x"), _dev(out, "out"), d, n, _stream(stream)), "q8_1_device")


def mat_mul(w, xq, y, K: int, N: int, M: int, algo: int = ALGO_AUTO, stream=None) -> None:
    """y[M, N] (fp32) = Q4_0 w [N, K/32 blocks] x Q8_1 xq (quantizer layout, M tokens)."""
    import torch
    if y.dtype != torch.float32:
        raise ValueError("y must be float32")
    if w.numel() * w.element_size() < N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small")
    if xq.numel() * xq.element_size() < M * (K // QSUPER) * Q8_BLOCK_BYTES:
        raise ValueError("Q8_1 buffer too small")
    if y.numel() < M * N:
        raise ValueError("output buffer too small")
    _check(lib().mat_mul_q4_0_q8_1_device_algo(_dev(w, "w"), _dev(xq, "xq"), _dev(y, "y"), K, N, M, algo,
                                               _stream(stream)), "mat_mul_q4_0_q8_1_device")


def mat_mul_f32(w, x, xq, y, K: int, N: int, M: int, stream=None) -> None:
    """Quantize fp32 x [M, K] (into xq, may be None when M == 1) and y[M, N] = W . x."""
    import torch
    if x.dtype != torch.float32 or y.dtype != torch.float32:
        raise ValueError("x and y must be float32")
    if x.numel() < M * K or y.numel() < M * N:
        raise ValueError("x or y too small")
    if xq is not None and xq.numel() * xq.element_size() < M * (K // QSUPER) * Q8_BLOCK_BYTES:
        raise ValueError("Q8_1 workspace too small")
    if w.numel() * w.element_size() < N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small")
    xqp = _dev(xq, "xq") if xq is not None else ctypes.c_void_p(0)
    _check(lib().mat_mul_q4_0_q8_1_f32_device(_dev(w, "w"), _dev(x, "x"), xqp, _dev(y, "y"), K, N, M,
                                              _stream(stream)), "mat_mul_q4_0_q8_1_f32_device")


def block_sums(w, xq, out, K: int, N: int, M: int, stream=None) -> None:
    """int32 out[M, N, K/32] per-block integer dots."""
    import torch
    if out.dtype != torch.int32 or out.numel() < M * N * (K // QK):
        raise ValueError("out must be int32 with M*N*K/32 elements")
    _check(lib().mat_mul_q4_0_q8_1_block_sums_device(_dev(w, "w"), _dev(xq, "xq"), _dev(out, "out"), K, N, M,
                                                     _stream(stream)), "block_sums")


def grouped_mat_mul(w, xq, expert_offsets, y, K: int, N: int, n_routes: int, route_dst=None,
                    stream=None) -> None:
    """One-launch MoE expert GEMM over routes sorted by expert (see the C header)."""
    import torch
    n_experts = expert_offsets.numel() - 1
    if expert_offsets.dtype != torch.int32:
        raise ValueError("expert_offsets must be int32")
    if route_dst is not None and (route_dst.dtype != torch.int32 or route_dst.numel() < n_routes):
        raise ValueError("route_dst must be int32 with n_routes entries")
    if w.numel() * w.element_size() < n_experts * N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small for all experts")
    rd = _dev(route_dst, "route_dst") if route_dst is not None else ctypes.c_void_p(0)
    _check(lib().mat_mul_q4_0_q8_1_grouped_device(_dev(w, "w"), _dev(xq, "xq"), _dev(expert_offsets, "offsets"),
                                                  n_experts, rd, _dev(y, "y"), K, N, n_routes,
                                                  _stream(stream)), "grouped_mat_mul")


def parse_q8_1(raw, n_blocks: int):
    """Host parse through the C ABI: returns (qs int8[n,128], d f32[n,4], s f32[n,4])."""
    import numpy as np
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if raw.size < n_blocks * Q8_BLOCK_BYTES:
        raise ValueError("raw buffer too small")
    qs = np.empty((n_blocks, 128), np.int8)
    d = np.empty((n_blocks, 4), np.float32)
    s = np.empty((n_blocks, 4), np.float32)
    lib().parse_q8_1_output(raw.ctypes.data, qs.ctypes.data, d.ctypes.data, s.ctypes.data, n_blocks)
    return qs, d, s
