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
ALGO_SKINNY_LDS = 4
ALGO_MFMA64 = 5
ALGO_MFMA32 = 6
ALGO_MFMA_W32 = 7

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
    "mat_mul_q4_0s_q8_1_grouped_device",
    "jjo_read_floor_device",
    "linear_q4_0_workspace_bytes",
    "linear_q4_0_forward_device",
    "linear_q4_0s_forward_device",
    "linear_q4_0_forward_host",
    "linear_q4_0_noalloc_max_bytes",
    "linear_q4_0_forward_device_noalloc",
    "moe_top_k_device",
    "moe_dispatch_q8_1_device",
    "moe_q4_0_gate_up_device",
    "moe_q4_0_gate_up_swiglu_q8_1_device",
    "swiglu_quantize_q8_1_device",
    "moe_combine_device",
    "moe_q4_0_ffn_workspace_bytes",
    "moe_q4_0_ffn_forward_device",
    "moe_q4_0s_ffn_forward_device",
    "q4_0_bytes",
    "quantize_q4_0_host",
    "quantize_q4_0_device",
    "safetensors_read_file_q4_0",
    "jjo_host_tensors_free",
    "jjo_host_tensors_find",
    "safetensors_write_file_q4_0",
    "safetensors_quantize_q4_0",
    "q4_0_split_bytes",
    "q4_0_to_split",
    "q4_0_from_split",
    "q4_0_to_split_device",
    "mat_mul_q4_0s_q8_1_device",
    "mat_mul_q4_0s_q8_1_f32_device",
)

WEIGHT_DTYPE_F32 = 0
WEIGHT_DTYPE_Q4_0 = 1


class HostTensor(ctypes.Structure):
    """jjo_host_tensor (include/jjjetson_ops_amd.h)."""
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("data", ctypes.c_void_p),
        ("dims", ctypes.POINTER(ctypes.c_int64)),
        ("ndim", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("nbytes", ctypes.c_int64),
    ]


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
        L.mat_mul_q4_0s_q8_1_grouped_device.restype = i32
        L.mat_mul_q4_0s_q8_1_grouped_device.argtypes = [vp, vp, vp, i32, vp, vp, i32, i32, i32, vp]
        L.jjo_read_floor_device.restype = i32
        L.jjo_read_floor_device.argtypes = [vp, i64, vp, vp]
        L.linear_q4_0_workspace_bytes.restype = i64
        L.linear_q4_0_workspace_bytes.argtypes = [i32, i32]
        L.linear_q4_0_forward_device.restype = i32
        L.linear_q4_0_forward_device.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32]
        L.linear_q4_0s_forward_device.restype = i32
        L.linear_q4_0s_forward_device.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32]
        L.linear_q4_0_noalloc_max_bytes.restype = i64
        L.linear_q4_0_noalloc_max_bytes.argtypes = []
        L.linear_q4_0_forward_device_noalloc.restype = i32
        L.linear_q4_0_forward_device_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, i32]
        L.linear_q4_0_forward_host.restype = i32
        L.linear_q4_0_forward_host.argtypes = [vp, vp, vp, i32, i32, i32]
        L.moe_top_k_device.restype = i32
        L.moe_top_k_device.argtypes = [vp, vp, vp, vp, i32, i32, i32]
        L.moe_dispatch_q8_1_device.restype = i32
        L.moe_dispatch_q8_1_device.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp]
        L.moe_q4_0_gate_up_device.restype = i32
        L.moe_q4_0_gate_up_device.argtypes = [vp, vp, vp, vp, vp, i32, vp, i32, i32, i32]
        L.moe_q4_0_gate_up_swiglu_q8_1_device.restype = i32
        L.moe_q4_0_gate_up_swiglu_q8_1_device.argtypes = [vp, vp, vp, vp, vp, i32, vp, i32, i32, i32]
        L.swiglu_quantize_q8_1_device.restype = i32
        L.swiglu_quantize_q8_1_device.argtypes = [vp, vp, vp, vp, i32, i32]
        L.moe_combine_device.restype = i32
        L.moe_combine_device.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32]
        L.moe_q4_0_ffn_workspace_bytes.restype = i64
        L.moe_q4_0_ffn_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
        L.moe_q4_0_ffn_forward_device.restype = i32
        L.moe_q4_0_ffn_forward_device.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64]
        L.moe_q4_0s_ffn_forward_device.restype = i32
        L.moe_q4_0s_ffn_forward_device.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64]
        L.q4_0_bytes.restype = i64
        L.q4_0_bytes.argtypes = [i64, i64]
        L.quantize_q4_0_host.restype = i32
        L.quantize_q4_0_host.argtypes = [vp, vp, i64, i64, i32]
        L.quantize_q4_0_device.restype = i32
        L.quantize_q4_0_device.argtypes = [vp, vp, vp, i64, i64]
        ht_p = ctypes.POINTER(HostTensor)
        L.safetensors_read_file_q4_0.restype = i32
        L.safetensors_read_file_q4_0.argtypes = [ctypes.c_char_p, ctypes.POINTER(ht_p), ctypes.POINTER(i32)]
        L.jjo_host_tensors_free.restype = None
        L.jjo_host_tensors_free.argtypes = [ht_p, i32]
        L.jjo_host_tensors_find.restype = ht_p
        L.jjo_host_tensors_find.argtypes = [ht_p, i32, ctypes.c_char_p]
        L.safetensors_write_file_q4_0.restype = i32
        L.safetensors_write_file_q4_0.argtypes = [ctypes.c_char_p, ht_p, i32]
        L.safetensors_quantize_q4_0.restype = i32
        L.safetensors_quantize_q4_0.argtypes = [ctypes.c_char_p, ctypes.c_char_p,
                                                ctypes.POINTER(ctypes.c_char_p), i32, i32]
        L.q4_0_split_bytes.restype = i64
        L.q4_0_split_bytes.argtypes = [i64, i64]
        L.q4_0_to_split.restype = i32
        L.q4_0_to_split.argtypes = [vp, vp, i64, i64]
        L.q4_0_from_split.restype = i32
        L.q4_0_from_split.argtypes = [vp, vp, i64, i64]
        L.q4_0_to_split_device.restype = i32
        L.q4_0_to_split_device.argtypes = [vp, vp, i32, i32, vp]
        L.mat_mul_q4_0s_q8_1_device.restype = i32
        L.mat_mul_q4_0s_q8_1_device.argtypes = [vp, vp, vp, i32, i32, i32, vp]
        L.mat_mul_q4_0s_q8_1_f32_device.restype = i32
        L.mat_mul_q4_0s_q8_1_f32_device.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp]
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


# ---------------------------------------------------------------- split weight layout
def q4_0_to_split_host(w, nrows: int, ncols_k: int):
    """Host repack: uint8 block_q4_0 rows -> split layout (a new uint8 ndarray)."""
    import numpy as np
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    n = int(lib().q4_0_split_bytes(nrows, ncols_k))
    if n < 0 or w.size < n:
        raise ValueError("invalid shape or weight buffer too small")
    out = np.empty(n, np.uint8)
    _check(lib().q4_0_to_split(w.ctypes.data, out.ctypes.data, nrows, ncols_k), "q4_0_to_split")
    return out


def q4_0_from_split_host(ws, nrows: int, ncols_k: int):
    """Host inverse repack: split layout -> block_q4_0 rows (a new uint8 ndarray)."""
    import numpy as np
    ws = np.ascontiguousarray(ws, dtype=np.uint8).reshape(-1)
    n = int(lib().q4_0_split_bytes(nrows, ncols_k))
    if n < 0 or ws.size < n:
        raise ValueError("invalid shape or weight buffer too small")
    out = np.empty(n, np.uint8)
    _check(lib().q4_0_from_split(ws.ctypes.data, out.ctypes.data, nrows, ncols_k), "q4_0_from_split")
    return out


def q4_0_to_split(w, out, nrows: int, ncols_k: int, stream=None) -> None:
    """Device repack of block_q4_0 rows (w) into the split layout (out, 16-byte aligned)."""
    n = nrows * (ncols_k // QK) * Q4_BLOCK_BYTES
    if w.numel() * w.element_size() < n or out.numel() * out.element_size() < n:
        raise ValueError("buffer too small")
    _check(lib().q4_0_to_split_device(_dev(w, "w"), _dev(out, "out"), nrows, ncols_k, _stream(stream)),
           "q4_0_to_split_device")


def mat_mul_split(ws, xq, y, K: int, N: int, M: int, stream=None) -> None:
    """y[M, N] = split-layout Q4_0 ws x Q8_1 xq (quantizer layout)."""
    if ws.numel() * ws.element_size() < N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small")
    if xq.numel() * xq.element_size() < M * (K // QSUPER) * Q8_BLOCK_BYTES or y.numel() < M * N:
        raise ValueError("Q8_1 or output buffer too small")
    _check(lib().mat_mul_q4_0s_q8_1_device(_dev(ws, "w"), _dev(xq, "xq"), _dev(y, "y"), K, N, M, _stream(stream)),
           "mat_mul_q4_0s_q8_1_device")


def mat_mul_split_f32(ws, x, xq, y, K: int, N: int, M: int, stream=None) -> None:
    """Quantize fp32 x [M, K] (into xq, may be None when M == 1) and y = split W . x."""
    import torch
    if x.dtype != torch.float32 or y.dtype != torch.float32:
        raise ValueError("x and y must be float32")
    if x.numel() < M * K or y.numel() < M * N:
        raise ValueError("x or y too small")
    if xq is not None and xq.numel() * xq.element_size() < M * (K // QSUPER) * Q8_BLOCK_BYTES:
        raise ValueError("Q8_1 workspace too small")
    if ws.numel() * ws.element_size() < N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small")
    xqp = _dev(xq, "xq") if xq is not None else ctypes.c_void_p(0)
    _check(lib().mat_mul_q4_0s_q8_1_f32_device(_dev(ws, "w"), _dev(x, "x"), xqp, _dev(y, "y"), K, N, M,
                                               _stream(stream)), "mat_mul_q4_0s_q8_1_f32_device")


def block_sums(w, xq, out, K: int, N: int, M: int, stream=None) -> None:
    """int32 out[M, N, K/32] per-block integer dots."""
    import torch
    if out.dtype != torch.int32 or out.numel() < M * N * (K // QK):
        raise ValueError("out must be int32 with M*N*K/32 elements")
    _check(lib().mat_mul_q4_0_q8_1_block_sums_device(_dev(w, "w"), _dev(xq, "xq"), _dev(out, "out"), K, N, M,
                                                     _stream(stream)), "block_sums")


def grouped_mat_mul(w, xq, expert_offsets, y, K: int, N: int, n_routes: int, route_dst=None,
                    stream=None, split: bool = False) -> None:
    """One-launch MoE expert GEMM over routes sorted by expert (see the C header);
    split: w holds the stacked experts repacked into the split layout."""
    import torch
    n_experts = expert_offsets.numel() - 1
    if expert_offsets.dtype != torch.int32:
        raise ValueError("expert_offsets must be int32")
    if route_dst is not None and (route_dst.dtype != torch.int32 or route_dst.numel() < n_routes):
        raise ValueError("route_dst must be int32 with n_routes entries")
    if w.numel() * w.element_size() < n_experts * N * (K // QK) * Q4_BLOCK_BYTES:
        raise ValueError("weight buffer too small for all experts")
    rd = _dev(route_dst, "route_dst") if route_dst is not None else ctypes.c_void_p(0)
    fn = lib().mat_mul_q4_0s_q8_1_grouped_device if split else lib().mat_mul_q4_0_q8_1_grouped_device
    _check(fn(_dev(w, "w"), _dev(xq, "xq"), _dev(expert_offsets, "offsets"), n_experts, rd, _dev(y, "y"), K, N,
              n_routes, _stream(stream)), "grouped_mat_mul")


def read_floor(src, nbytes: int, out, stream=None) -> None:
    """jjo_read_floor_device: one plain read of nbytes of a device tensor."""
    _check(lib().jjo_read_floor_device(_dev(src, "src"), int(nbytes), _dev(out, "out"), _stream(stream)),
           "jjo_read_floor_device")


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


# ---------------------------------------------------------------- engine linear
def linear_q4_0(x, w, y, in_features: int, out_features: int, num_tokens: int, ws=None, stream=None) -> None:
    """linear_q4_0_forward_device: y [T, out] = x [T, in] . dequant(w [out, in/32 blocks]).T"""
    _check(lib().linear_q4_0_forward_device(_stream(stream), None if ws is None else _dev(ws, "ws"), _dev(x, "x"),
                                            _dev(w, "w"), _dev(y, "y"), in_features, out_features, num_tokens),
           "linear_q4_0_forward_device")


def linear_q4_0_split(x, ws_split, y, in_features: int, out_features: int, num_tokens: int, ws=None,
                      stream=None) -> None:
    """linear_q4_0s_forward_device: linear_q4_0 on weights repacked into the split layout."""
    _check(lib().linear_q4_0s_forward_device(_stream(stream), None if ws is None else _dev(ws, "ws"), _dev(x, "x"),
                                             _dev(ws_split, "w"), _dev(y, "y"), in_features, out_features,
                                             num_tokens),
           "linear_q4_0s_forward_device")


def linear_q4_0_noalloc(x, w, y, in_features: int, out_features: int, num_tokens: int, stream=None) -> None:
    """linear_q4_0_forward_device_noalloc: as linear_q4_0 with the library's static
    Q8_1 buffer instead of a workspace (calls on one device must not overlap)."""
    _check(lib().linear_q4_0_forward_device_noalloc(_stream(stream), _dev(x, "x"), _dev(w, "w"), _dev(y, "y"),
                                                    in_features, out_features, num_tokens),
           "linear_q4_0_forward_device_noalloc")


def linear_q4_0_noalloc_max_bytes() -> int:
    return int(lib().linear_q4_0_noalloc_max_bytes())


def linear_q4_0_workspace_bytes(in_features: int, num_tokens: int) -> int:
    return int(lib().linear_q4_0_workspace_bytes(in_features, num_tokens))


# ---------------------------------------------------------------- MoE FFN
def moe_top_k(logits, weights, ids, num_tokens: int, num_experts: int, top_k: int, stream=None) -> None:
    _check(lib().moe_top_k_device(_stream(stream), _dev(logits, "logits"), _dev(weights, "weights"),
                                  _dev(ids, "ids"), num_tokens, num_experts, top_k), "moe_top_k_device")


def moe_dispatch(ids, offsets, src_route, dst_of_route, num_tokens: int, top_k: int, hidden: int,
                 num_experts: int, xq=None, xq_perm=None, stream=None) -> None:
    _check(lib().moe_dispatch_q8_1_device(_stream(stream), _dev(ids, "ids"), None if xq is None else _dev(xq, "xq"),
                                          num_tokens, top_k, hidden, num_experts, _dev(offsets, "offsets"),
                                          _dev(src_route, "src_route"), _dev(dst_of_route, "dst_of_route"),
                                          None if xq_perm is None else _dev(xq_perm, "xq_perm")),
           "moe_dispatch_q8_1_device")


def moe_gate_up(w_gate, w_up, xq_perm, offsets, num_experts: int, gate_up, hidden: int, inter: int,
                n_routes: int, stream=None) -> None:
    _check(lib().moe_q4_0_gate_up_device(_stream(stream), _dev(w_gate, "w_gate"), _dev(w_up, "w_up"),
                                         _dev(xq_perm, "xq_perm"), _dev(offsets, "offsets"), num_experts,
                                         _dev(gate_up, "gate_up"), hidden, inter, n_routes),
           "moe_q4_0_gate_up_device")


def moe_gate_up_swiglu(w_gate, w_up, xq_perm, offsets, num_experts: int, mid_q, hidden: int, inter: int,
                       n_routes: int, stream=None) -> None:
    _check(lib().moe_q4_0_gate_up_swiglu_q8_1_device(_stream(stream), _dev(w_gate, "w_gate"), _dev(w_up, "w_up"),
                                                     _dev(xq_perm, "xq_perm"), _dev(offsets, "offsets"), num_experts,
                                                     _dev(mid_q, "mid_q"), hidden, inter, n_routes),
           "moe_q4_0_gate_up_swiglu_q8_1_device")


def swiglu_quantize(gate_up, mid_q, rows: int, inter: int, mid_f32=None, stream=None) -> None:
    _check(lib().swiglu_quantize_q8_1_device(_stream(stream), _dev(gate_up, "gate_up"), _dev(mid_q, "mid_q"),
                                             None if mid_f32 is None else _dev(mid_f32, "mid_f32"), rows, inter),
           "swiglu_quantize_q8_1_device")


def moe_combine(expert_out, dst_of_route, weights, y, num_tokens: int, hidden: int, top_k: int,
                stream=None) -> None:
    _check(lib().moe_combine_device(_stream(stream), _dev(expert_out, "expert_out"),
                                    _dev(dst_of_route, "dst_of_route"), _dev(weights, "weights"), _dev(y, "y"),
                                    num_tokens, hidden, top_k), "moe_combine_device")


def moe_ffn_workspace_bytes(num_tokens: int, hidden: int, inter: int, num_experts: int, top_k: int) -> int:
    return int(lib().moe_q4_0_ffn_workspace_bytes(num_tokens, hidden, inter, num_experts, top_k))


def moe_ffn(x, logits, w_gate, w_up, w_down, y, num_tokens: int, hidden: int, inter: int, num_experts: int,
            top_k: int, ws, stream=None, split: bool = False) -> None:
    """The Q4_0 MoE FFN; split: the three expert weight buffers are in the split layout."""
    fn = lib().moe_q4_0s_ffn_forward_device if split else lib().moe_q4_0_ffn_forward_device
    _check(fn(_stream(stream), _dev(x, "x"), _dev(logits, "logits"), _dev(w_gate, "w_gate"), _dev(w_up, "w_up"),
              _dev(w_down, "w_down"), _dev(y, "y"), num_tokens, hidden, inter, num_experts, top_k, _dev(ws, "ws"),
              ws.numel() * ws.element_size()),
           "moe_q4_0s_ffn_forward_device" if split else "moe_q4_0_ffn_forward_device")
