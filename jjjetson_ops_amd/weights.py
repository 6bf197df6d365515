"""On-disk Q4_0 weights: the host side of the engine's weight loader with a Q4_0 dtype.

Mirrors the reference's loader (src/model/weight_loader.h:12-44: WeightDtype,
HostTensor, weight_load_result_find; src/model/safetensors_reader.cpp:369-494:
safetensors_read_file), which holds F32 tensors only.  Every call goes through the
C ABI (include/jjjetson_ops_amd.h); the GPU quantizer runs on device tensors.

File convention: a Q4_0 tensor of logical shape [rows, cols] is stored as dtype
U8, shape [rows, cols/32, 18] (row-major block_q4_0, the layout the kernels read)
with the header metadata entry ``"q4_0:<name>": "Q4_0"``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from os import fspath

import numpy as np

from . import capi

F32 = capi.WEIGHT_DTYPE_F32
Q4_0 = capi.WEIGHT_DTYPE_Q4_0


@dataclass
class WeightTensor:
    """One loaded tensor: F32 data shaped ``dims``, or Q4_0 bytes [rows, cols/32, 18]."""
    dtype: int
    dims: tuple
    data: np.ndarray

    @property
    def nbytes(self) -> int:
        return int(self.data.nbytes)


def q4_0_bytes(rows: int, cols: int) -> int:
    return int(capi.lib().q4_0_bytes(int(rows), int(cols)))


def quantize_q4_0(w: np.ndarray, num_threads: int = 0) -> np.ndarray:
    """Host fp32 [rows, cols] -> Q4_0 bytes, uint8 [rows, cols/32, 18]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("w must be 2-D [rows, cols]")
    rows, cols = w.shape
    n = q4_0_bytes(rows, cols)
    if n < 0:
        raise ValueError(f"cols ({cols}) must be a positive multiple of 32")
    out = np.empty((rows, cols // 32, 18), dtype=np.uint8)
    capi._check(capi.lib().quantize_q4_0_host(w.ctypes.data, out.ctypes.data, rows, cols, int(num_threads)),
                "quantize_q4_0_host")
    return out


def quantize_q4_0_device(w, out, rows: int, cols: int, stream=None) -> None:
    """Device fp32 [rows, cols] (torch) -> Q4_0 bytes into ``out`` (torch uint8)."""
    import torch
    if w.dtype != torch.float32 or out.dtype != torch.uint8:
        raise ValueError("w must be float32 and out uint8")
    need = q4_0_bytes(rows, cols)
    if need < 0 or w.numel() < rows * cols or out.numel() < need:
        raise ValueError("bad shape or buffer too small")
    capi._check(capi.lib().quantize_q4_0_device(capi._stream(stream), capi._dev(w, "w"), capi._dev(out, "out"),
                                                int(rows), int(cols)), "quantize_q4_0_device")


def read_safetensors(path) -> dict:
    """All tensors of a .safetensors file (F32 and Q4_0) as {name: WeightTensor}."""
    L = capi.lib()
    arr = ctypes.POINTER(capi.HostTensor)()
    n = ctypes.c_int(0)
    capi._check(L.safetensors_read_file_q4_0(fspath(path).encode(), ctypes.byref(arr), ctypes.byref(n)),
                "safetensors_read_file_q4_0")
    out = {}
    try:
        for i in range(n.value):
            t = arr[i]
            dims = tuple(int(t.dims[j]) for j in range(t.ndim))
            raw = np.ctypeslib.as_array(ctypes.cast(t.data, ctypes.POINTER(ctypes.c_uint8)),
                                        shape=(int(t.nbytes),)).copy() if t.nbytes else np.empty(0, np.uint8)
            if t.dtype == F32:
                data = raw.view(np.float32).reshape(dims)
            else:
                data = raw.reshape(dims[0], dims[1] // 32, 18)
            out[t.name.decode()] = WeightTensor(int(t.dtype), dims, data)
    finally:
        L.jjo_host_tensors_free(arr, n.value)
    return out


def write_safetensors(path, tensors: dict) -> None:
    """Write {name: WeightTensor | float32 ndarray} in insertion order."""
    items = []
    for name, t in tensors.items():
        if isinstance(t, np.ndarray):
            t = WeightTensor(F32, tuple(t.shape), np.ascontiguousarray(t, dtype=np.float32))
        items.append((name, t))
    arr = (capi.HostTensor * max(1, len(items)))()
    keep = []
    for i, (name, t) in enumerate(items):
        data = np.ascontiguousarray(t.data)
        dims = (ctypes.c_int64 * len(t.dims))(*t.dims)
        nm = name.encode()
        keep += [data, dims, nm]
        arr[i].name = nm
        arr[i].data = data.ctypes.data if data.nbytes else None
        arr[i].dims = dims
        arr[i].ndim = len(t.dims)
        arr[i].dtype = t.dtype
        arr[i].nbytes = data.nbytes
    capi._check(capi.lib().safetensors_write_file_q4_0(fspath(path).encode(), arr, len(items)),
                "safetensors_write_file_q4_0")


def quantize_file(in_path, out_path, names=None, num_threads: int = 0) -> None:
    """Offline repacker: copy a checkpoint with the named 2-D F32 tensors (all
    eligible ones when ``names`` is None) quantized to Q4_0."""
    if names is None:
        arr, n = None, -1
    else:
        enc = [s.encode() for s in names]
        arr = (ctypes.c_char_p * max(1, len(enc)))(*enc)
        n = len(enc)
    capi._check(capi.lib().safetensors_quantize_q4_0(fspath(in_path).encode(), fspath(out_path).encode(), arr, n,
                                                     int(num_threads)), "safetensors_quantize_q4_0")
