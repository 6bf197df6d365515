"""Q4_0 weight packing (fp32 [N, K] -> 18-byte blocks, row-major [N][K/32]).

The reference ships no Q4_0 quantizer (its MMQ consumes ready-made ggml Q4_0
bytes, src/cuda/mm_q4_0_q8_1.cu:35-38); this is the ggml-style packer used to
make test and benchmark weights: per 32-block take the element of largest
magnitude ``mx``, ``d = mx / -8`` (stored fp16), ``nib = min(15, int(w/d + 8.5))``
with ``1/d`` precomputed, element j in the low nibble of byte j and element
j+16 in its high nibble.
"""
from __future__ import annotations

import numpy as np


def quantize_q4_0_np(wf: np.ndarray) -> np.ndarray:
    wf = np.asarray(wf, dtype=np.float32)
    N, K = wf.shape
    assert K % 32 == 0
    nb = K // 32
    g = wf.reshape(N, nb, 32)
    idx = np.argmax(np.abs(g), axis=2)
    mx = np.take_along_axis(g, idx[..., None], axis=2)[..., 0]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (g * idv[..., None]).astype(np.float32) + np.float32(8.5)
    nib = np.clip(np.trunc(v), 0, 15).astype(np.uint8)
    out = np.empty((N, nb, 18), dtype=np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).reshape(N, nb, 1).view(np.uint8)
    out[:, :, 2:18] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    return out.reshape(-1)


def quantize_q4_0_torch(wf):
    """Same packing on a torch tensor (any device); returns uint8 [N*K/32*18]."""
    import torch
    N, K = wf.shape
    assert K % 32 == 0
    nb = K // 32
    g = wf.to(torch.float32).reshape(N, nb, 32)
    idx = torch.argmax(g.abs(), dim=2, keepdim=True)
    mx = torch.gather(g, 2, idx)[..., 0]
    d = mx / -8.0
    idv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    v = g * idv[..., None]
    v = v + 8.5
    nib = torch.clamp(torch.trunc(v), 0, 15).to(torch.uint8)
    out = torch.empty((N, nb, 18), dtype=torch.uint8, device=wf.device)
    out[:, :, 0:2] = d.to(torch.float16).reshape(N, nb, 1).view(torch.uint8)
    out[:, :, 2:18] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    return out.reshape(-1)


def dequantize_q4_0_np(w: np.ndarray, N: int, K: int) -> np.ndarray:
    nb = K // 32
    b = np.asarray(w, dtype=np.uint8).reshape(N, nb, 18)
    d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    nib = np.concatenate([b[:, :, 2:18] & 0x0F, b[:, :, 2:18] >> 4], axis=2).astype(np.float32)
    return ((nib - 8.0) * d[..., None]).reshape(N, K)
