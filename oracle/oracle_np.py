"""Vectorised NumPy oracle — TEST INFRASTRUCTURE ONLY.

Restates the reference's Q8_1 quantizer and Q4_0 x Q8_1 matmul
(AshburnLee/JJJetson_Ops) with NumPy array arithmetic.  It is the checker the
parity tests and bench.py's ``cpu_baseline`` leg use; the product package never
imports it.  It must agree bit-for-bit with ``q4q8_oracle.c`` (pinned in
tests/test_oracle.py), which in turn is pinned against known answers.

Functions and the reference lines they follow:

* ``quantize_q8_1``      — quantize_q8_1_kernel, src/cuda/q8_1.cu:40-103, layout :84-87
* ``parse_q8_1``         — parse_q8_1_output,    src/cuda/q8_1.cu:197-216
* ``block_sums``         — q4_0_q8_1_vec_dot_impl integer part, src/cuda/mm_q4_0_q8_1.cu:75-90
* ``matmul``             — per-block epilogue :91-92 summed over K (:256-269)
* ``quantize_q4_0``      — this build's weight generator (the reference has none)
"""
from __future__ import annotations

import numpy as np

QK = 32
SUPER = 128
BLOCK_Q8_1_BYTES = 144
BLOCK_Q4_0_BYTES = 18


def _round_half_away(v: np.ndarray) -> np.ndarray:
    """roundf semantics (ties away from zero) on float32 input, exactly."""
    r = np.round(v)  # ties to even
    frac = v - np.trunc(v)  # exact for binary floats
    tie = np.abs(frac) == np.float32(0.5)
    return np.where(tie, np.trunc(v) + np.sign(v), r)


def n_q8_1_blocks(dims) -> int:
    K, ne1, ne2, ne3 = (list(dims) + [1, 1, 1])[:4]
    nz = ne2 * ne3
    if nz <= 1:
        return ne1 * ((K + 127) // 128)
    return nz * ne1 * 4 * ((K + 511) // 512)


def quantize_groups(xg: np.ndarray):
    """xg: float32 [..., 32] groups.  Returns (q int8 [...,32], d_f16 [...], s_f16 [...])."""
    xg = np.ascontiguousarray(xg, dtype=np.float32)
    lanes = xg.reshape(xg.shape[:-1] + (8, 4))
    a = np.abs(lanes)
    lane_max = np.maximum(a[..., 0], np.maximum(a[..., 1], np.maximum(a[..., 2], a[..., 3])))
    lane_sum = ((lanes[..., 0] + lanes[..., 1]) + lanes[..., 2]) + lanes[..., 3]
    for off in (4, 2, 1):
        idx = np.arange(8) ^ off
        lane_max = np.maximum(lane_max, lane_max[..., idx])
        lane_sum = lane_sum + lane_sum[..., idx]
    amax = lane_max[..., 0]
    ssum = lane_sum[..., 0]
    with np.errstate(divide="ignore", invalid="ignore"):
        d_inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
        q = _round_half_away((xg * d_inv[..., None]).astype(np.float32)).astype(np.int8)
        d = (np.float32(1.0) / d_inv).astype(np.float32).astype(np.float16)
    s = ssum.astype(np.float16)
    return q, d, s


def quantize_q8_1(x: np.ndarray, dims) -> np.ndarray:
    """x: float32 with dim0 fastest, dims [K, ne1, ne2, ne3].  Returns uint8 blocks."""
    K, ne1, ne2, ne3 = (list(dims) + [1, 1, 1])[:4]
    assert K % 32 == 0
    nz = ne2 * ne3
    flat = np.ravel(np.asarray(x, dtype=np.float32), order="K")
    xs = flat.reshape(nz, ne1, K)
    n_super = (K + 127) // 128
    slice_blocks = ne1 * 4 * ((K + 511) // 512)
    out = np.zeros((n_q8_1_blocks(dims), BLOCK_Q8_1_BYTES), dtype=np.uint8)
    ng = K // 32
    q, d, s = quantize_groups(xs.reshape(nz, ne1, ng, 32))
    for sb in range(n_super):
        g_lo, g_hi = 4 * sb, min(4 * sb + 4, ng)
        cnt = g_hi - g_lo
        rows = (np.arange(nz)[:, None] * slice_blocks + sb * ne1 + np.arange(ne1)[None, :]).reshape(-1)
        qq = q[:, :, g_lo:g_hi, :].reshape(nz * ne1, cnt * 32)
        out[rows, 16:16 + 32 * cnt] = qq.view(np.uint8)
        ds = np.stack([d[:, :, g_lo:g_hi], s[:, :, g_lo:g_hi]], axis=-1)  # [nz,ne1,cnt,2] f16
        out[rows, 0:4 * cnt] = ds.reshape(nz * ne1, cnt * 2).view(np.uint8).reshape(nz * ne1, 4 * cnt)
    return out.reshape(-1)


def parse_q8_1(raw: np.ndarray, n_blocks: int):
    b = np.asarray(raw, dtype=np.uint8).reshape(-1)[: n_blocks * 144].reshape(n_blocks, 144)
    qs = b[:, 16:].view(np.int8).copy()
    ds = b[:, :16].copy().view(np.float16).reshape(n_blocks, 4, 2).astype(np.float32)
    return qs, ds[:, :, 0].copy(), ds[:, :, 1].copy()


def _split_x(xq: np.ndarray, K: int, M: int):
    """Quantizer-layout activation -> q int8 [M, K], d f32 [M, K/32], s f32 [M, K/32]."""
    n_super = K // 128
    b = np.asarray(xq, dtype=np.uint8).reshape(-1)[: n_super * M * 144].reshape(n_super, M, 144)
    q = b[:, :, 16:].view(np.int8).transpose(1, 0, 2).reshape(M, K)
    ds = b[:, :, :16].copy().view(np.float16).reshape(n_super, M, 4, 2).transpose(1, 0, 2, 3)
    ds = ds.reshape(M, K // 32, 2).astype(np.float32)
    return q, ds[:, :, 0], ds[:, :, 1]


def _split_w(w: np.ndarray, N: int, K: int):
    """Q4_0 rows -> unsigned nibbles uint8 [N, K], d f32 [N, K/32]."""
    nb = K // 32
    b = np.asarray(w, dtype=np.uint8).reshape(-1)[: N * nb * 18].reshape(N, nb, 18)
    d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    qs = b[:, :, 2:18]
    nib = np.concatenate([qs & 0x0F, qs >> 4], axis=2).reshape(N, K)
    return nib, d


def block_sums(w: np.ndarray, xq: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
    """int32 [M, N, K/32]: sum_j nib_j * q_j per 32-block (unsigned nibbles)."""
    assert K % 128 == 0
    nib, _ = _split_w(w, N, K)
    q, _, _ = _split_x(xq, K, M)
    nb = K // 32
    out = np.empty((M, N, nb), dtype=np.int32)
    ni = nib.reshape(N, nb, 32).astype(np.int32)
    qi = q.reshape(M, nb, 32).astype(np.int32)
    for b in range(nb):
        out[:, :, b] = qi[:, b, :] @ ni[:, b, :].T
    return out


def matmul(w: np.ndarray, xq: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
    """fp32 y [M, N] = sum_b dw*(sumi*dx - 8*sx), evaluated in fp64 then rounded once."""
    assert K % 128 == 0
    nib, dw = _split_w(w, N, K)
    q, dx, sx = _split_x(xq, K, M)
    nb = K // 32
    ni = nib.reshape(N, nb, 32).astype(np.float64)
    qf = q.reshape(M, nb, 32).astype(np.float64)
    dw64 = dw.astype(np.float64)
    y = np.zeros((M, N), dtype=np.float64)
    for b in range(nb):
        sumi = qf[:, b, :] @ ni[:, b, :].T  # exact (integers < 2^53)
        y += (sumi * dx[:, b, None].astype(np.float64) - 8.0 * sx[:, b, None].astype(np.float64)) * dw64[None, :, b]
    return y.astype(np.float32)


def matmul_fast(w: np.ndarray, xq: np.ndarray, K: int, N: int, M: int) -> np.ndarray:
    """Same contraction as ``matmul`` but batched over blocks with BLAS (fp64).

    Used as the CPU baseline's timed kernel: y = sum_b dw_b*dx_b*(Q_b N_b^T) - 8*(sx @ dw^T).
    """
    nib, dw = _split_w(w, N, K)
    q, dx, sx = _split_x(xq, K, M)
    nb = K // 32
    ni = nib.reshape(N, nb, 32).transpose(1, 2, 0).astype(np.float32)  # [nb, 32, N]
    qf = q.reshape(M, nb, 32).transpose(1, 0, 2).astype(np.float32)  # [nb, M, 32]
    sumi = np.matmul(qf, ni)  # [nb, M, N] exact in fp32 (|sumi| < 2^24)
    t = sumi * dx.T[:, :, None] * dw.T[:, None, :]
    y = t.astype(np.float64).sum(axis=0) - 8.0 * (sx.astype(np.float64) @ dw.astype(np.float64).T)
    return y.astype(np.float32)


def quantize_q4_0(wf: np.ndarray) -> np.ndarray:
    """fp32 [N, K] -> Q4_0 bytes (ggml-style: d = signed-max/-8, nib = min(15, int(w/d + 8.5)))."""
    wf = np.asarray(wf, dtype=np.float32)
    N, K = wf.shape
    nb = K // 32
    g = wf.reshape(N, nb, 32)
    idx = np.argmax(np.abs(g), axis=2)
    mx = np.take_along_axis(g, idx[..., None], axis=2)[..., 0]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (g * idv[..., None]).astype(np.float32) + np.float32(8.5)
    nib = np.clip(np.trunc(v.astype(np.float32)), 0, 15).astype(np.uint8)
    out = np.zeros((N, nb, 18), dtype=np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).reshape(N, nb, 1).view(np.uint8)
    out[:, :, 2:18] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    return out.reshape(-1)


def dequantize_q4_0(w: np.ndarray, N: int, K: int) -> np.ndarray:
    nib, d = _split_w(w, N, K)
    return ((nib.astype(np.float32) - 8.0).reshape(N, K // 32, 32) * d[..., None]).reshape(N, K)
