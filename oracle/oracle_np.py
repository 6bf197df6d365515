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
* ``moe_top_k``          — moe_top_k_kernel<E, false, true>, src/cuda/moe/moe_top_k.cu:120-205,
                           softmax_warp_inplace :12-55, warp_reduce_xor_sum include/cuda_utils.cuh:37-43
* ``moe_dispatch``       — moe_dispatch_sota_launch_cuda, src/cuda/moe/moe_dispatch_sota.cu:113-151
                           (stable radix sort :127-136, lower-bound offsets :45-71, rows :73-95)
* ``swiglu``             — swiglu_silu_mul_kernel, src/cuda/swiglu.cu:5-14
* ``moe_combine``        — moe_combine_sota_unpermute_kernel, src/cuda/moe/moe_combine_sota.cu:21-41
* ``gather_q8_1``        — the dispatch row permutation applied to Q8_1 blocks
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


# ---------------------------------------------------------------- MoE routing
def _xor_butterfly_sum32(vals: np.ndarray) -> np.float32:
    """warp_reduce_xor_sum (include/cuda_utils.cuh:37-43) over 32 float32 lanes:
    offsets 16, 8, 4, 2, 1; lane 0's result."""
    x = np.asarray(vals, dtype=np.float32).copy()
    idx = np.arange(32)
    for off in (16, 8, 4, 2, 1):
        x = (x + x[idx ^ off]).astype(np.float32)
    return x[0]


def moe_top_k(logits: np.ndarray, top_k: int):
    """ids [T, top_k] (int32) and weights [T, top_k] (float32).

    Selection: top_k rounds over the remaining logits, each the largest value and
    the smallest expert id on ties (moe_top_k.cu:120-176).  Weights: softmax over
    the selected logits with max = the first selected, e = expf(v - max), the sum
    as the 32-lane xor butterfly with e in lanes 0..top_k-1, w = e * (1/sum)
    (moe_top_k.cu:12-55 with use_limit, :190-195).
    """
    lg = np.asarray(logits, dtype=np.float32)
    T, E = lg.shape
    ids = np.zeros((T, top_k), dtype=np.int32)
    wts = np.zeros((T, top_k), dtype=np.float32)
    for t in range(T):
        row = lg[t].copy()
        taken = np.zeros(E, dtype=bool)
        sel = []
        for k in range(top_k):
            best, best_id = np.float32(-np.inf), -1
            for e in range(E):
                v = np.float32(-np.inf) if taken[e] else row[e]
                if best_id < 0 or v > best:
                    best, best_id = v, e
            taken[best_id] = True
            ids[t, k] = best_id
            sel.append(best)
        sel = np.array(sel, dtype=np.float32)
        ex = np.exp((sel - sel[0]).astype(np.float32)).astype(np.float32)
        lanes = np.zeros(32, dtype=np.float32)
        lanes[:top_k] = ex
        inv = np.float32(1.0) / _xor_butterfly_sum32(lanes)
        wts[t] = (ex * inv).astype(np.float32)
    return ids, wts


def moe_dispatch(ids: np.ndarray, num_experts: int):
    """Stable sort of the routes r = t*top_k + k by expert.

    Returns (expert_offsets [E+1], src_route [R], dst_of_route [R]):
    src_route[p] = route at permuted row p, dst_of_route[r] = its row
    (moe_dispatch_sota.cu:113-151; inv_permuted_idx of moe_combine_sota.cu:6-19).
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    R = flat.size
    src = np.zeros(R, dtype=np.int32)
    counts = np.zeros(num_experts, dtype=np.int64)
    for e in flat:
        counts[e] += 1
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    cursor = offsets[:-1].astype(np.int64).copy()
    for r in range(R):  # routes in increasing r: stable
        e = flat[r]
        src[cursor[e]] = r
        cursor[e] += 1
    dst = np.zeros(R, dtype=np.int32)
    dst[src] = np.arange(R, dtype=np.int32)
    return offsets, src, dst


def gather_q8_1(xq: np.ndarray, src_route: np.ndarray, num_tokens: int, top_k: int, K: int) -> np.ndarray:
    """Q8_1 blocks of the permuted rows: block (s*R + p) = block (s*T + src_route[p] // top_k)."""
    R = src_route.size
    blocks = np.asarray(xq, dtype=np.uint8).reshape(K // SUPER, num_tokens, BLOCK_Q8_1_BYTES)
    return np.ascontiguousarray(blocks[:, np.asarray(src_route) // top_k, :]).reshape(-1)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(g) * u = g * (1 / (1 + exp(-g))) * u in float32, the reference's
    operation order (swiglu.cu:5-14)."""
    g = np.asarray(gate, dtype=np.float32)
    u = np.asarray(up, dtype=np.float32)
    one = np.float32(1.0)
    with np.errstate(over="ignore"):
        sig = (one / (one + np.exp(-g).astype(np.float32))).astype(np.float32)
    return ((g * sig).astype(np.float32) * u).astype(np.float32)


def moe_combine(expert_out: np.ndarray, dst_of_route: np.ndarray, weights: np.ndarray, top_k: int) -> np.ndarray:
    """y[t] = sum over k in order of w[t,k] * expert_out[dst(t,k)], float32, acc from 0
    with one rounding per multiply-add (fma, moe_combine_sota.cu:31-38)."""
    eo = np.asarray(expert_out, dtype=np.float32)
    w = np.asarray(weights, dtype=np.float32).reshape(-1)
    T = w.size // top_k
    y = np.zeros((T, eo.shape[1]), dtype=np.float32)
    for t in range(T):
        acc = np.zeros(eo.shape[1], dtype=np.float64)
        for k in range(top_k):
            r = t * top_k + k
            acc = (acc + np.float64(w[r]) * eo[dst_of_route[r]].astype(np.float64)).astype(np.float32).astype(np.float64)
        y[t] = acc.astype(np.float32)
    return y
