"""Crafted inputs whose exact products sit just beside a rounding boundary.

A quantizer that lets the compiler fuse its multiply into the following add (one
fma instead of a rounded product, then an add) gives different bytes on exactly
these inputs; on random data that happens about once in 10^8 values.

* Q8_1 (q = roundf(fl(x * d_inv)), src/cuda/q8_1.cu:71-79): fl(x * d_inv) is a
  tie k + 0.5 (so roundf gives k + 1, away from zero) while the exact product is
  below it by enough that a fused round-away (trunc(x*d_inv + 0.49999997) in one
  rounding) gives k.
* Q4_0 (nib = (int)(fl(fl(v * id) + 8.5))): fl(v * id) + 8.5 is an integer n while
  the exact v * id + 8.5 rounds (once) to a value below n, so a fused form gives n - 1.

Exactness of the emulation: fp32 x fp32 products are exact in fp64 (48 bits), and
so are their sums with the constants used here (the span stays under 53 bits), so
one np.float32() of the fp64 value is the single rounding of an fma.
"""
from __future__ import annotations

import numpy as np

C_AWAY = np.float64(np.float32(0.49999997))  # 0.5 - 2^-25


def _neighbours(v0: np.ndarray, span: int) -> np.ndarray:
    """float32 values within `span` ulps of v0 (positive v0): shape [len(v0), 2*span+1]."""
    bits = v0.astype(np.float32).view(np.int32)[:, None] + np.arange(-span, span + 1, dtype=np.int32)[None, :]
    return bits.view(np.float32)


def q8_tie_cases(rng, n: int):
    """n tuples (A, v, k): with d_inv = fl(127/A), fl(v*d_inv) == k + 0.5 (0 < v < A),
    roundf gives k + 1 and the fused round-away gives k."""
    out = []
    while len(out) < n:
        A = rng.uniform(1.0, 2.0, 4096).astype(np.float32)
        D = (np.float32(127.0) / A).astype(np.float32)
        k = rng.integers(1, 126, 4096)
        v0 = ((k + 0.5) / D.astype(np.float64)).astype(np.float32)
        V = _neighbours(v0, 3)
        p = V.astype(np.float64) * D.astype(np.float64)[:, None]
        P = p.astype(np.float32)
        tie = P.astype(np.float64) == (k + 0.5)[:, None]
        fused = np.trunc((p + C_AWAY).astype(np.float32))
        bad = tie & (fused != (k + 1)[:, None]) & (V < A[:, None])
        for i, j in zip(*np.nonzero(bad)):
            out.append((np.float32(A[i]), np.float32(V[i, j]), int(k[i])))
            if len(out) == n:
                break
    return out


def q8_tie_input(K: int, seed: int):
    """x fp32 [K] (K % 32 == 0): group g holds one crafted value (random slot and
    sign) and its amax A at another slot; the rest are small.  Returns (x, slots,
    expected q at the slots)."""
    rng = np.random.default_rng(seed)
    G = K // 32
    cases = q8_tie_cases(rng, G)
    x = (rng.standard_normal(K) * 0.05).astype(np.float32)
    slots, qexp = [], []
    for g, (A, v, k) in enumerate(cases):
        a_slot, v_slot = rng.choice(32, 2, replace=False)
        sgn = np.float32(1.0 if rng.random() < 0.5 else -1.0)
        x[32 * g + a_slot] = A if rng.random() < 0.5 else -A
        x[32 * g + v_slot] = sgn * v
        slots.append(32 * g + v_slot)
        qexp.append(int(sgn) * (k + 1))
    return x, np.array(slots), np.array(qexp)


def q4_tie_cases(rng, n: int):
    """n tuples (mx, v, n_exact): d = fl(mx/-8), id = fl(1/d); fl(fl(v*id) + 8.5) is the
    integer n_exact while the fused fl(v*id + 8.5) truncates to n_exact - 1; |v| < |mx|."""
    out = []
    while len(out) < n:
        mx = rng.uniform(0.01, 1.0, 4096).astype(np.float32) * np.where(rng.random(4096) < 0.5, -1, 1).astype(np.float32)
        d = (mx / np.float32(-8.0)).astype(np.float32)
        idv = (np.float32(1.0) / d).astype(np.float32)
        nt = rng.integers(1, 5, 4096)                 # targets 1..4: fl(v*id) = nt - 8.5
        target = nt - 8.5
        v0 = np.abs((target / idv.astype(np.float64)).astype(np.float32))
        V = _neighbours(v0, 3) * np.sign(target / idv)[:, None].astype(np.float32)
        p = V.astype(np.float64) * idv.astype(np.float64)[:, None]
        P = p.astype(np.float32)
        two = (P.astype(np.float64) + 8.5).astype(np.float32)
        fused = (p + 8.5).astype(np.float32)
        bad = (two.astype(np.float64) == nt[:, None]) & (np.trunc(fused) != nt[:, None]) & \
            (np.abs(V) < np.abs(mx)[:, None])
        for i, j in zip(*np.nonzero(bad)):
            out.append((np.float32(mx[i]), np.float32(V[i, j]), int(nt[i])))
            if len(out) == n:
                break
    return out


def q4_tie_matrix(rows: int, cols: int, seed: int, per_block: int = 1):
    """fp32 [rows, cols]: every 32-block holds its max-magnitude value mx and
    `per_block` crafted values; returns (w, flat indices, expected nibbles)."""
    rng = np.random.default_rng(seed)
    nblk = rows * cols // 32
    cases = q4_tie_cases(rng, nblk)
    w = (rng.standard_normal(rows * cols) * 1e-3).astype(np.float32)
    idx, nib = [], []
    for b, (mx, v, nt) in enumerate(cases):
        slots = rng.choice(32, 1 + per_block, replace=False)
        w[32 * b + slots[0]] = mx
        for s in slots[1:]:
            w[32 * b + s] = v
            idx.append(32 * b + s)
            nib.append(nt)
    return w.reshape(rows, cols), np.array(idx), np.array(nib)
