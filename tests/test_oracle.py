"""Pins of the CPU oracle (oracle/) against known answers, the reference's own
test, brute force and closed forms.  No GPU needed.

Each check is chosen so a plausible restatement mistake fails it:
  * rounding mode of q (ties away vs ties to even)        -> test_q_rounds_ties_away
  * zero group semantics (d = +inf, reference kernel)     -> test_zero_group
  * summation tree of s (intra-lane and cross-lane order) -> test_sum_tree_witnesses
  * d = fp16(1/(127/amax)) double rounding                -> test_d_exact_rational
  * block placement (superblock-major)                    -> test_block_layout
  * nibble pairing (j, j+16) / unsigned nibbles           -> test_block_sums_bruteforce
  * epilogue sign / factor 8 / scale operands             -> test_matmul_closed_forms
"""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
from fractions import Fraction

import numpy as np
import pytest

from oracle import c_oracle, oracle_np
from jjjetson_ops_amd import q4_0


# ---------------------------------------------------------------- fp16 helpers
def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([c_oracle.f16_bits_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    r = ref[::7]
    nan = np.isnan(r)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), r[~nan].view(np.uint32))


def test_f32_to_f16_rne_sweep():
    rng = np.random.default_rng(5)
    # magnitudes spanning subnormal..overflow, plus exact fp16 midpoints (ties)
    v = np.concatenate([
        (rng.standard_normal(20000) * np.exp2(rng.integers(-30, 18, 20000))).astype(np.float32),
        ((np.arange(1, 4000, dtype=np.float32) + 0.5) * np.float32(2 ** -10)),  # ties at scale 1
        ((np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2 ** -24)),  # ties in subnormals
        np.array([65504, 65519.99, 65520, 1e6, -1e6, 0.0, -0.0, 2 ** -25, 2 ** -26, 3 * 2 ** -26], np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    got = np.array([c_oracle.f32_to_f16_bits(float(x)) for x in v], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- quantizer
def _one_group(vals):
    x = np.zeros(128, np.float32)
    x[: len(vals)] = vals
    out = c_oracle.quantize_q8_1(x, [128, 1, 1, 1])
    qs, d, s = c_oracle.parse_q8_1(out, 1)
    dh = out[0:2].view(np.uint16)[0]
    sh = out[2:4].view(np.uint16)[0]
    return qs[0, :32], dh, sh, d[0, 0], s[0, 0]


def test_q_rounds_ties_away():
    # amax = 127 gives d_inv = 127/127 = 1 exactly, so q = roundf(x).
    vals = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 3.5, -126.5] + [0.0] * 24, np.float32)
    q, dh, *_ = _one_group(vals)
    assert list(q[:8]) == [127, 3, -3, 1, -1, 2, 4, -127]
    assert dh == np.float16(1.0).view(np.uint16)


def test_zero_group():
    q, dh, sh, d, s = _one_group(np.zeros(32, np.float32))
    assert np.all(q == 0)
    assert dh == 0x7C00  # 1/0 = +inf stored by the reference kernel
    assert sh == 0x0000
    assert np.isinf(d) and d > 0


def test_extremes_map_to_127():
    vals = np.full(32, -3.25, np.float32)
    vals[::2] = 3.25
    q, *_ = _one_group(vals)
    assert np.all(np.abs(q) == 127)
    assert np.all(q[::2] == 127) and np.all(q[1::2] == -127)


def _lanes(lane_vals):
    """Build a 32-group from 8 lanes of 4 values each."""
    return np.array(lane_vals, np.float32).reshape(32)


@pytest.mark.parametrize(
    "lanes, expected",
    [
        # cross-lane butterfly: ((t0+t4)+(t2+t6)) + ((t1+t5)+(t3+t7)) = 0 + 1 = 1;
        # a sequential t0+t1+... gives (2^25+1)->2^25, -2^25 -> 0.
        ([[2 ** 25, 0, 0, 0], [1, 0, 0, 0], [0] * 4, [0] * 4, [-(2 ** 25), 0, 0, 0], [0] * 4, [0] * 4, [0] * 4], 1.0),
        # intra-lane ((x0+x1)+x2)+x3: each +1 is absorbed (ties to even at 2^25), lane 4 cancels -> 0;
        # reversed order (1+1+1)+2^25 would give 2^25+4 -> 4.
        ([[2 ** 25, 1, 1, 1], [0] * 4, [0] * 4, [0] * 4, [-(2 ** 25), 0, 0, 0], [0] * 4, [0] * 4, [0] * 4], 0.0),
        # plain values: exact sum
        ([[1, 2, 3, 4], [5, 6, 7, 8], [0.5] * 4, [0.25] * 4, [-1] * 4, [0] * 4, [2] * 4, [-0.125] * 4], 42.5),
    ],
)
def test_sum_tree_witnesses(lanes, expected):
    _, _, sh, _, s = _one_group(_lanes(lanes))
    assert s == expected
    assert sh == np.float16(expected).view(np.uint16)


def test_d_exact_rational():
    """d bits == fp16(RN32(1 / RN32(127/amax))) computed with exact rationals."""
    rng = np.random.default_rng(11)
    amaxes = np.concatenate([
        np.abs(rng.standard_normal(300)).astype(np.float32) + np.float32(1e-3),
        np.array([1.0, 127.0, 3.0, 0.1, 1e-3, 60.0, 1e4], np.float32),
    ])

    def rn32(fr: Fraction) -> float:
        # exact rational -> nearest float32 (ties to even) via float64 then check
        f64 = float(fr)  # correctly rounded to binary64
        cand = np.float32(f64)
        # double rounding guard: pick the nearest float32 neighbour exactly
        best = None
        for c in (np.nextafter(cand, np.float32(-np.inf)), cand, np.nextafter(cand, np.float32(np.inf))):
            err = abs(Fraction(float(c)) - fr)
            if best is None or err < best[0] or (err == best[0] and (np.float32(c).view(np.uint32) & 1) == 0):
                best = (err, c)
        return float(best[1])

    for a in amaxes:
        vals = np.zeros(32, np.float32)
        vals[7] = a
        vals[3] = -a / 3
        _, dh, *_ = _one_group(vals)
        d_inv = rn32(Fraction(127) / Fraction(float(a)))
        d = rn32(Fraction(1) / Fraction(d_inv))
        assert dh == np.float16(np.float32(d)).view(np.uint16), a
        # and d is within one fp16 ulp of the mathematical amax/127
        assert abs(float(np.float16(np.float32(d))) - float(a) / 127) <= float(np.spacing(np.float16(float(a) / 127)))


def _q8_1_ref_restated(x):
    """The reference test's own expectation (tests/test_q8_1.py:5-62), restated:
    np.round (ties to even), fp32 d = 1/(127/amax), d=0 for a zero group,
    sum = float(group.sum()), block id = group*ne1 + j."""
    ne0, ne1 = x.shape[:2]
    n_sb = ne0 // 128
    qs = np.zeros((ne1 * n_sb, 128), np.int8)
    dr = np.zeros((ne1 * n_sb, 4), np.float32)
    sr = np.zeros((ne1 * n_sb, 4), np.float32)
    for j in range(ne1):
        for grp in range(n_sb):
            bid = grp * ne1 + j
            vals = x[grp * 128:(grp + 1) * 128, j, 0, 0]
            for g in range(4):
                v = vals[g * 32:(g + 1) * 32]
                amax = np.max(np.abs(v))
                d_inv = np.float32(127.0) / amax if amax > 0 else np.float32(0)
                dr[bid, g] = np.float32(1.0) / d_inv if amax > 0 else 0.0
                qs[bid, g * 32:(g + 1) * 32] = np.round(v * d_inv).astype(np.int8)
                sr[bid, g] = float(v.sum())
    return qs, dr, sr


def test_reference_q8_1_test_case():
    """tests/test_q8_1.py:65-123 with its tolerances: qs exact, d atol 1e-5, s atol 1e-2."""
    np.random.seed(24)
    x = np.asfortranarray(np.random.randn(2048, 13, 1, 1).astype(np.float32))
    out = c_oracle.quantize_q8_1(x, [2048, 13, 1, 1])
    assert out.size == 208 * 144
    qs, d, s = c_oracle.parse_q8_1(out, 208)
    qr, dr, sr = _q8_1_ref_restated(x)
    assert np.array_equal(qs, qr)
    assert np.allclose(d, dr, atol=1e-5)
    assert np.allclose(s, sr, atol=1e-2)


def test_reference_test_golden_fixture():
    """The committed fixture of the same input equals the oracle bytes."""
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "q8_1_seed24_2048x13.npz")
    np.random.seed(24)
    x = np.asfortranarray(np.random.randn(2048, 13, 1, 1).astype(np.float32))
    assert np.array_equal(c_oracle.quantize_q8_1(x, [2048, 13, 1, 1]), g["q8_1"])


def test_block_layout():
    """Block (k/128)*ne1 + m holds token m's values k..k+127 (src/cuda/q8_1.cu:85)."""
    K, T = 512, 3
    x = np.zeros((T, K), np.float32)
    for m in range(T):
        for sb in range(K // 128):
            x[m, sb * 128] = 100 * m + sb + 1  # marker at each superblock start
    out = c_oracle.quantize_q8_1(x, [K, T, 1, 1]).reshape(-1, 144)
    for m in range(T):
        for sb in range(K // 128):
            blk = out[sb * T + m]
            d = blk[0:2].view(np.float16)[0]
            s = blk[2:4].view(np.float16)[0]
            assert s == np.float16(100 * m + sb + 1)
            assert blk[16] == 127  # the marker is the amax of its group
            assert np.isfinite(d)


@pytest.mark.parametrize("dims", [[256, 5, 1, 1], [4096, 1, 1, 1], [160, 3, 1, 1], [640, 2, 2, 3], [96, 4, 3, 1]])
def test_numpy_oracle_equals_c_oracle(dims):
    rng = np.random.default_rng(sum(dims))
    n = int(np.prod(dims))
    x = rng.standard_normal(n).astype(np.float32)
    x[: dims[0] // 2] *= 20.0
    x[32:64] = 0.0  # a zero group
    x[64] = 0.5  # ties after scaling are rare; force amax=127 style group
    x[65:96] = np.float32(127.0) * 0 + 2.5
    x[64] = 127.0
    a = c_oracle.quantize_q8_1(x, dims)
    b = oracle_np.quantize_q8_1(x, dims)
    assert np.array_equal(a, b)


def test_q8_1_rejects_bad_k():
    with pytest.raises(ValueError):
        c_oracle.quantize_q8_1(np.zeros(48, np.float32), [48, 1, 1, 1])


# ---------------------------------------------------------------- matmul
def _rand_case(K, N, M, seed, outliers=False):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w = c_oracle.quantize_q4_0(wf)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        ch = rng.choice(K, max(1, K // 1000), replace=False)
        x[:, ch] *= 20
    xq = c_oracle.quantize_q8_1(x, [K, M, 1, 1])
    return wf, w, x, xq


def _brute_sumi(w, xq, K, N, M):
    nb = K // 32
    wb = w.reshape(N, nb, 18)
    xb = xq.reshape(-1, 144)
    out = np.zeros((M, N, nb), np.int64)
    for m in range(M):
        for n in range(N):
            for b in range(nb):
                blk = xb[(b // 4) * M + m]
                q = blk[16 + 32 * (b % 4): 16 + 32 * (b % 4) + 32].view(np.int8)
                s = 0
                for j in range(32):
                    byte = int(wb[n, b, 2 + (j % 16)])
                    nib = (byte & 0xF) if j < 16 else (byte >> 4)
                    s += nib * int(q[j])
                out[m, n, b] = s
    return out


def test_block_sums_bruteforce():
    K, N, M = 256, 5, 3
    _, w, _, xq = _rand_case(K, N, M, 1)
    bf = _brute_sumi(w, xq, K, N, M)
    assert np.array_equal(c_oracle.block_sums(w, xq, K, N, M), bf)
    assert np.array_equal(oracle_np.block_sums(w, xq, K, N, M), bf)


def test_block_sums_constant_nibbles():
    K, N, M = 128, 2, 2
    _, w, _, xq = _rand_case(K, N, M, 2)
    w = w.reshape(N, K // 32, 18).copy()
    w[0, :, 2:] = 0x77  # every nibble = 7
    w[1, :, 2:] = 0xF0  # low nibbles 0, high nibbles 15
    w = w.reshape(-1)
    qs, _, _ = oracle_np._split_x(xq, K, M)
    q = qs.reshape(M, K // 32, 32).astype(np.int64)
    got = c_oracle.block_sums(w, xq, K, N, M)
    assert np.array_equal(got[:, 0, :], 7 * q.sum(axis=2))
    assert np.array_equal(got[:, 1, :], 15 * q[:, :, 16:].sum(axis=2))


def test_matmul_textbook_single_block_row():
    """K=128, N=1, M=1: y = sum over 4 blocks of d_w*(d_x*sum(nib*q) - 8*s_x), by hand."""
    K = 128
    _, w, _, xq = _rand_case(K, 1, 1, 3)
    wb = w.reshape(4, 18)
    xb = xq.reshape(144)
    y = 0.0
    for b in range(4):
        dw = float(wb[b, 0:2].view(np.float16)[0])
        dx = float(xb[4 * b:4 * b + 2].view(np.float16)[0])
        sx = float(xb[4 * b + 2:4 * b + 4].view(np.float16)[0])
        q = xb[16 + 32 * b:48 + 32 * b].view(np.int8).astype(int)
        nib = [int(wb[b, 2 + j]) & 15 for j in range(16)] + [int(wb[b, 2 + j]) >> 4 for j in range(16)]
        y += dw * (dx * sum(n * qq for n, qq in zip(nib, q)) - 8 * sx)
    got = c_oracle.matmul(w, xq, K, 1, 1)[0, 0]
    assert abs(got - y) <= 1e-6 * max(1.0, abs(y))


def test_matmul_closed_forms():
    K, N, M = 256, 3, 2
    _, w, x, xq = _rand_case(K, N, M, 4)
    w = w.reshape(N, K // 32, 18).copy()
    w[:, :, 2:] = 0x88  # every nibble 8: weight value 0, y = 8*sum_b dw*(dx*sum q - sx)
    w = w.reshape(-1)
    y = c_oracle.matmul(w, xq, K, N, M)
    qs, dx, sx = oracle_np._split_x(xq, K, M)
    _, dw = oracle_np._split_w(w, N, K)
    sq = qs.reshape(M, K // 32, 32).astype(np.float64).sum(axis=2)
    exp = 8.0 * ((dx * sq - sx).astype(np.float64) @ dw.T.astype(np.float64))
    assert np.allclose(y, exp, rtol=1e-6, atol=1e-9)
    # ... and that residual is small but non-zero (s is fp16(sum x), not d*sum q)
    assert np.all(np.abs(exp) < 0.1)


@pytest.mark.parametrize("K,N,M", [(4096, 64, 1), (512, 40, 5)])
def test_matmul_matches_dequantized_dense(K, N, M):
    """y ~ dequant(W) . x within the quantisation error (the plumbing case's sanity check)."""
    wf, w, x, xq = _rand_case(K, N, M, 5)
    y = c_oracle.matmul(w, xq, K, N, M)
    wdq = q4_0.dequantize_q4_0_np(w, N, K).astype(np.float64)
    dense = x.astype(np.float64) @ wdq.T
    rel = np.linalg.norm(y - dense) / np.linalg.norm(dense)
    assert rel < 0.02, rel
    # the fp32 kernel-order evaluation agrees with the fp64 one at the parity tolerance
    y32 = c_oracle.matmul(w, xq, K, N, M, mode=1)
    assert np.allclose(y32, y, rtol=1e-3, atol=1e-4)
    assert np.allclose(oracle_np.matmul(w, xq, K, N, M), y, rtol=1e-6, atol=1e-6)
    assert np.allclose(oracle_np.matmul_fast(w, xq, K, N, M), y, rtol=1e-3, atol=1e-4)


def test_matmul_zero_activation_group_is_nan():
    """A zero activation group has d_x = +inf, so sumi*d_x = 0*inf = NaN (reference semantics)."""
    K, N, M = 128, 2, 1
    _, w, x, _ = _rand_case(K, N, M, 6)
    x[0, 32:64] = 0.0
    xq = c_oracle.quantize_q8_1(x, [K, M, 1, 1])
    y = c_oracle.matmul(w, xq, K, N, M)
    assert np.all(np.isnan(y))


# ---------------------------------------------------------------- Q4_0 packer
def test_q4_0_packer_matches_oracle_and_bounds():
    rng = np.random.default_rng(7)
    wf = (rng.standard_normal((33, 256)) * 0.02).astype(np.float32)
    wf[3, :32] = 0.0
    a = c_oracle.quantize_q4_0(wf)
    b = q4_0.quantize_q4_0_np(wf)
    assert np.array_equal(a, b)
    deq = q4_0.dequantize_q4_0_np(a, 33, 256)
    d = np.abs(a.reshape(33, 8, 18)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32))
    err = np.abs(deq - wf).reshape(33, 8, 32)
    # round-to-nearest (error <= d/2) except where the nibble clamps at 15 (w = -mx, error <= |d|);
    # plus the fp16 rounding of d scaled by |nib - 8| <= 8.
    slack = 8 * d[..., None] * 2 ** -10 + 1e-9
    nib = np.concatenate([a.reshape(33, 8, 18)[:, :, 2:] & 15, a.reshape(33, 8, 18)[:, :, 2:] >> 4], axis=2)
    bound = np.where(nib == 15, d[..., None], d[..., None] * 0.5) + slack
    assert np.all(err <= bound)


# ---------------------------------------------------------------- MoE routing oracle pins
def test_moe_top_k_selection_matches_stable_argsort():
    """ids = experts sorted by descending logit, smaller id first on ties: the same
    order as a stable argsort of -logits (a library routine)."""
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((40, 8)).astype(np.float32)
    lg[3] = 0.5  # all tied
    lg[4, [1, 5, 6]] = 2.0  # partial tie at the top
    for k in (1, 2, 3, 8):
        ids, _ = oracle_np.moe_top_k(lg, k)
        ref = np.argsort(-lg, axis=1, kind="stable")[:, :k]
        assert np.array_equal(ids, ref)


def test_moe_top_k_weights_are_softmax_of_selected():
    rng = np.random.default_rng(8)
    lg = (rng.standard_normal((50, 16)) * 3).astype(np.float32)
    for k in (1, 2, 4, 7):
        ids, w = oracle_np.moe_top_k(lg, k)
        sel = np.take_along_axis(lg, ids, 1).astype(np.float64)
        ex = np.exp(sel - sel.max(1, keepdims=True))
        np.testing.assert_allclose(w, ex / ex.sum(1, keepdims=True), rtol=2e-6, atol=1e-7)
    _, w1 = oracle_np.moe_top_k(lg, 1)
    assert np.all(w1 == 1.0)


def test_moe_top_k_sum_order_is_the_xor_butterfly():
    """With 3 values in lanes 0..2 the butterfly computes (e0 + e2) + e1.  Witness:
    e0 = 1, e1 = 2^-24, e2 = 1.5 * 2^-24 gives (e0+e2)+e1 = 1 + 2^-22, while
    (e0+e1)+e2 and e0+(e1+e2) both give 1 + 2^-23."""
    lanes = np.zeros(32, dtype=np.float32)
    e0, e1, e2 = np.float32(1.0), np.float32(2.0 ** -24), np.float32(1.5 * 2.0 ** -24)
    lanes[:3] = [e0, e1, e2]
    b = oracle_np._xor_butterfly_sum32(lanes)
    assert b == np.float32(1.0 + 2.0 ** -22)
    assert (e0 + e1) + e2 == np.float32(1.0 + 2.0 ** -23) and e0 + (e1 + e2) == np.float32(1.0 + 2.0 ** -23)
    for n in range(1, 33):
        v = np.zeros(32, dtype=np.float32)
        v[:n] = 1.0
        assert oracle_np._xor_butterfly_sum32(v) == n


def test_moe_dispatch_is_a_stable_sort():
    rng = np.random.default_rng(9)
    for T, k, E in ((64, 2, 8), (7, 1, 4), (100, 4, 16), (3, 3, 3)):
        ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
        off, src, dst = oracle_np.moe_dispatch(ids, E)
        flat = ids.reshape(-1)
        assert np.array_equal(src, np.argsort(flat, kind="stable"))
        assert np.array_equal(off, np.searchsorted(np.sort(flat), np.arange(E + 1), side="left"))
        assert np.array_equal(dst[src], np.arange(T * k))


def test_gather_q8_1_bruteforce():
    rng = np.random.default_rng(10)
    T, k, K = 5, 2, 256
    xq = rng.integers(0, 256, size=T * K // 128 * 144).astype(np.uint8)
    src = rng.permutation(T * k).astype(np.int32)
    got = oracle_np.gather_q8_1(xq, src, T, k, K).reshape(K // 128, T * k, 144)
    blocks = xq.reshape(K // 128, T, 144)
    for s in range(K // 128):
        for p in range(T * k):
            assert np.array_equal(got[s, p], blocks[s, src[p] // k])


def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 4.5], dtype=np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0, -0.5], dtype=np.float32)
    got = oracle_np.swiglu(g, u).astype(np.float64)
    exact = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(got, exact, rtol=1e-6, atol=1e-30)
    assert got[0] == 0.0 and got[3] == 30.0  # silu(0) = 0, silu(30) = 30 in fp32


def test_moe_combine_closed_forms():
    rng = np.random.default_rng(11)
    T, k, H = 6, 3, 16
    eo = rng.standard_normal((T * k, H)).astype(np.float32)
    dst = rng.permutation(T * k).astype(np.int32)
    w = rng.random(T * k).astype(np.float32)
    y = oracle_np.moe_combine(eo, dst, w, k)
    ref = np.stack([sum(np.float64(w[t * k + j]) * eo[dst[t * k + j]].astype(np.float64) for j in range(k))
                    for t in range(T)])
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-7)
    # top_k = 1 and weight 1: the inverse permutation, exactly
    y1 = oracle_np.moe_combine(eo, dst, np.ones(T * k, np.float32), 1)
    assert np.array_equal(y1, eo[dst])


def test_q8_1_tie_inputs_pin_the_rounded_product():
    """q = roundf(fl(x * d_inv)) (src/cuda/q8_1.cu:71-79): on crafted values whose
    rounded product is a tie k + 0.5, the oracle gives k + 1 (away from zero), while
    a fused round-away (the product left unrounded) would give k."""
    from _ties import q8_tie_input, C_AWAY
    K = 1024
    x, slots, qexp = q8_tie_input(K, seed=21)
    qs, d, s = c_oracle.parse_q8_1(c_oracle.quantize_q8_1(x.reshape(1, K), [K, 1]), K // 128)
    q = qs.reshape(-1)
    assert np.array_equal(q[slots].astype(np.int64), qexp)
    g = x.reshape(-1, 32)
    dinv = (np.float32(127.0) / np.abs(g).max(axis=1)).astype(np.float32)
    p = x[slots].astype(np.float64) * dinv[slots // 32].astype(np.float64)
    fused = np.trunc((p + np.sign(p) * C_AWAY).astype(np.float32)).astype(np.int64)
    assert np.all(np.abs(fused - qexp) == 1)


def test_config1_plumbing_oracle_against_dequantized_product():
    """Benchmark configuration 1 (M=1, K=N=4096, seed 0) on the CPU path: the oracle's y differs
    from the dequantized product (dequant W).(dequant x) only by the reference's sum
    term, 8*d_w*(d_x*sum(q) - s) per block, and tracks the unquantized fp32 W.x at the
    quantization level."""
    K = N = 4096
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, K)).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w = c_oracle.quantize_q4_0(wf)
    xq = c_oracle.quantize_q8_1(x, [K, 1])
    y = c_oracle.matmul(w, xq, K, N, 1)[0].astype(np.float64)
    qs, d, s = c_oracle.parse_q8_1(xq, K // 128)
    qs = qs.reshape(-1).astype(np.float64)
    dx = d.reshape(-1).astype(np.float64)
    sx = s.reshape(-1).astype(np.float64)
    wdeq = q4_0.dequantize_q4_0_np(w, N, K).astype(np.float64)
    dw = w.reshape(N, K // 32, 18)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    corr = 8.0 * dw @ (dx * qs.reshape(-1, 32).sum(axis=1) - sx)
    deq = wdeq @ (qs * np.repeat(dx, 32))
    # exact identity up to fp32 evaluation error of y
    np.testing.assert_allclose(y, deq + corr, rtol=1e-5, atol=1e-5)
    assert np.abs(corr).max() > 1e-6  # the sum term is really there
    dense = wf.astype(np.float64) @ x[0].astype(np.float64)
    assert np.linalg.norm(y - dense) / np.linalg.norm(dense) < 0.15
