"""Every benchmark configuration of the path at its full size and seed, HIP path against the oracle.

  config 1  plumbing: M=1, K=4096, N=4096, seed 0 (x and W from one generator);
            full oracle compare through both device entries, plus a bound against
            the dequantized fp32 product that the oracle itself does not enter
  config 2  M=1 decode, K=4096->N=11008 and K=11008->N=4096, weights seed 1,
            quantized on device each call (the fused entry): every output checked
  config 3  M in {4, 8, 16}, K=4096, N=14336, weights seed 2, through AUTO, and through
            the split weight layout (repacked on the device)
  config 5  8 experts, top-2 of N(0,1) router logits [512, 8] (seed 4), 512 tokens,
            K=4096 -> N=14336 in ONE grouped launch, outputs scattered per route;
            and the whole Q4_0 MoE FFN of that layer (I=14336) stage by stage

Large outputs are checked through exact sub-problems: the oracle evaluates a
random subset of output rows for a subset of tokens (or routes), always including
each expert's first and last route and the routes on both sides of every 128-route
tile boundary (bench.py times the same shapes; config 4, M=2048, is covered in
test_gpu_parity.py).  Bars as everywhere: Q8_1 bytes and routing tables exact,
fp32 outputs rtol 1e-3 / atol 1e-4 against the fp64-accumulating oracle.
"""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import sys

import numpy as np
import pytest

from jjjetson_ops_amd import capi
from oracle import c_oracle, oracle_np

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def outlier_x(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, max(1, K // 1000), replace=False)] *= 20
    return x


def dev_weights(N, K, seed, dev):
    """Q4_0 weights of N(0, 0.02) fp32 drawn on the device (seeded) and packed by the
    gfx950 quantizer, which is bit-exact with the oracle's packer
    (test_gpu_weights.py); returns (device bytes, host bytes)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    wf = torch.randn(N, K, generator=g, device=dev) * 0.02
    w = torch.empty(N * (K // 32) * 18, dtype=torch.uint8, device=dev)
    from jjjetson_ops_amd import weights
    weights.quantize_q4_0_device(wf, w, N, K)
    del wf
    return w, host(w)


def sub_weights(w_host, rows, K):
    nb = K // 32
    return np.ascontiguousarray(w_host.reshape(-1, nb * 18)[rows]).reshape(-1)


def sub_q8_1(xq_host, toks, K, M):
    return np.ascontiguousarray(xq_host.reshape(K // 128, M, 144)[:, toks]).reshape(-1)


# ------------------------------------------------------------------ config 1
def test_config1_plumbing_full(dev):
    import torch
    K = N = 4096
    note("config 1: M=1 K=4096 N=4096 seed 0")
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, K)).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w = c_oracle.quantize_q4_0(wf)
    xq_ref = c_oracle.quantize_q8_1(x, [K, 1])
    y_ref = c_oracle.matmul(w, xq_ref, K, N, 1)

    # fused quantize + GEMV entry
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x, dev), xq, y, K, N, 1)
    assert np.array_equal(host(xq), xq_ref)
    np.testing.assert_allclose(host(y).reshape(1, N), y_ref, rtol=RTOL, atol=ATOL)
    # standalone quantizer + AUTO matmul
    xq2 = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(to_dev(x, dev), xq2, [K, 1])
    y2 = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul(to_dev(w, dev), xq2, y2, K, N, 1)
    assert np.array_equal(host(xq2), xq_ref)
    got = host(y2).reshape(1, N)
    np.testing.assert_allclose(got, y_ref, rtol=RTOL, atol=ATOL)

    # The dequantized product differs from the reference formula only by the sum
    # term: d_w*(d_x*sumi - 8*s) = (dequant W).(dequant x) + 8*d_w*(d_x*sum(q) - s).
    from jjjetson_ops_amd import q4_0
    qs, d, s = c_oracle.parse_q8_1(xq_ref, K // 128)
    qs = qs.reshape(-1).astype(np.float64)
    dx = d.reshape(-1).astype(np.float64)
    sx = s.reshape(-1).astype(np.float64)
    xdeq = qs * np.repeat(dx, 32)
    wdeq = q4_0.dequantize_q4_0_np(w, N, K).astype(np.float64)
    dw = w.reshape(N, K // 32, 18)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    sum_q = qs.reshape(-1, 32).sum(axis=1)
    bound = 8.0 * np.abs(dw) @ np.abs(dx * sum_q - sx) + 1e-4 + 1e-5 * np.abs(wdeq) @ np.abs(xdeq)
    assert np.all(np.abs(got[0] - wdeq @ xdeq) <= bound)
    # and it tracks the unquantized fp32 product at the quantization level
    dense = wf.astype(np.float64) @ x[0].astype(np.float64)
    rel = np.linalg.norm(got[0] - dense) / np.linalg.norm(dense)
    assert rel < 0.15, rel


# ------------------------------------------------------------------ config 2
@pytest.mark.parametrize("K,N", [(4096, 11008), (11008, 4096)])
def test_config2_decode_full(K, N, dev):
    import torch
    note(f"config 2: M=1 K={K} N={N} seed 1, fused entry, every output")
    w_d, w = dev_weights(N, K, 1, dev)
    x = outlier_x(np.random.default_rng(11), 1, K)
    xq_ref = c_oracle.quantize_q8_1(x, [K, 1])
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_f32(w_d, to_dev(x, dev), xq, y, K, N, 1)
    assert np.array_equal(host(xq), xq_ref)
    np.testing.assert_allclose(host(y).reshape(1, N), c_oracle.matmul(w, xq_ref, K, N, 1), rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------ config 3
@pytest.mark.parametrize("M", [4, 8, 16])
def test_config3_small_batch(M, dev):
    import torch
    K, N = 4096, 14336
    note(f"config 3: M={M} K={K} N={N} seed 2, AUTO")
    w_d, w = dev_weights(N, K, 2, dev)
    x = outlier_x(np.random.default_rng(20 + M), M, K)
    xq_d = torch.zeros(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(to_dev(x, dev), xq_d, [K, M])
    xq = host(xq_d)
    assert np.array_equal(xq, c_oracle.quantize_q8_1(x, [K, M]))
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul(w_d, xq_d, y, K, N, M)
    got = host(y).reshape(M, N)
    rng = np.random.default_rng(M)
    rows = np.unique(np.concatenate([rng.choice(N, 1500, replace=False), [0, 15, 16, 31, 32, N - 1]]))
    exp = c_oracle.matmul(sub_weights(w, rows, K), xq, K, rows.size, M)
    np.testing.assert_allclose(got[:, rows], exp, rtol=RTOL, atol=ATOL)
    # the same weights repacked into the split layout on the device, through the
    # split entry with the fp32 activation (quantize + matmul)
    ws = torch.empty_like(w_d)
    capi.q4_0_to_split(w_d, ws, N, K)
    xq2 = torch.zeros_like(xq_d)
    y2 = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split_f32(ws, to_dev(x, dev), xq2, y2, K, N, M)
    assert np.array_equal(host(xq2), xq)
    np.testing.assert_allclose(host(y2).reshape(M, N)[:, rows], exp, rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------ config 5
E5, T5, TOPK5, H5, I5 = 8, 512, 2, 4096, 14336


def _routing(dev):
    """Router logits N(0,1) [512, 8] from seed 4; routes, tables and weights from the
    pinned oracle (top-k by value, smaller id on ties; stable sort by expert), and the
    device routing entries must give the same tables."""
    import torch
    lg = np.random.default_rng(4).standard_normal((T5, E5)).astype(np.float32)
    ids, rw = oracle_np.moe_top_k(lg, TOPK5)
    off, src, dst = oracle_np.moe_dispatch(ids, E5)
    R = T5 * TOPK5
    rw_d = torch.empty(R, dtype=torch.float32, device=dev)
    ids_d = torch.empty(R, dtype=torch.int32, device=dev)
    capi.moe_top_k(to_dev(lg, dev), rw_d, ids_d, T5, E5, TOPK5)
    assert np.array_equal(host(ids_d), ids.reshape(-1))
    np.testing.assert_allclose(host(rw_d), rw.reshape(-1), rtol=2e-6)
    off_d = torch.empty(E5 + 1, dtype=torch.int32, device=dev)
    src_d = torch.empty(R, dtype=torch.int32, device=dev)
    dst_d = torch.empty(R, dtype=torch.int32, device=dev)
    capi.moe_dispatch(ids_d, off_d, src_d, dst_d, T5, TOPK5, H5, E5)
    assert np.array_equal(host(off_d), off)
    assert np.array_equal(host(src_d), src)
    assert np.array_equal(host(dst_d), dst)
    counts = np.diff(off)
    assert counts.min() != counts.max(), "seed 4 gives uneven expert loads"
    return lg, ids, rw, off, src, dst


def _route_sample(off, e, rng, n=12):
    """Routes of expert e to check: first, last, both sides of each 128-route tile
    boundary inside the expert, and a few random ones (indices into the sorted rows)."""
    beg, end = int(off[e]), int(off[e + 1])
    if end == beg:
        return np.zeros(0, dtype=np.int64)
    pick = [beg, end - 1]
    for b in range(beg + 128, end, 128):
        pick += [b - 1, b]
    pick += list(rng.integers(beg, end, size=min(n, end - beg)))
    return np.unique(np.array(pick, dtype=np.int64))


def test_config5_grouped_full_size(dev):
    """One grouped launch over all 8 experts; y row of route r at dst(r)."""
    import torch
    note("config 5: grouped E=8 top-2 T=512 K=4096 N=14336 (one launch)")
    K, N = H5, I5
    _, _, _, off, src, dst = _routing(dev)
    R = T5 * TOPK5
    x = outlier_x(np.random.default_rng(45), T5, K)
    xr = x[src // TOPK5]                        # permuted rows, sorted by expert
    xq_d = torch.zeros(capi.q8_1_output_bytes([K, R]), dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(to_dev(xr, dev), xq_d, [K, R])
    xq = host(xq_d)
    ws = [dev_weights(N, K, 40 + e, dev) for e in range(E5)]
    w_all = torch.cat([wd for wd, _ in ws])
    y = torch.full((R * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(w_all, xq_d, to_dev(off, dev), y, K, N, R, route_dst=to_dev(src.astype(np.int32), dev))
    got = host(y).reshape(R, N)
    assert not np.isnan(got).any(), "a route's output row was never written"
    rng = np.random.default_rng(5)
    for e in range(E5):
        rows_p = _route_sample(off, e, rng)
        if rows_p.size == 0:
            continue
        note(f"  expert {e}: {off[e + 1] - off[e]} routes, checking {rows_p.size}")
        assert np.array_equal(sub_q8_1(xq, rows_p, K, R), c_oracle.quantize_q8_1(xr[rows_p], [K, rows_p.size]))
        cols = np.unique(np.concatenate([rng.choice(N, 160, replace=False), [0, 127, 128, N - 1]]))
        exp = c_oracle.matmul(sub_weights(ws[e][1], cols, K), sub_q8_1(xq, rows_p, K, R), K, cols.size, rows_p.size)
        np.testing.assert_allclose(got[np.ix_(src[rows_p], cols)], exp, rtol=RTOL, atol=ATOL)


def test_config5_moe_ffn_full_size(dev):
    """The whole FFN (H=4096, I=14336) through its one entry equals the stage entries
    bit for bit; each stage is checked against the oracle (tables, gather and SwiGLU
    quantization exactly, matmuls on sub-problems, combine in full), and sampled tokens
    run through the whole oracle chain."""
    import torch
    note("config 5: MoE FFN E=8 top-2 T=512 H=4096 I=14336")
    T, H, I, E, k = T5, H5, I5, E5, TOPK5
    R = T * k
    lg, ids, rw, off, src, dst = _routing(dev)
    x = outlier_x(np.random.default_rng(46), T, H)
    wg = [dev_weights(I, H, 60 + e, dev) for e in range(E)]
    wu = [dev_weights(I, H, 70 + e, dev) for e in range(E)]
    wdn = [dev_weights(H, I, 80 + e, dev) for e in range(E)]
    d_wg = torch.cat([a for a, _ in wg])
    d_wu = torch.cat([a for a, _ in wu])
    d_wd = torch.cat([a for a, _ in wdn])
    d_x, d_lg = to_dev(x, dev), to_dev(lg, dev)

    ws = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, k), dtype=torch.uint8, device=dev)
    y = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
    capi.moe_ffn(d_x, d_lg, d_wg, d_wu, d_wd, y, T, H, I, E, k, ws)
    y_ffn = host(y).reshape(T, H)
    assert np.isfinite(y_ffn).all()

    # stages through their own entries
    rw_d = torch.empty(R, dtype=torch.float32, device=dev)
    ids_d = torch.empty(R, dtype=torch.int32, device=dev)
    capi.moe_top_k(d_lg, rw_d, ids_d, T, E, k)
    xq_d = torch.empty(T * H // 128 * 144, dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(d_x, xq_d, [H, T])
    off_d = torch.empty(E + 1, dtype=torch.int32, device=dev)
    src_d = torch.empty(R, dtype=torch.int32, device=dev)
    dst_d = torch.empty(R, dtype=torch.int32, device=dev)
    xp_d = torch.empty(R * H // 128 * 144, dtype=torch.uint8, device=dev)
    capi.moe_dispatch(ids_d, off_d, src_d, dst_d, T, k, H, E, xq=xq_d, xq_perm=xp_d)
    gu_d = torch.empty(R * 2 * I, dtype=torch.float32, device=dev)
    capi.moe_gate_up(d_wg, d_wu, xp_d, off_d, E, gu_d, H, I, R)
    mq_d = torch.empty(R * I // 128 * 144, dtype=torch.uint8, device=dev)
    mid_d = torch.empty(R * I, dtype=torch.float32, device=dev)
    capi.swiglu_quantize(gu_d, mq_d, R, I, mid_f32=mid_d)
    # the fused gate|up + SwiGLU + Q8_1 launch the FFN entry runs: the same bytes
    mq_f = torch.empty_like(mq_d)
    capi.moe_gate_up_swiglu(d_wg, d_wu, xp_d, off_d, E, mq_f, H, I, R)
    assert torch.equal(mq_f, mq_d)
    eo_d = torch.empty(R * H, dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(d_wd, mq_d, off_d, eo_d, I, H, R)
    y2 = torch.empty(T * H, dtype=torch.float32, device=dev)
    capi.moe_combine(eo_d, dst_d, rw_d, y2, T, H, k)
    assert np.array_equal(y_ffn, host(y2).reshape(T, H))

    # quantize + gather: exact
    xq = host(xq_d)
    assert np.array_equal(xq, c_oracle.quantize_q8_1(x, [H, T]))
    xp = host(xp_d)
    assert np.array_equal(xp, oracle_np.gather_q8_1(xq, src, T, k, H))
    # gate|up on sub-problems of every expert (gate half and up half)
    gu = host(gu_d).reshape(R, 2 * I)
    rng = np.random.default_rng(7)
    for e in range(E):
        rows_p = _route_sample(off, e, rng, n=6)
        if rows_p.size == 0:
            continue
        xs = sub_q8_1(xp, rows_p, H, R)
        cols = np.unique(np.concatenate([rng.choice(I, 96, replace=False), [0, I - 1]]))
        for half, wexp in ((0, wg[e][1]), (1, wu[e][1])):
            exp = c_oracle.matmul(sub_weights(wexp, cols, H), xs, H, cols.size, rows_p.size)
            np.testing.assert_allclose(gu[np.ix_(rows_p, half * I + cols)], exp, rtol=RTOL, atol=ATOL)
    # SwiGLU: fp32 values within 2 ulp-ish of the oracle, Q8_1 bytes exact given them
    mid = host(mid_d).reshape(R, I)
    np.testing.assert_allclose(mid, oracle_np.swiglu(gu[:, :I], gu[:, I:]), rtol=2e-6, atol=1e-30)
    mq = host(mq_d)
    assert np.array_equal(mq, c_oracle.quantize_q8_1(mid, [I, R]))
    # down projection on sub-problems
    eo = host(eo_d).reshape(R, H)
    for e in range(E):
        rows_p = _route_sample(off, e, rng, n=6)
        if rows_p.size == 0:
            continue
        cols = np.unique(np.concatenate([rng.choice(H, 96, replace=False), [0, H - 1]]))
        exp = c_oracle.matmul(sub_weights(wdn[e][1], cols, I), sub_q8_1(mq, rows_p, I, R), I, cols.size,
                              rows_p.size)
        np.testing.assert_allclose(eo[np.ix_(rows_p, cols)], exp, rtol=RTOL, atol=ATOL)
    # combine: in full
    np.testing.assert_allclose(y_ffn, oracle_np.moe_combine(eo, dst, rw.reshape(-1), k), rtol=1e-6, atol=1e-6)

    # whole oracle chain for a few tokens (fp64-accumulating matmuls, re-quantized
    # SwiGLU output: the end-to-end bar of the FFN tests)
    for t in (0, 137, T - 1):
        acc = np.zeros(H, dtype=np.float32)
        xt = c_oracle.quantize_q8_1(x[t:t + 1], [H, 1])
        for j in range(k):
            e = int(ids[t, j])
            g = c_oracle.matmul(wg[e][1], xt, H, I, 1)
            u = c_oracle.matmul(wu[e][1], xt, H, I, 1)
            m = oracle_np.swiglu(g, u)
            o = c_oracle.matmul(wdn[e][1], c_oracle.quantize_q8_1(m, [I, 1]), I, H, 1)[0]
            acc = (acc.astype(np.float64) + np.float64(rw[t, j]) * o.astype(np.float64)).astype(np.float32)
        np.testing.assert_allclose(y_ffn[t], acc, rtol=2e-3, atol=2e-3)
