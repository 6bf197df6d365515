"""GPU parity of the Q4_0 MoE FFN and the engine linear, stage by stage, through
the C ABI, against the CPU oracle.

Bars:
  * expert ids, routing tables (offsets, src_route, dst_of_route), permuted Q8_1
    bytes, and the Q8_1 bytes of the SwiGLU output given its fp32 values: exact;
  * top-k weights and fp32 SwiGLU values: rtol 2e-6 (expf of the GPU's libm and
    NumPy differ by at most an ulp or two);
  * gate/up, down and linear outputs: rtol 1e-3, atol 1e-4 against the fp64 oracle;
  * combine: rtol 1e-6 (fp32 fma chain against fp64);
  * end to end: the eight-launch FFN entry equals the stage-by-stage run bit for bit,
    and the fp64 oracle chain within rtol 2e-3 / atol 2e-3 (the chain re-quantizes the
    SwiGLU output, which the fp32/fp64 difference of the gate/up sums can move by one
    Q8_1 step in rare elements).
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


def make_w(N, K, rng):
    return c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))


def expert_slice(blocks_q8, off, e):
    """Q8_1 rows [off[e], off[e+1]) of a quantizer-layout buffer of R rows, as its own buffer."""
    return np.ascontiguousarray(blocks_q8[:, off[e]:off[e + 1], :]).reshape(-1)


# ------------------------------------------------------------------ engine linear
@pytest.mark.parametrize("K,N,T", [(4096, 1024, 1), (4096, 300, 7), (1024, 256, 64), (11008, 128, 1)])
def test_linear_q4_0(K, N, T, dev):
    import torch
    note(f"linear_q4_0 K={K} N={N} T={T}")
    rng = np.random.default_rng(K + N + T)
    w = make_w(N, K, rng)
    x = rng.standard_normal((T, K)).astype(np.float32)
    ws = torch.empty(max(1, capi.linear_q4_0_workspace_bytes(K, T)), dtype=torch.uint8, device=dev)
    y = torch.full((T * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.linear_q4_0(to_dev(x, dev), to_dev(w, dev), y, K, N, T, ws=ws)
    xq = c_oracle.quantize_q8_1(x, [K, T])
    np.testing.assert_allclose(host(y).reshape(T, N), c_oracle.matmul(w, xq, K, N, T), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,T", [(4096, 1024, 1), (4096, 300, 7), (1024, 256, 16), (1024, 256, 64),
                                   (11008, 128, 1)])
def test_linear_q4_0_split_layout(K, N, T, dev):
    """The engine linear on weights repacked into the split layout: the oracle's
    result at the usual bars, the Q8_1 workspace bytes exact when one is used, and
    bit for bit the split-layout matmul entry it forwards to."""
    import torch
    note(f"linear_q4_0s K={K} N={N} T={T}")
    rng = np.random.default_rng(3 * K + N + T)
    w = make_w(N, K, rng)
    x = rng.standard_normal((T, K)).astype(np.float32)
    wd = to_dev(w, dev)
    wsplit = torch.empty_like(wd)
    capi.q4_0_to_split(wd, wsplit, N, K)
    nq = max(1, capi.linear_q4_0_workspace_bytes(K, T))
    ws = torch.empty(nq, dtype=torch.uint8, device=dev)
    y = torch.full((T * N,), float("nan"), dtype=torch.float32, device=dev)
    xd = to_dev(x, dev)
    capi.linear_q4_0_split(xd, wsplit, y, K, N, T, ws=ws)
    xq = c_oracle.quantize_q8_1(x, [K, T])
    np.testing.assert_allclose(host(y).reshape(T, N), c_oracle.matmul(w, xq, K, N, T), rtol=RTOL, atol=ATOL)
    if T > 1:
        assert np.array_equal(host(ws)[:xq.size], xq)
    y2 = torch.full_like(y, float("nan"))
    ws2 = torch.empty_like(ws)
    capi.mat_mul_split_f32(wsplit, xd, ws2, y2, K, N, T)
    assert np.array_equal(host(y), host(y2))


def test_linear_q4_0_host_entry():
    import ctypes
    K, N, T = 512, 96, 3
    rng = np.random.default_rng(5)
    w = make_w(N, K, rng)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = np.zeros(T * N, dtype=np.float32)
    rc = capi.lib().linear_q4_0_forward_host(x.ctypes.data, w.ctypes.data, y.ctypes.data, K, T, N)
    assert rc == 0, capi.lib().jjo_last_error()
    xq = c_oracle.quantize_q8_1(x, [K, T])
    np.testing.assert_allclose(y.reshape(T, N), c_oracle.matmul(w, xq, K, N, T), rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------ MoE stages
MOE_CASES = [  # T, H, I, E, top_k
    (64, 256, 384, 8, 2),
    (5, 128, 128, 4, 1),
    (300, 512, 256, 16, 4),
    (64, 256, 256, 64, 8),     # many experts, top-8: mostly short (narrow / paired) tiles
    (40, 128, 128, 256, 8),    # 256 experts for 320 routes: most get 0..3
    (33, 1024, 384, 8, 2),     # wider hidden size
]
# Decode-sized batches: the FFN runs its expert matrices as routed GEMVs (a
# token's experts are distinct, so no expert holds more than T routes).
MOE_DECODE_T = 16  # the FFN's routed-GEMV token limit


def _ffn_routed(T, E, top_k):
    """Whether the FFN runs routed GEMVs: up to MOE_DECODE_T tokens, or at most two
    routes per active expert on average (many experts)."""
    R = T * top_k
    active = min(E, R)
    return T <= MOE_DECODE_T or -(-R // active) <= 2
MOE_DECODE_CASES = [  # T, H, I, E, top_k
    (1, 256, 384, 8, 2),       # one route per active expert
    (2, 512, 256, 16, 4),
    (3, 128, 128, 256, 8),     # 256 experts: the active-expert scan crosses 4 ballots
    (4, 1024, 384, 8, 2),
    (8, 256, 256, 64, 8),      # two route chunks per expert
    (8, 256, 256, 2, 2),       # every token on both experts: 8 routes each
    (2, 512, 5120, 4, 2),      # down projection K = 5120: two K slices
    (1, 9216, 256, 4, 2),      # gate|up K = 9216: three K slices
    (3, 16384, 128, 3, 1),     # gate|up K = 16384: four K slices
    (16, 128, 128, 32, 25),    # 400 routes: routing in four launches, then the routed GEMVs
]


def _routing(T, E, top_k, seed, dev):
    import torch
    rng = np.random.default_rng(seed)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    w = torch.empty(T * top_k, dtype=torch.float32, device=dev)
    ids = torch.empty(T * top_k, dtype=torch.int32, device=dev)
    capi.moe_top_k(to_dev(lg, dev), w, ids, T, E, top_k)
    return lg, host(w), host(ids)


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES)
def test_moe_top_k(T, H, I, E, top_k, dev):
    note(f"moe_top_k T={T} E={E} k={top_k}")
    lg, w, ids = _routing(T, E, top_k, 100 + T, dev)
    ref_ids, ref_w = oracle_np.moe_top_k(lg, top_k)
    assert np.array_equal(ids.reshape(T, top_k), ref_ids)
    np.testing.assert_allclose(w.reshape(T, top_k), ref_w, rtol=2e-6, atol=1e-7)


def test_moe_top_k_ties_take_smaller_id(dev):
    import torch
    note("moe_top_k ties")
    lg = np.zeros((4, 8), dtype=np.float32)
    lg[1, [2, 5]] = 1.0
    lg[2] = np.float32(-3.0)
    lg[3, 7] = 2.0
    w = torch.empty(12, dtype=torch.float32, device=dev)
    ids = torch.empty(12, dtype=torch.int32, device=dev)
    capi.moe_top_k(to_dev(lg, dev), w, ids, 4, 8, 3)
    assert host(ids).reshape(4, 3).tolist() == [[0, 1, 2], [2, 5, 0], [0, 1, 2], [7, 0, 1]]


@pytest.mark.parametrize("E,top_k", [(8, 3), (64, 8), (256, 8), (1024, 32), (70, 5)])
def test_moe_top_k_special_values(E, top_k, dev):
    """The wave-per-token selection reproduces the reference's sequential scan on the
    rows that tell them apart: NaN at expert 0 (kept every round) and elsewhere
    (never chosen), all -inf (expert 0 re-selected), a single finite logit, +-0 ties,
    and ties spread over the whole row (smaller id first)."""
    import torch
    note(f"moe_top_k special E={E} k={top_k}")
    rng = np.random.default_rng(E + top_k)
    rows = [rng.standard_normal(E).astype(np.float32) for _ in range(8)]
    rows[0][0] = np.nan
    rows[1][[1, E // 2, E - 1]] = np.nan
    rows[2][:] = -np.inf
    rows[3][:] = -np.inf
    rows[3][E - 1] = 0.5
    rows[4][:] = 0.0
    rows[4][1::2] = -0.0
    rows[5][:] = np.float32(1.25)
    rows[6][rng.permutation(E)[: min(E, 3 * top_k)]] = np.float32(9.0)  # many equal maxima
    rows[7][0] = -np.inf
    lg = np.stack(rows).astype(np.float32)
    T = lg.shape[0]
    w = torch.empty(T * top_k, dtype=torch.float32, device=dev)
    ids = torch.empty(T * top_k, dtype=torch.int32, device=dev)
    capi.moe_top_k(to_dev(lg, dev), w, ids, T, E, top_k)
    with np.errstate(invalid="ignore"):  # NaN rows give NaN weights on both sides
        ref_ids, ref_w = oracle_np.moe_top_k(lg, top_k)
    assert np.array_equal(host(ids).reshape(T, top_k), ref_ids)
    np.testing.assert_allclose(host(w).reshape(T, top_k), ref_w, rtol=2e-6, atol=1e-7, equal_nan=True)


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES)
def test_moe_dispatch_and_gather(T, H, I, E, top_k, dev):
    import torch
    note(f"moe_dispatch T={T} H={H} E={E} k={top_k}")
    rng = np.random.default_rng(200 + T)
    ids = rng.integers(0, E, size=T * top_k).astype(np.int32)
    ids[: min(len(ids), 10)] = 0  # a crowded expert
    x = rng.standard_normal((T, H)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [H, T])
    R = T * top_k
    off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    src = torch.empty(R, dtype=torch.int32, device=dev)
    dst = torch.empty(R, dtype=torch.int32, device=dev)
    xp = torch.empty(R * H // 128 * 144, dtype=torch.uint8, device=dev)
    capi.moe_dispatch(to_dev(ids, dev), off, src, dst, T, top_k, H, E, xq=to_dev(xq, dev), xq_perm=xp)
    r_off, r_src, r_dst = oracle_np.moe_dispatch(ids, E)
    assert np.array_equal(host(off), r_off)
    assert np.array_equal(host(src), r_src)
    assert np.array_equal(host(dst), r_dst)
    assert np.array_equal(host(xp), oracle_np.gather_q8_1(xq, r_src, T, top_k, H))


def test_moe_dispatch_large_route_count(dev):
    """Routes spread over all 16 waves of the dispatch workgroup, several steps each."""
    import torch
    note("moe_dispatch R=8192 E=64")
    rng = np.random.default_rng(3)
    T, top_k, E = 2048, 4, 64
    ids = rng.integers(0, E, size=T * top_k).astype(np.int32)
    R = T * top_k
    off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    src = torch.empty(R, dtype=torch.int32, device=dev)
    dst = torch.empty(R, dtype=torch.int32, device=dev)
    capi.moe_dispatch(to_dev(ids, dev), off, src, dst, T, top_k, 128, E)
    r_off, r_src, r_dst = oracle_np.moe_dispatch(ids, E)
    assert np.array_equal(host(off), r_off)
    assert np.array_equal(host(src), r_src)
    assert np.array_equal(host(dst), r_dst)


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES)
def test_moe_gate_up(T, H, I, E, top_k, dev):
    import torch
    note(f"moe_gate_up T={T} H={H} I={I} E={E} k={top_k}")
    rng = np.random.default_rng(300 + T)
    R = T * top_k
    ids = rng.integers(0, E, size=R).astype(np.int32)
    off, src, _ = oracle_np.moe_dispatch(ids, E)
    x = rng.standard_normal((R, H)).astype(np.float32)  # already-permuted rows
    xp = c_oracle.quantize_q8_1(x, [H, R])
    wg = [make_w(I, H, rng) for _ in range(E)]
    wu = [make_w(I, H, rng) for _ in range(E)]
    gu = torch.full((R * 2 * I,), float("nan"), dtype=torch.float32, device=dev)
    capi.moe_gate_up(to_dev(np.concatenate(wg), dev), to_dev(np.concatenate(wu), dev), to_dev(xp, dev),
                     to_dev(off, dev), E, gu, H, I, R)
    got = host(gu).reshape(R, 2 * I)
    blocks = xp.reshape(H // 128, R, 144)
    for e in range(E):
        m = off[e + 1] - off[e]
        if m == 0:
            continue
        xe = expert_slice(blocks, off, e)
        np.testing.assert_allclose(got[off[e]:off[e + 1], :I], c_oracle.matmul(wg[e], xe, H, I, m), rtol=RTOL,
                                   atol=ATOL)
        np.testing.assert_allclose(got[off[e]:off[e + 1], I:], c_oracle.matmul(wu[e], xe, H, I, m), rtol=RTOL,
                                   atol=ATOL)


def _q8_1_scales(buf, rows, K):
    """Per-value scale d of a superblock-major Q8_1 buffer of `rows` rows of K values."""
    blk = buf.reshape(K // 128, rows, 144)
    d = blk[:, :, :16].copy().view(np.float16).astype(np.float32)[:, :, 0::2]  # [K/128, rows, 4]
    return np.repeat(d.transpose(1, 0, 2).reshape(rows, K // 32), 32, axis=1)


def _dequant_q8_1(buf, rows, K):
    blk = buf.reshape(K // 128, rows, 144)
    q = blk[:, :, 16:].view(np.int8).astype(np.float32)  # [K/128, rows, 128]
    return q.transpose(1, 0, 2).reshape(rows, K) * _q8_1_scales(buf, rows, K)


GROUPED_GEMV_ROUTES = 48  # the grouped entries run routed GEMVs up to this many routes


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES + [(3, 256, 256, 2, 2), (200, 128, 128, 2, 1),
                                                     (160, 256, 128, 1, 1), (330, 128, 256, 2, 1)])
def test_moe_gate_up_swiglu_fused(T, H, I, E, top_k, dev):
    """The fused gate|up + SwiGLU + Q8_1 launch writes exactly the bytes of the
    unfused chain (grouped gate|up GEMM into fp32, then the SwiGLU quantizer); the
    cases cover experts of <= 8, <= 32, 160 (five column tiles in one chunk) and
    about 165 routes (two chunks), and experts with no routes.  At 48 routes or fewer
    the unfused gate|up runs as a routed GEMV (another summation order), so there
    each value may sit one quantization step away."""
    import torch
    note(f"moe_gate_up_swiglu T={T} H={H} I={I} E={E} k={top_k}")
    rng = np.random.default_rng(500 + T)
    R = T * top_k
    ids = rng.integers(0, E, size=R).astype(np.int32)
    off, _, _ = oracle_np.moe_dispatch(ids, E)
    x = rng.standard_normal((R, H)).astype(np.float32)
    xp = to_dev(c_oracle.quantize_q8_1(x, [H, R]), dev)
    wg = to_dev(np.concatenate([make_w(I, H, rng) for _ in range(E)]), dev)
    wu = to_dev(np.concatenate([make_w(I, H, rng) for _ in range(E)]), dev)
    off_d = to_dev(off, dev)
    gu = torch.empty(R * 2 * I, dtype=torch.float32, device=dev)
    capi.moe_gate_up(wg, wu, xp, off_d, E, gu, H, I, R)
    mq_ref = torch.empty(R * I // 128 * 144, dtype=torch.uint8, device=dev)
    capi.swiglu_quantize(gu, mq_ref, R, I)
    mq = torch.full((R * I // 128 * 144,), 0xA5, dtype=torch.uint8, device=dev)
    capi.moe_gate_up_swiglu(wg, wu, xp, off_d, E, mq, H, I, R)
    if R > GROUPED_GEMV_ROUTES:
        assert np.array_equal(host(mq), host(mq_ref))
    else:
        a, b = _dequant_q8_1(host(mq), R, I), _dequant_q8_1(host(mq_ref), R, I)
        step = np.maximum(_q8_1_scales(host(mq), R, I), _q8_1_scales(host(mq_ref), R, I))
        assert (np.abs(a - b) <= step * 1.2).all()  # one step, and the fp16 scale's own rounding


@pytest.mark.parametrize("rows,I", [(64, 384), (5, 128), (300, 256)])
def test_swiglu_quantize(rows, I, dev):
    import torch
    note(f"swiglu_quantize rows={rows} I={I}")
    rng = np.random.default_rng(rows + I)
    gu = (rng.standard_normal((rows, 2 * I)) * 3).astype(np.float32)
    gu[0, :32] = 0.0  # an all-zero group: d = +inf as the quantizer
    mid = torch.empty(rows * I, dtype=torch.float32, device=dev)
    mq = torch.empty(rows * I // 128 * 144, dtype=torch.uint8, device=dev)
    capi.swiglu_quantize(to_dev(gu, dev), mq, rows, I, mid_f32=mid)
    mid_h = host(mid).reshape(rows, I)
    np.testing.assert_allclose(mid_h, oracle_np.swiglu(gu[:, :I], gu[:, I:]), rtol=2e-6, atol=1e-30)
    assert np.array_equal(host(mq), c_oracle.quantize_q8_1(mid_h, [I, rows]))


@pytest.mark.parametrize("T,H,top_k", [(64, 256, 2), (5, 128, 1), (300, 512, 4)])
def test_moe_combine(T, H, top_k, dev):
    import torch
    note(f"moe_combine T={T} H={H} k={top_k}")
    rng = np.random.default_rng(T + H)
    R = T * top_k
    eo = rng.standard_normal((R, H)).astype(np.float32)
    dst = rng.permutation(R).astype(np.int32)
    w = rng.random(R).astype(np.float32)
    y = torch.empty(T * H, dtype=torch.float32, device=dev)
    capi.moe_combine(to_dev(eo, dev), to_dev(dst, dev), to_dev(w, dev), y, T, H, top_k)
    np.testing.assert_allclose(host(y).reshape(T, H), oracle_np.moe_combine(eo, dst, w, top_k), rtol=1e-6,
                               atol=1e-6)


# ------------------------------------------------------------------ whole FFN
def _ffn_inputs(T, H, I, E, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    wg = [make_w(I, H, rng) for _ in range(E)]
    wu = [make_w(I, H, rng) for _ in range(E)]
    wd = [make_w(H, I, rng) for _ in range(E)]
    return x, lg, wg, wu, wd


def _oracle_ffn(x, lg, wg, wu, wd, top_k):
    T, H = x.shape
    I = wg[0].size * 32 // 18 // H
    E = len(wg)
    R = T * top_k
    xq = c_oracle.quantize_q8_1(x, [H, T])
    ids, w = oracle_np.moe_top_k(lg, top_k)
    off, src, dst = oracle_np.moe_dispatch(ids, E)
    xp = oracle_np.gather_q8_1(xq, src, T, top_k, H).reshape(H // 128, R, 144)
    gu = np.zeros((R, 2 * I), dtype=np.float32)
    for e in range(E):
        m = off[e + 1] - off[e]
        if m:
            xe = expert_slice(xp, off, e)
            gu[off[e]:off[e + 1], :I] = c_oracle.matmul(wg[e], xe, H, I, m)
            gu[off[e]:off[e + 1], I:] = c_oracle.matmul(wu[e], xe, H, I, m)
    mid = oracle_np.swiglu(gu[:, :I], gu[:, I:])
    mq = c_oracle.quantize_q8_1(mid, [I, R]).reshape(I // 128, R, 144)
    eo = np.zeros((R, H), dtype=np.float32)
    for e in range(E):
        m = off[e + 1] - off[e]
        if m:
            eo[off[e]:off[e + 1]] = c_oracle.matmul(wd[e], expert_slice(mq, off, e), I, H, m)
    return oracle_np.moe_combine(eo, dst, w.reshape(-1), top_k)


def _ffn_ws_combine(ws, T, H, I, E, top_k, dev):
    """moe_combine over the FFN workspace's own route weights, sorted-route indices and
    expert outputs (the workspace carve-up of moe_q4_0_ffn_device: route weights,
    ids, offsets, src, dst, Q8_1 x, permuted Q8_1 x, Q8_1 mid, expert outputs, each
    256-byte aligned)."""
    import torch
    R = T * top_k
    sizes = [R * 4, R * 4, (E + 1) * 4, R * 4, R * 4, T * H // 128 * 144, R * H // 128 * 144, R * I // 128 * 144,
             R * H * 4]
    offs, o = [], 0
    for n in sizes:
        offs.append(o)
        o += -(-n // 256) * 256
    rw = ws[offs[0]:offs[0] + R * 4].view(torch.float32)
    dst = ws[offs[4]:offs[4] + R * 4].view(torch.int32)
    eo = ws[offs[8]:offs[8] + R * H * 4].view(torch.float32)
    y = torch.empty(T * H, dtype=torch.float32, device=dev)
    capi.moe_combine(eo, dst, rw, y, T, H, top_k)
    return host(y).reshape(T, H)


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES + MOE_DECODE_CASES)
def test_moe_ffn_end_to_end(T, H, I, E, top_k, dev):
    import torch
    note(f"moe_ffn T={T} H={H} I={I} E={E} k={top_k}")
    x, lg, wg, wu, wd = _ffn_inputs(T, H, I, E, 400 + T)
    d = {k: to_dev(v, dev) for k, v in dict(x=x, lg=lg, wg=np.concatenate(wg), wu=np.concatenate(wu),
                                          wd=np.concatenate(wd)).items()}
    ws = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, top_k), dtype=torch.uint8, device=dev)
    y = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
    capi.moe_ffn(d["x"], d["lg"], d["wg"], d["wu"], d["wd"], y, T, H, I, E, top_k, ws)
    y_ffn = host(y).reshape(T, H)

    # the same stages through their own entries
    R = T * top_k
    rw = torch.empty(R, dtype=torch.float32, device=dev)
    ids = torch.empty(R, dtype=torch.int32, device=dev)
    capi.moe_top_k(d["lg"], rw, ids, T, E, top_k)
    xq = torch.empty(T * H // 128 * 144, dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(d["x"], xq, [H, T])
    off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    src = torch.empty(R, dtype=torch.int32, device=dev)
    dst = torch.empty(R, dtype=torch.int32, device=dev)
    xp = torch.empty(R * H // 128 * 144, dtype=torch.uint8, device=dev)
    capi.moe_dispatch(ids, off, src, dst, T, top_k, H, E, xq=xq, xq_perm=xp)
    gu = torch.empty(R * 2 * I, dtype=torch.float32, device=dev)
    capi.moe_gate_up(d["wg"], d["wu"], xp, off, E, gu, H, I, R)
    mq = torch.empty(R * I // 128 * 144, dtype=torch.uint8, device=dev)
    capi.swiglu_quantize(gu, mq, R, I)
    eo = torch.empty(R * H, dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(d["wd"], mq, off, eo, I, H, R)
    y2 = torch.empty(T * H, dtype=torch.float32, device=dev)
    capi.moe_combine(eo, dst, rw, y2, T, H, top_k)
    ref = _oracle_ffn(x, lg, wg, wu, wd, top_k)
    if not _ffn_routed(T, E, top_k):  # the same kernels as the stage entries: the same bits
        assert np.array_equal(y_ffn, host(y2).reshape(T, H))
    else:  # routed GEMVs sum each row in another order than the MFMA tiles
        np.testing.assert_allclose(host(y2).reshape(T, H), ref, rtol=2e-3, atol=2e-3)
        # the FFN's combine: the bits of moe_combine on its own expert outputs
        assert np.array_equal(y_ffn, _ffn_ws_combine(ws, T, H, I, E, top_k, dev))
    np.testing.assert_allclose(y_ffn, ref, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("T,H,I,E,top_k", [(16, 256, 384, 8, 2), (9, 512, 256, 4, 1), (2, 256, 5120, 8, 2),
                                            (16, 128, 128, 64, 8)])
def test_moe_ffn_decode_skewed_routing(T, H, I, E, top_k, dev):
    """Every token on the same top_k experts: each active expert holds T routes, so a
    routed-GEMV workgroup takes them in several chunks (weights kept in registers)."""
    import torch
    note(f"moe_ffn skewed T={T} H={H} I={I} E={E} k={top_k}")
    x, lg, wg, wu, wd = _ffn_inputs(T, H, I, E, 700 + T)
    lg = lg.copy()
    lg[:, :top_k] += 20.0
    ref = _oracle_ffn(x, lg, wg, wu, wd, top_k)
    d = {k: to_dev(v, dev) for k, v in dict(x=x, lg=lg, wg=np.concatenate(wg), wu=np.concatenate(wu),
                                          wd=np.concatenate(wd)).items()}
    ws = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, top_k), dtype=torch.uint8, device=dev)
    for split in (False, True):
        mats = [d["wg"], d["wu"], d["wd"]]
        if split:
            mats = [_split_stack(d["wg"], E * I, H, dev), _split_stack(d["wu"], E * I, H, dev),
                    _split_stack(d["wd"], E * H, I, dev)]
        y = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
        capi.moe_ffn(d["x"], d["lg"], *mats, y, T, H, I, E, top_k, ws, split=split)
        np.testing.assert_allclose(host(y).reshape(T, H), ref, rtol=2e-3, atol=2e-3)
        assert np.array_equal(host(y).reshape(T, H), _ffn_ws_combine(ws, T, H, I, E, top_k, dev))


@pytest.mark.parametrize("T", [1, 3])
def test_moe_ffn_decode_repeated_expert(T, dev):
    """A token whose only finite logit is expert 0 selects expert 0 twice (the
    reference's top-k rule: a taken expert reads -inf, and the first id wins a tie
    of -inf), so expert 0 holds more routes than tokens: the routed GEMVs must take
    every route (the second has weight 0 and must still be computed, not left as
    whatever the workspace held)."""
    import torch
    H, I, E, k = 256, 384, 8, 2
    note(f"moe_ffn repeated expert T={T}")
    x, lg, wg, wu, wd = _ffn_inputs(T, H, I, E, 800 + T)
    lg = lg.copy()
    lg[0, 1:] = -np.inf
    ids, _ = oracle_np.moe_top_k(lg, k)
    assert list(ids[0]) == [0, 0]
    ref = _oracle_ffn(x, lg, wg, wu, wd, k)
    d = {n: to_dev(v, dev) for n, v in dict(x=x, lg=lg, wg=np.concatenate(wg), wu=np.concatenate(wu),
                                          wd=np.concatenate(wd)).items()}
    ws = torch.full((capi.moe_ffn_workspace_bytes(T, H, I, E, k),), 255, dtype=torch.uint8, device=dev)  # NaN fill
    for split in (False, True):
        mats = [d["wg"], d["wu"], d["wd"]]
        if split:
            mats = [_split_stack(d["wg"], E * I, H, dev), _split_stack(d["wu"], E * I, H, dev),
                    _split_stack(d["wd"], E * H, I, dev)]
        y = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
        capi.moe_ffn(d["x"], d["lg"], *mats, y, T, H, I, E, k, ws, split=split)
        np.testing.assert_allclose(host(y).reshape(T, H), ref, rtol=2e-3, atol=2e-3)
        assert np.array_equal(host(y).reshape(T, H), _ffn_ws_combine(ws, T, H, I, E, k, dev))


def test_moe_ffn_rejects_small_workspace(dev):
    import torch
    T, H, I, E, k = 4, 128, 128, 4, 2
    need = capi.moe_ffn_workspace_bytes(T, H, I, E, k)
    ws = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    z = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    y = torch.empty(T * H, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="workspace"):
        capi.moe_ffn(z, z, z, z, z, y, T, H, I, E, k, ws)


# ------------------------------------------------------------------ split-layout experts
def _split_stack(w_dev, rows, K, dev):
    """The stacked expert matrices repacked into the split layout as one matrix."""
    import torch
    out = torch.empty_like(w_dev)
    capi.q4_0_to_split(w_dev, out, rows, K)
    return out


@pytest.mark.parametrize("counts,N,K", [([1, 129, 0, 31, 160, 32, 33, 7], 256, 512), ([3, 2, 1, 4], 384, 512),
                                        ([200, 0, 5], 300, 512), ([0, 7, 0, 1], 100, 512), ([32], 256, 512),
                                        ([2, 0, 9, 1], 256, 5120), ([5, 1], 96, 14336),
                                        ([1, 0, 1, 1], 100, 11008), ([1, 1], 100, 14336), ([2, 0, 1], 64, 11008),
                                        ([0] * 200 + [3] + [0] * 50 + [7, 1] + [0] * 11, 64, 512)])
def test_grouped_split_layout(counts, N, K, dev):
    """The grouped GEMM on split-layout experts equals the block_q4_0 launch bit for
    bit above 48 routes (the same MFMA kernel; only the weight loads differ), with route
    scatter, empty experts, narrow and paired tails and a ragged N.  At 48 routes or
    fewer both run as routed GEMVs, whose two layouts sum a row in different orders:
    both are checked against the oracle, scattered through route_dst."""
    import torch
    E = len(counts)
    note(f"grouped split E={len(counts)} R={sum(counts)} N={N} K={K}")
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(offsets[-1])
    rng = np.random.default_rng(R + N)
    xq = c_oracle.quantize_q8_1(rng.standard_normal((R, K)).astype(np.float32), [K, R])
    w_h = [make_w(N, K, rng) for _ in range(E)]
    w = to_dev(np.concatenate(w_h), dev)
    ws = _split_stack(w, E * N, K, dev)
    perm = rng.permutation(R).astype(np.int32)
    dst = to_dev(perm, dev)
    off_d, xq_d = to_dev(offsets, dev), to_dev(xq, dev)
    y1 = torch.full((R * N,), float("nan"), dtype=torch.float32, device=dev)
    y2 = torch.full((R * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(w, xq_d, off_d, y1, K, N, R, route_dst=dst)
    capi.grouped_mat_mul(ws, xq_d, off_d, y2, K, N, R, route_dst=dst, split=True)
    a, b = host(y1), host(y2)
    assert not np.isnan(a).any()
    if R > GROUPED_GEMV_ROUTES:
        assert np.array_equal(a, b)
    else:
        ref = np.zeros((R, N), dtype=np.float32)
        blocks = xq.reshape(K // 128, R, 144)
        for e in range(E):
            if counts[e]:
                ref[perm[offsets[e]:offsets[e + 1]]] = c_oracle.matmul(w_h[e], expert_slice(blocks, offsets, e), K,
                                                                       N, counts[e])
        np.testing.assert_allclose(a.reshape(R, N), ref, rtol=RTOL, atol=ATOL)
        np.testing.assert_allclose(b.reshape(R, N), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("T,H,I,E,top_k", MOE_CASES + MOE_DECODE_CASES)
def test_moe_ffn_split_layout(T, H, I, E, top_k, dev):
    """The FFN on split-layout expert weights equals the block_q4_0 FFN bit for bit
    (MFMA tiles); at decode sizes both match the oracle (the routed GEMVs of the two
    layouts give each lane other blocks, so their sums differ in the last bits)."""
    import torch
    note(f"moe_ffn split T={T} H={H} I={I} E={E} k={top_k}")
    x, lg, wg, wu, wd = _ffn_inputs(T, H, I, E, 900 + T)
    d = {k: to_dev(v, dev) for k, v in dict(x=x, lg=lg, wg=np.concatenate(wg), wu=np.concatenate(wu),
                                          wd=np.concatenate(wd)).items()}
    sg = _split_stack(d["wg"], E * I, H, dev)
    su = _split_stack(d["wu"], E * I, H, dev)
    sd = _split_stack(d["wd"], E * H, I, dev)
    ws = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, top_k), dtype=torch.uint8, device=dev)
    y1 = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
    y2 = torch.full((T * H,), float("nan"), dtype=torch.float32, device=dev)
    capi.moe_ffn(d["x"], d["lg"], d["wg"], d["wu"], d["wd"], y1, T, H, I, E, top_k, ws)
    capi.moe_ffn(d["x"], d["lg"], sg, su, sd, y2, T, H, I, E, top_k, ws, split=True)
    a, b = host(y1), host(y2)
    assert np.isfinite(a).all()
    if not _ffn_routed(T, E, top_k):
        assert np.array_equal(a, b)
    else:
        ref = _oracle_ffn(x, lg, wg, wu, wd, top_k)
        np.testing.assert_allclose(a.reshape(T, H), ref, rtol=2e-3, atol=2e-3)
        np.testing.assert_allclose(b.reshape(T, H), ref, rtol=2e-3, atol=2e-3)

