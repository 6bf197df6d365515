"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars:
  * Q8_1 bytes (qs + half2 bits)       : bit-exact
  * per-block int32 dot sums           : bit-exact
  * fp32 outputs                       : rtol 1e-3, atol 1e-4 against the fp64 oracle
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


def make_x(K, M, seed, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        ch = rng.choice(K, max(1, K // 1000), replace=False)
        x[:, ch] *= 20
    return x


def make_w(N, K, seed):
    rng = np.random.default_rng(seed)
    return c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))


def gpu_quantize(x, dims, dev):
    import torch
    xt = to_dev(x.reshape(-1), dev)
    out = torch.zeros(capi.q8_1_output_bytes(dims), dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(xt, out, dims)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("dims", [
    [2048, 13, 1, 1],      # the reference test's shape
    [4096, 1, 1, 1],
    [11008, 1, 1, 1],
    [4096, 16, 1, 1],
    [160, 3, 1, 1],        # K % 128 != 0: tail groups
    [640, 2, 2, 3],        # ne2*ne3 > 1: slice stride of the reference kernel
    [4096, 2048, 1, 1],    # prefill activation
])
def test_quantize_bit_exact(dims, dev):
    note(f"quantize dims={dims}")
    n = int(np.prod(dims))
    rng = np.random.default_rng(n % 1000)
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.choice(n, max(1, n // 1000), replace=False)] *= 20
    x[32:64] = 0.0                                  # zero group -> d = +inf
    x[64:96] = np.arange(32, dtype=np.float32) - 15.5  # exact ties after scaling by 127/16.5? (mixed)
    x[96:128] = 2.5
    x[96] = 127.0                                   # d_inv = 1: q = roundf(2.5) = 3
    got = gpu_quantize(x, dims, dev)
    exp = c_oracle.quantize_q8_1(x, dims)
    assert got.shape == exp.shape
    bad = np.flatnonzero(got != exp)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


def test_reference_test_through_pybind(dev):
    """tests/test_q8_1.py:65-123 through q8_1_me, against the committed fixture."""
    import q8_1_me
    from pathlib import Path
    note("q8_1_me.quantize seed24 [2048,13,1,1]")
    np.random.seed(24)
    x = np.asfortranarray(np.random.randn(2048, 13, 1, 1).astype(np.float32))
    out = np.zeros(208 * 144, np.uint8)
    q8_1_me.quantize(x, out, [2048, 13, 1, 1])
    g = np.load(Path(__file__).parent / "golden" / "q8_1_seed24_2048x13.npz")
    assert np.array_equal(out, g["q8_1"])
    qs, d, s = q8_1_me.parse(out, 208)
    qr, dr, sr = c_oracle.parse_q8_1(g["q8_1"], 208)
    assert np.array_equal(qs, qr) and np.array_equal(d, dr) and np.array_equal(s, sr)


# ------------------------------------------------------------------ integer stage
@pytest.mark.parametrize("K,N,M", [(256, 48, 3), (4096, 33, 1), (128, 7, 17)])
def test_block_sums_bit_exact(K, N, M, dev):
    import torch
    note(f"block_sums K={K} N={N} M={M}")
    w = make_w(N, K, K + N)
    x = make_x(K, M, M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    out = torch.empty(M * N * (K // 32), dtype=torch.int32, device=dev)
    capi.block_sums(to_dev(w, dev), to_dev(xq, dev), out, K, N, M)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().reshape(M, N, K // 32), c_oracle.block_sums(w, xq, K, N, M))


def test_golden_small_case(dev):
    import torch
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "mmq_small.npz")
    K, N, M = int(g["K"]), int(g["N"]), int(g["M"])
    note(f"golden mmq_small K={K} N={N} M={M}")
    assert np.array_equal(gpu_quantize(g["x"], [K, M], dev), g["xq"])
    for algo in (capi.ALGO_GEMV, capi.ALGO_MFMA):
        y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
        capi.mat_mul(to_dev(g["w"], dev), to_dev(g["xq"], dev), y, K, N, M, algo=algo)
        torch.cuda.synchronize()
        np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), g["y"], rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------ matmul
def run_mm(w, xq, K, N, M, algo, dev):
    import torch
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul(to_dev(w, dev), to_dev(xq, dev), y, K, N, M, algo=algo)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(M, N)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("K,N", [(4096, 257), (11008, 64), (128, 5), (640, 96)])
def test_gemv(K, N, M, dev):
    note(f"gemv K={K} N={N} M={M}")
    w = make_w(N, K, 7 * N + K)
    x = make_x(K, M, 100 + M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    got = run_mm(w, xq, K, N, M, capi.ALGO_GEMV, dev)
    np.testing.assert_allclose(got, c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,M", [
    (4096, 256, 128), (4096, 300, 130), (256, 128, 1), (640, 200, 16), (11008, 128, 64), (384, 64, 257),
    (1024, 70, 33), (512, 4100, 96), (128, 96, 70), (128, 5, 40),
])
@pytest.mark.parametrize("algo", [capi.ALGO_MFMA, capi.ALGO_MFMA64, capi.ALGO_MFMA32, capi.ALGO_MFMA_W32])
def test_gemm_mfma(K, N, M, algo, dev):
    note(f"gemm mfma algo={algo} K={K} N={N} M={M}")
    w = make_w(N, K, 3 * N + K)
    x = make_x(K, M, 200 + M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    got = run_mm(w, xq, K, N, M, algo, dev)
    np.testing.assert_allclose(got, c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M", [1, 3, 4, 8, 13, 16, 17, 32])
@pytest.mark.parametrize("K,N", [(4096, 257), (11008, 64), (256, 5), (768, 96), (14336, 48), (512, 33)])
def test_gemm_skinny(K, N, M, dev):
    note(f"gemm skinny K={K} N={N} M={M}")
    w = make_w(N, K, 11 * N + K)
    x = make_x(K, M, 300 + M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    got = run_mm(w, xq, K, N, M, capi.ALGO_SKINNY, dev)
    np.testing.assert_allclose(got, c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M", [1, 3, 4, 5, 7, 8, 9, 13, 16])
@pytest.mark.parametrize("K,N", [(4096, 257), (11008, 64), (256, 5), (768, 96), (14336, 48), (4352, 257),
                                 (4096, 4100), (512, 16400)])
def test_gemm_skinny_lds(K, N, M, dev):
    """The LDS-resident skinny kernel: K windows of 4096 (14336 = 3.5 windows, 4352 =
    a one-stage last window), 1..4 tiles per workgroup (N=4100: 2, N=16400: 4 with a
    second round), rows and tokens past the end; M <= 8 takes the paired-block
    MFMA path, M = 9..16 one block per MFMA."""
    note(f"gemm skinny lds K={K} N={N} M={M}")
    w = make_w(N, K, 13 * N + K)
    x = make_x(K, M, 400 + M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    got = run_mm(w, xq, K, N, M, capi.ALGO_SKINNY_LDS, dev)
    np.testing.assert_allclose(got, c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


def test_gemm_skinny_lds_full_size(dev):
    """Small-batch decode at M=16 (K=4096, N=14336: four tiles per workgroup)."""
    K, N, M = 4096, 14336, 16
    note(f"gemm skinny lds full size K={K} N={N} M={M}")
    w = make_w(N, K, 2)
    x = make_x(K, M, 16)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    got = run_mm(w, xq, K, N, M, capi.ALGO_SKINNY_LDS, dev)
    np.testing.assert_allclose(got, c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


def test_gemm_skinny_lds_rejects_unsupported(dev):
    import torch
    for K, M in ((640, 4), (4096, 17)):
        w = torch.zeros(8 * K // 32 * 18, dtype=torch.uint8, device=dev)
        xq = torch.zeros(M * K // 128 * 144, dtype=torch.uint8, device=dev)
        y = torch.empty(M * 8, dtype=torch.float32, device=dev)
        with pytest.raises(RuntimeError, match="LDS-resident skinny"):
            capi.mat_mul(w, xq, y, K, 8, M, algo=capi.ALGO_SKINNY_LDS)


def test_gemm_skinny_rejects_unsupported(dev):
    """K % 256 != 0 and batch > 32 are refused with an error, not computed."""
    import torch
    for K, M in ((640, 4), (4096, 33)):
        w = torch.zeros(8 * K // 32 * 18, dtype=torch.uint8, device=dev)
        xq = torch.zeros(M * K // 128 * 144, dtype=torch.uint8, device=dev)
        y = torch.empty(M * 8, dtype=torch.float32, device=dev)
        with pytest.raises(RuntimeError, match="skinny"):
            capi.mat_mul(w, xq, y, K, 8, M, algo=capi.ALGO_SKINNY)


@pytest.mark.parametrize("K,N", [(4096, 11008), (11008, 4096), (128, 33), (640, 257), (4096, 5)])
def test_fused_quantize_gemv(K, N, dev):
    """mat_mul_q4_0_q8_1_f32_device at batch 1: the in-kernel quantization writes the
    same Q8_1 bytes as the oracle (bit-exact) and y is within tolerance."""
    import torch
    note(f"fused quantize+GEMV K={K} N={N}")
    w = make_w(N, K, K + 3 * N)
    x = make_x(K, 1, K)
    x[0, 64:96] = 2.5
    x[0, 70] = 127.0           # d_inv = 1: ties round away from zero
    xq_ref = c_oracle.quantize_q8_1(x, [K, 1])
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x, dev), xq, y, K, N, 1)
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_allclose(y.cpu().numpy().reshape(1, N), c_oracle.matmul(w, xq_ref, K, N, 1), rtol=RTOL, atol=ATOL)
    # without a workspace
    y2 = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x, dev), None, y2, K, N, 1)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.parametrize("K,N", [(4096, 256), (11008, 64)])
def test_quantizers_round_the_product_first(K, N, dev):
    """Crafted activations whose rounded product x*d_inv is a tie k + 0.5 while the
    exact product lies below it: the fused in-kernel quantizer and the standalone one
    both give roundf's k + 1 (an unrounded, fused multiply-add would give k)."""
    import torch
    from _ties import q8_tie_input
    note(f"tie-rounding quantizers K={K}")
    x, slots, qexp = q8_tie_input(K, seed=K)
    xq_ref = c_oracle.quantize_q8_1(x.reshape(1, K), [K, 1])
    qs, _, _ = c_oracle.parse_q8_1(xq_ref, K // 128)
    assert np.array_equal(qs.reshape(-1)[slots].astype(np.int64), qexp)
    assert np.array_equal(gpu_quantize(x, [K, 1], dev), xq_ref)
    w = make_w(N, K, 5)
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x, dev), xq, y, K, N, 1)
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), xq_ref)


@pytest.mark.parametrize("K,N,M", [(512, 100, 2), (512, 100, 5), (4096, 257, 2), (4096, 257, 3), (4096, 300, 4),
                                   (11008, 64, 2), (11008, 64, 3), (128, 7, 4)])
def test_f32_entry_batched(K, N, M, dev):
    """fp32 activation entry at batch > 1: a quantizer launch + matmul; the Q8_1
    workspace is bit-exact."""
    import torch
    note(f"f32 entry batched K={K} N={N} M={M}")
    w = make_w(N, K, 77)
    x = make_x(K, M, 78)
    xq_ref = c_oracle.quantize_q8_1(x, [K, M])
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.empty(M * N, dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x, dev), xq, y, K, N, M)
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), c_oracle.matmul(w, xq_ref, K, N, M), rtol=RTOL, atol=ATOL)


def test_zero_activation_group_gives_nan_like_reference(dev):
    K, N, M = 256, 64, 2
    note("zero activation group -> NaN rows")
    w = make_w(N, K, 9)
    x = make_x(K, M, 9)
    x[1, 32:64] = 0.0
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    assert np.all(np.isnan(exp[1])) and np.all(np.isfinite(exp[0]))
    for algo in (capi.ALGO_GEMV, capi.ALGO_MFMA, capi.ALGO_MFMA_W32):
        got = run_mm(w, xq, K, N, M, algo, dev)
        assert np.all(np.isnan(got[1]))
        np.testing.assert_allclose(got[0], exp[0], rtol=RTOL, atol=ATOL)
    # fused path, single token with a zero group
    import torch
    y = torch.empty(N, dtype=torch.float32, device=dev)
    capi.mat_mul_f32(to_dev(w, dev), to_dev(x[1:2], dev), None, y, K, N, 1)
    torch.cuda.synchronize()
    assert np.all(np.isnan(y.cpu().numpy()))


@pytest.mark.parametrize("M", [2, 6, 70])
def test_infinite_block_sum_gives_inf_like_reference(M, dev):
    """A block whose fp16 sum term s overflows to inf: the reference's
    d_w * (d_x * sumi - 8 * s) is +-inf for every output row of that token."""
    K, N = 256, 64
    note(f"infinite s block M={M}")
    w = make_w(N, K, 9)
    x = make_x(K, M, 9)
    x[1, 64:96] = 3000.0   # d = 3000/127, sum q = 4064 -> s = 96000 -> inf in fp16
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    assert np.all(np.isinf(exp[1]))
    algos = [capi.ALGO_MFMA, capi.ALGO_MFMA64, capi.ALGO_MFMA32, capi.ALGO_MFMA_W32] + ([capi.ALGO_GEMV] if M <= 8 else []) + ([capi.ALGO_SKINNY] if M <= 32 else [])
    algos += [capi.ALGO_SKINNY_LDS] if M <= 16 else []
    for algo in algos:
        got = run_mm(w, xq, K, N, M, algo, dev)
        assert np.array_equal(got[1], exp[1]), algo
        np.testing.assert_allclose(np.delete(got, 1, 0), np.delete(exp, 1, 0), rtol=RTOL, atol=ATOL)


def test_mmq_host_entry_through_pybind(dev):
    """mm_q4_0_q8_1_me.mmq: quant_workspace bit-exact, output within tolerance."""
    import mm_q4_0_q8_1_me
    for K, N, T in ((4096, 96, 1), (512, 64, 5), (256, 33, 70)):
        note(f"mmq host K={K} N={N} T={T}")
        w = make_w(N, K, K + T)
        x = np.asfortranarray(make_x(K, T, T).T.reshape(K, T, 1, 1))
        ws = np.zeros(T * (K // 128) * 144, np.uint8)
        y = np.zeros(T * N, np.float32)
        mm_q4_0_q8_1_me.mmq(w, x, ws, y, [K, T, 1, 1], N, K)
        xq = c_oracle.quantize_q8_1(x, [K, T, 1, 1])
        assert np.array_equal(ws, xq)
        np.testing.assert_allclose(y.reshape(T, N), c_oracle.matmul(w, xq, K, N, T), rtol=RTOL, atol=ATOL)


def test_read_floor_diagnostic(dev):
    """The read-floor diagnostic runs on any 16-byte multiple and refuses the rest."""
    import torch
    note("read floor diagnostic")
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    capi.read_floor(buf, buf.numel(), out)
    capi.read_floor(buf, 16, out)
    torch.cuda.synchronize()
    assert int(out.item()) == 0  # the checksum of all-ones data is not the sentinel
    for n in (0, 8, 17):
        with pytest.raises(RuntimeError, match="read_floor"):
            capi.read_floor(buf, n, out)


# ------------------------------------------------------------------ grouped (MoE)
def test_grouped_moe_small(dev):
    import torch
    E, K, N, T, topk = 4, 256, 96, 37, 2
    note(f"grouped E={E} K={K} N={N} T={T}")
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    experts = np.argsort(-logits, axis=1)[:, :topk]            # [T, topk]
    route_expert = experts.reshape(-1)                          # route r = t*topk + k
    order = np.argsort(route_expert, kind="stable")             # sorted routes
    counts = np.bincount(route_expert, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    x = make_x(K, T, 5)
    xr = x[order // topk]                                       # routed activations, sorted by expert
    R = T * topk
    xq = c_oracle.quantize_q8_1(xr, [K, R])
    ws = [make_w(N, K, 50 + e) for e in range(E)]
    w_all = np.concatenate(ws)
    y = torch.full((R * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(to_dev(w_all, dev), to_dev(xq, dev), to_dev(offsets, dev), y, K, N, R,
                         route_dst=to_dev(order.astype(np.int32), dev))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(R, N)
    for e in range(E):
        sel = order[offsets[e]:offsets[e + 1]]
        if sel.size == 0:
            continue
        xe = c_oracle.quantize_q8_1(x[sel // topk], [K, sel.size])
        exp = c_oracle.matmul(ws[e], xe, K, N, sel.size)
        np.testing.assert_allclose(got[sel], exp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("counts", [[1, 129, 0, 31, 160, 32, 33, 7], [3, 2, 1, 4], [64, 65, 0, 96, 1, 200],
                                    [8, 9, 136, 137, 5, 6], [161, 320, 321, 481, 0, 2]])
def test_grouped_tail_tiles(counts, dev):
    """Experts of 1..33 routes (one narrow chunk of 1..2 column tiles), 129..160 (one
    chunk of up to 5 column tiles), 161..481 (2..4 equal chunks, the last ones
    ragged), and empty experts; every output row is checked against the oracle."""
    import torch
    E, K, N = len(counts), 512, 256
    note(f"grouped tails counts={counts}")
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(offsets[-1])
    x = make_x(K, R, 31)
    xq = c_oracle.quantize_q8_1(x, [K, R])
    ws = [make_w(N, K, 60 + e) for e in range(E)]
    dst = np.random.default_rng(1).permutation(R).astype(np.int32)
    y = torch.full((R * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.grouped_mat_mul(to_dev(np.concatenate(ws), dev), to_dev(xq, dev), to_dev(offsets, dev), y, K, N, R,
                         route_dst=to_dev(dst, dev))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(R, N)
    assert not np.isnan(got).any()
    blocks = xq.reshape(K // 128, R, 144)
    for e in range(E):
        m = counts[e]
        if m == 0:
            continue
        xe = np.ascontiguousarray(blocks[:, offsets[e]:offsets[e + 1]]).reshape(-1)
        np.testing.assert_allclose(got[dst[offsets[e]:offsets[e + 1]]], c_oracle.matmul(ws[e], xe, K, N, m),
                                   rtol=RTOL, atol=ATOL)


def test_grouped_malformed_offsets_stay_in_bounds(dev):
    """A malformed expert table (negative start, decreasing, past n_routes) drops or
    overlaps routes but never reads or writes outside the buffers: guard rows around
    y keep their sentinel, and each clamped range [clamp(off[e]), clamp(off[e+1]))
    holds expert e's result."""
    import torch
    K, N, R = 256, 96, 90
    offsets = np.array([-5, 50, 30, 200, 90], dtype=np.int32)
    E = offsets.size - 1
    note(f"grouped malformed offsets {offsets.tolist()}")
    x = make_x(K, R, 41)
    xq = c_oracle.quantize_q8_1(x, [K, R])
    ws = [make_w(N, K, 70 + e) for e in range(E)]
    guard = 64
    buf = torch.full((R * N + 2 * guard * N,), 12345.0, dtype=torch.float32, device=dev)
    y = buf[guard * N: guard * N + R * N]
    capi.grouped_mat_mul(to_dev(np.concatenate(ws), dev), to_dev(xq, dev), to_dev(offsets, dev), y, K, N, R)
    torch.cuda.synchronize()
    b = buf.cpu().numpy()
    assert np.all(b[:guard * N] == 12345.0) and np.all(b[guard * N + R * N:] == 12345.0)
    got = b[guard * N: guard * N + R * N].reshape(R, N)
    blocks = xq.reshape(K // 128, R, 144)
    clamp = lambda v, lo: min(max(int(v), lo), R)
    ranges = []
    for e in range(E):
        beg = clamp(offsets[e], 0)
        end = clamp(offsets[e + 1], beg)
        ranges.append((beg, end))
    # rows covered by exactly one expert must equal that expert's result
    owner = np.full(R, -1)
    count = np.zeros(R, dtype=int)
    for e, (beg, end) in enumerate(ranges):
        owner[beg:end] = e
        count[beg:end] += 1
    for e, (beg, end) in enumerate(ranges):
        rows = np.arange(beg, end)[count[beg:end] == 1]
        if rows.size == 0:
            continue
        xe = np.ascontiguousarray(blocks[:, rows]).reshape(-1)
        np.testing.assert_allclose(got[rows], c_oracle.matmul(ws[e], xe, K, N, rows.size), rtol=RTOL, atol=ATOL)
    assert np.isfinite(got[count > 0]).all()


# ------------------------------------------------------------------ full-size configs
def _sample_check(w, xq, y, K, N, M, n_rows=96, n_tok=64, seed=0):
    """Oracle on a random subset of output rows and tokens (exact sub-problem)."""
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(N, min(n_rows, N), replace=False))
    toks = np.sort(rng.choice(M, min(n_tok, M), replace=False))
    nb = K // 32
    wsub = w.reshape(N, nb * 18)[rows].reshape(-1)
    xb = xq.reshape(K // 128, M, 144)[:, toks].reshape(-1)
    exp = c_oracle.matmul(wsub, xb, K, rows.size, toks.size)
    np.testing.assert_allclose(y[np.ix_(toks, rows)], exp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,M,seed", [(4096, 11008, 1, 1), (11008, 4096, 1, 1), (4096, 14336, 8, 2),
                                        (4096, 14336, 16, 2), (4096, 4096, 2048, 3), (4096, 14336, 2048, 3)])
def test_baseline_configs_sampled(K, N, M, seed, dev):
    import torch
    note(f"baseline config K={K} N={N} M={M}")
    from jjjetson_ops_amd import q4_0
    g = torch.Generator(device="cpu").manual_seed(seed)
    wf = torch.randn(N, K, generator=g) * 0.02
    w = q4_0.quantize_q4_0_np(wf.numpy())
    x = make_x(K, M, seed + 10)
    xt = to_dev(x, dev)
    xq_t = torch.empty(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(xt, xq_t, [K, M])
    y = torch.empty(M * N, dtype=torch.float32, device=dev)
    capi.mat_mul(to_dev(w, dev), xq_t, y, K, N, M)
    torch.cuda.synchronize()
    xq = xq_t.cpu().numpy()
    # quantizer bytes for a token subset are exact
    toks = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
    assert np.array_equal(xq.reshape(K // 128, M, 144)[:, toks].reshape(-1),
                          c_oracle.quantize_q8_1(x[toks], [K, toks.size]))
    _sample_check(w, xq, y.cpu().numpy().reshape(M, N), K, N, M, seed=seed)

