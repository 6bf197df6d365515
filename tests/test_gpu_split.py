"""The split Q4_0 weight layout on the GPU: the device repacker equals the host one
byte for byte, and every split-layout matmul entry matches the oracle (which reads
the reference block_q4_0 layout) at the reference's bars: Q8_1 workspace bytes
exact, fp32 outputs rtol 1e-3 / atol 1e-4.  Includes BASELINE config 2 (M=1,
K=4096->N=11008 and K=11008->N=4096, weights seed 1, quantized on device each call)
through the fused entry, every output checked."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import sys

import numpy as np
import pytest

from jjjetson_ops_amd import capi
from oracle import c_oracle

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


def split_dev(w, N, K, dev):
    """Device repack of host Q4_0 bytes w; checked against the host repacker."""
    import torch
    wd = to_dev(w, dev)
    out = torch.empty(w.size, dtype=torch.uint8, device=dev)
    capi.q4_0_to_split(wd, out, N, K)
    assert np.array_equal(host(out), capi.q4_0_to_split_host(w, N, K))
    return out


@pytest.mark.parametrize("N,K", [(1, 32), (3, 96), (257, 4096), (4096 + 5, 128)])
def test_device_repack_equals_host(N, K, dev):
    note(f"split repack N={N} K={K}")
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8)
    split_dev(w, N, K, dev)


def _weights(rng, N, K):
    return c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("K,N", [(128, 77), (4096, 1000), (11008, 300), (11008, 77), (16384, 64)])
def test_split_matmul_q8_1_input(M, K, N, dev):
    import torch
    if M * (K // 32) * 48 > 150 * 1024:
        pytest.skip("outside the split GEMV's LDS limit (the entry rejects it; tested below)")
    note(f"split matmul M={M} K={K} N={N}")
    rng = np.random.default_rng(M * 1000 + K + N)
    w = _weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    ws = split_dev(w, N, K, dev)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split(ws, to_dev(xq, dev), y, K, N, M)
    np.testing.assert_allclose(host(y).reshape(M, N), c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N", [(4096, 11008), (11008, 4096)])
def test_config2_split_fused_full(K, N, dev):
    """BASELINE config 2 through the split layout: weights N(0,0.02) seed 1 (drawn on
    the device, packed by the gfx950 quantizer, repacked on the device), x N(0,1)
    with 0.1% outlier channels x20, quantized in the fused kernel."""
    import torch
    from jjjetson_ops_amd import weights
    note(f"config 2 split fused: M=1 K={K} N={N}")
    g = torch.Generator(device=dev).manual_seed(1)
    wf = torch.randn(N, K, generator=g, device=dev) * 0.02
    wq = torch.empty(N * (K // 32) * 18, dtype=torch.uint8, device=dev)
    weights.quantize_q4_0_device(wf, wq, N, K)
    del wf
    w = host(wq)
    ws = torch.empty_like(wq)
    capi.q4_0_to_split(wq, ws, N, K)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((1, K)).astype(np.float32)
    x[:, rng.choice(K, max(1, K // 1000), replace=False)] *= 20
    xq_ref = c_oracle.quantize_q8_1(x, [K, 1])
    y_ref = c_oracle.matmul(w, xq_ref, K, N, 1)
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split_f32(ws, to_dev(x, dev), xq, y, K, N, 1)
    assert np.array_equal(host(xq), xq_ref)
    np.testing.assert_allclose(host(y).reshape(1, N), y_ref, rtol=RTOL, atol=ATOL)
    # without a workspace (the Q8_1 bytes are not wanted)
    y2 = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split_f32(ws, to_dev(x, dev), None, y2, K, N, 1)
    assert np.array_equal(host(y2), host(y))


@pytest.mark.parametrize("M", [2, 4, 8])
def test_split_f32_batch(M, dev):
    import torch
    K, N = 4096, 515
    note(f"split f32 entry M={M} K={K} N={N}")
    rng = np.random.default_rng(40 + M)
    w = _weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xq_ref = c_oracle.quantize_q8_1(x, [K, M])
    ws = split_dev(w, N, K, dev)
    xq = torch.zeros(xq_ref.size, dtype=torch.uint8, device=dev)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split_f32(ws, to_dev(x, dev), xq, y, K, N, M)
    assert np.array_equal(host(xq), xq_ref)
    np.testing.assert_allclose(host(y).reshape(M, N), c_oracle.matmul(w, xq_ref, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,M", [(4096, 256, 128), (4096, 300, 130), (384, 64, 257), (128, 96, 9),
                                   (11008, 128, 64), (512, 4100, 96), (4096, 257, 5), (4096, 1000, 8),
                                   (11264, 77, 12), (256, 33, 16), (4096, 14336, 16), (4096, 70, 17),
                                   # K % 256 != 0: the skinny kernel is unsupported, batch 3/6 take
                                   # the GEMV (two K slices), batch 12 the GEMM
                                   (4224, 100, 3), (4224, 100, 6), (4224, 100, 12),
                                   # the per-wave skinny kernel (batch 17..32; 3..16 above K = 4096)
                                   (4096, 300, 24), (4096, 1000, 32), (11008, 257, 3), (14336, 200, 9),
                                   # the small-tile GEMM, 32- and 64-row tiles
                                   (4096, 4096, 48), (4096, 1000, 64), (14336, 520, 200)])
def test_split_gemm(K, N, M, dev):
    import torch
    note(f"split gemm M={M} K={K} N={N}")
    rng = np.random.default_rng(K + 3 * N + M)
    w = _weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    ws = split_dev(w, N, K, dev)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split(ws, to_dev(xq, dev), y, K, N, M)
    np.testing.assert_allclose(host(y).reshape(M, N), c_oracle.matmul(w, xq, K, N, M), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,M", [(256, 5120, 1700), (256, 14336, 2048), (128, 128 * 33, 128 * 16 + 5)])
def test_split_gemm_tail_round(K, N, M, dev):
    """Tile counts that leave a partial last round of at most half the 512 slots
    (2 per CU): that round runs as 64-token half tiles, including a half that lies
    entirely past M.  Checked on a row subset that includes both ends of every
    128-row tile boundary touched."""
    import torch
    note(f"split gemm tail round M={M} K={K} N={N}")
    rng = np.random.default_rng(K + N + M)
    w = _weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    ws = split_dev(w, N, K, dev)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split(ws, to_dev(xq, dev), y, K, N, M)
    got = host(y).reshape(M, N)
    rows = np.unique(np.concatenate([rng.choice(N, 200, replace=False), [0, 127, 128, N - 129, N - 128, N - 1]]))
    nb = K // 32
    wsub = np.ascontiguousarray(w.reshape(N, nb * 18)[rows]).reshape(-1)
    exp = c_oracle.matmul(wsub, xq, K, rows.size, M)
    np.testing.assert_allclose(got[:, rows], exp, rtol=RTOL, atol=ATOL)
    assert np.all(np.isfinite(got))


def test_split_rejects_unsupported(dev):
    import torch
    K, N, M = 4096, 64, 1
    ws = torch.zeros(N * (K // 32) * 18 + 16, dtype=torch.uint8, device=dev)
    xq = torch.zeros(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    y = torch.full((M * N,), 5.0, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        capi.mat_mul_split(ws[4:], xq, y, K, N, M)
    assert bool((y == 5.0).all())
