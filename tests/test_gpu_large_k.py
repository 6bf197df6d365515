"""Parity past the decode kernels' K limits: ncols_k above 16384 (the GEMV's limit and
the fused quantize+GEMV's) and above 4096 (the LDS-resident skinny kernel's activation
window), on both weight layouts, against the CPU oracle.  K = 16512 is not a multiple
of 256 (the skinny kernels' requirement)."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import numpy as np
import pytest

from jjjetson_ops_amd import capi
from oracle import c_oracle

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4
CASES = [(K, N, M) for K, N in ((16512, 40), (20480, 64), (28672, 33)) for M in (1, 2, 5, 16, 17)]


def _data(K, N, M):
    w = c_oracle.quantize_q4_0((np.random.default_rng(K + N).standard_normal((N, K)) * 0.02).astype(np.float32))
    x = np.random.default_rng(K + M).standard_normal((M, K)).astype(np.float32)
    return w, x


@pytest.mark.parametrize("K,N,M", CASES)
def test_large_k_block_layout(K, N, M, dev):
    """AUTO from Q8_1 bytes, and the fp32 entry (quantize into the workspace, then AUTO;
    at M = 1 the fused GEMV does not apply above K = 16384)."""
    import torch
    print(f"[case] large K block K={K} N={N} M={M}", flush=True)
    w, x = _data(K, N, M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    w_d = torch.from_numpy(w).to(dev)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul(w_d, torch.from_numpy(xq).to(dev), y, K, N, M)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL)
    ws = torch.empty(xq.size, dtype=torch.uint8, device=dev)
    y.fill_(float("nan"))
    capi.mat_mul_f32(w_d, torch.from_numpy(x).to(dev), ws, y, K, N, M)
    torch.cuda.synchronize()
    assert np.array_equal(ws.cpu().numpy(), xq)
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("K,N,M", CASES)
def test_large_k_split_layout(K, N, M, dev):
    import torch
    print(f"[case] large K split K={K} N={N} M={M}", flush=True)
    w, x = _data(K, N, M)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    ws_w = torch.empty(w.size, dtype=torch.uint8, device=dev)
    capi.q4_0_to_split(torch.from_numpy(w).to(dev), ws_w, N, K)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split(ws_w, torch.from_numpy(xq).to(dev), y, K, N, M)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL)
    ws = torch.empty(xq.size, dtype=torch.uint8, device=dev)
    y.fill_(float("nan"))
    capi.mat_mul_split_f32(ws_w, torch.from_numpy(x).to(dev), ws, y, K, N, M)
    torch.cuda.synchronize()
    assert np.array_equal(ws.cpu().numpy(), xq)
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL)
