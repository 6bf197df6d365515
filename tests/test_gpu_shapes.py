"""Parity over a seeded spread of shapes: every kernel that accepts a shape, and
AUTO, against the CPU oracle.  The shapes cover tails in all three dimensions
(K in 128..1024, N in 1..300, M in 1..160).  Each kernel that accepts a shape also
runs on a 4-byte-offset weight buffer, which is the layout's guaranteed alignment."""
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

rng = np.random.default_rng(2024)
SHAPES = sorted({(int(128 * rng.integers(1, 9)), int(rng.integers(1, 301)), int(rng.integers(1, 161)))
                 for _ in range(24)})


def _accepts(algo, K, N, M):
    if algo == capi.ALGO_GEMV:
        return M <= 8 and M * (K // 64) * 80 <= 150 * 1024
    if algo == capi.ALGO_SKINNY:
        return M <= 32 and K % 256 == 0
    if algo == capi.ALGO_SKINNY_LDS:
        return M <= 16 and K % 256 == 0
    return True


@pytest.mark.parametrize("K,N,M", SHAPES)
def test_every_kernel_on_shape(K, N, M, dev):
    import torch
    print(f"[case] shapes K={K} N={N} M={M}", flush=True)
    sys.stdout.flush()
    w = c_oracle.quantize_q4_0((np.random.default_rng(K * N + M).standard_normal((N, K)) * 0.02).astype(np.float32))
    x = np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    xq_d = torch.from_numpy(xq).to(dev)
    # weights at a 4-byte (not 16-byte) offset as well as at the allocation's start
    w_pad = torch.zeros(w.size + 16, dtype=torch.uint8, device=dev)
    w_pad[4:4 + w.size] = torch.from_numpy(w).to(dev)
    for algo in (capi.ALGO_AUTO, capi.ALGO_GEMV, capi.ALGO_SKINNY, capi.ALGO_SKINNY_LDS, capi.ALGO_MFMA,
                 capi.ALGO_MFMA64, capi.ALGO_MFMA32, capi.ALGO_MFMA_W32):
        if not _accepts(algo, K, N, M):
            continue
        for off in (0, 4):
            if off and algo in (capi.ALGO_SKINNY, capi.ALGO_SKINNY_LDS):
                continue  # these need 16-byte aligned weights
            w_d = torch.from_numpy(w).to(dev) if off == 0 else w_pad[4:4 + w.size]
            y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
            capi.mat_mul(w_d, xq_d, y, K, N, M, algo=algo)
            torch.cuda.synchronize()
            np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL,
                                       err_msg=f"algo={algo} offset={off}")


@pytest.mark.parametrize("K,N,M", SHAPES)
def test_split_layout_on_shape(K, N, M, dev):
    """The same shapes through the split weight layout (repacked on the device)."""
    import torch
    print(f"[case] split shapes K={K} N={N} M={M}", flush=True)
    w = c_oracle.quantize_q4_0((np.random.default_rng(K * N + M).standard_normal((N, K)) * 0.02).astype(np.float32))
    x = np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)
    xq = c_oracle.quantize_q8_1(x, [K, M])
    exp = c_oracle.matmul(w, xq, K, N, M)
    ws = torch.empty(w.size, dtype=torch.uint8, device=dev)
    capi.q4_0_to_split(torch.from_numpy(w).to(dev), ws, N, K)
    y = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    capi.mat_mul_split(ws, torch.from_numpy(xq).to(dev), y, K, N, M)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy().reshape(M, N), exp, rtol=RTOL, atol=ATOL)
