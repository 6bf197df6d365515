"""The device entries inside a captured HIP graph: every replay must reproduce the
eager result bit for bit (no memset nodes, no hidden allocation, no state carried
between calls).  Each graph is replayed several times with unrelated eager work and
synchronisations in between."""
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


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _w(N, K, rng):
    return c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))


def _replays_match(fn, outs, dev, n_replays=3):
    import torch
    fn()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    for o in outs:
        o.fill_(float("nan")) if o.dtype.is_floating_point else o.zero_()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
    for r in range(n_replays):
        for o in outs:
            o.fill_(float("nan")) if o.dtype.is_floating_point else o.zero_()
        torch.randn(1 << 20, device=dev).sum().item()  # unrelated eager work
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"replay {r} differs"


@pytest.mark.parametrize("M", [1, 3, 16, 200])
def test_graph_matmul_f32(M, dev):
    import torch
    note(f"graph mat_mul_f32 M={M}")
    K, N = 1024, 384
    rng = np.random.default_rng(M)
    w = torch.from_numpy(_w(N, K, rng)).to(dev)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev)
    xq = torch.empty(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    y = torch.empty(M * N, dtype=torch.float32, device=dev)
    _replays_match(lambda: capi.mat_mul_f32(w, x, xq, y, K, N, M), [y, xq], dev)


@pytest.mark.parametrize("T", [48, 3])  # MFMA tiles; routed GEMVs (decode)
def test_graph_moe_ffn(T, dev):
    import torch
    note(f"graph moe_ffn T={T}")
    H, I, E, k = 256, 256, 8, 2
    rng = np.random.default_rng(9)
    wg = torch.from_numpy(np.concatenate([_w(I, H, rng) for _ in range(E)])).to(dev)
    wu = torch.from_numpy(np.concatenate([_w(I, H, rng) for _ in range(E)])).to(dev)
    wd = torch.from_numpy(np.concatenate([_w(H, I, rng) for _ in range(E)])).to(dev)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dev)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    ws = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, k), dtype=torch.uint8, device=dev)
    y = torch.empty(T * H, dtype=torch.float32, device=dev)
    _replays_match(lambda: capi.moe_ffn(x, lg, wg, wu, wd, y, T, H, I, E, k, ws), [y], dev)


@pytest.mark.parametrize("M", [1, 5, 16, 200])
def test_graph_split_layout_matmul_f32(M, dev):
    """The split-layout entries in a graph: the fused decode step (the headline path),
    the skinny kernel and the MFMA GEMM."""
    import torch
    note(f"graph split mat_mul_f32 M={M}")
    K, N = 1024, 384
    rng = np.random.default_rng(100 + M)
    w = torch.from_numpy(_w(N, K, rng)).to(dev)
    ws = torch.empty_like(w)
    capi.q4_0_to_split(w, ws, N, K)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev)
    xq = torch.empty(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    y = torch.empty(M * N, dtype=torch.float32, device=dev)
    _replays_match(lambda: capi.mat_mul_split_f32(ws, x, xq, y, K, N, M), [y, xq], dev)


@pytest.mark.parametrize("T", [48, 3])
def test_graph_moe_ffn_split_layout(T, dev):
    import torch
    note(f"graph moe_ffn split T={T}")
    H, I, E, k = 256, 256, 8, 2
    rng = np.random.default_rng(19)
    mats = []
    for rows, cols in ((I, H), (I, H), (H, I)):
        w = torch.from_numpy(np.concatenate([_w(rows, cols, rng) for _ in range(E)])).to(dev)
        s = torch.empty_like(w)
        capi.q4_0_to_split(w, s, E * rows, cols)
        mats.append(s)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dev)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    wsp = torch.empty(capi.moe_ffn_workspace_bytes(T, H, I, E, k), dtype=torch.uint8, device=dev)
    y = torch.empty(T * H, dtype=torch.float32, device=dev)
    _replays_match(lambda: capi.moe_ffn(x, lg, *mats, y, T, H, I, E, k, wsp, split=True), [y], dev)
