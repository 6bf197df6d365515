"""The allocation-free engine linear (linear_q4_0_forward_device_noalloc) through the
C ABI against linear_q4_0_forward_device with a caller workspace: bit-identical
outputs on consecutive calls, the second one smaller (the static Q8_1 buffer keeps
the first call's bytes, which must not leak into the second), and sizes past the
static buffer refused without touching the output."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from jjjetson_ops_amd import capi
from oracle import c_oracle

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _with_workspace(x, w, K, N, T, dev):
    import torch
    ws = torch.empty(max(1, capi.linear_q4_0_workspace_bytes(K, T)), dtype=torch.uint8, device=dev)
    y = torch.full((T * N,), float("nan"), dtype=torch.float32, device=dev)
    rc = capi.lib().linear_q4_0_forward_device(None, _ptr(ws), _ptr(x), _ptr(w), _ptr(y), K, N, T)
    assert rc == 0, capi.lib().jjo_last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(T, N)


def _no_alloc(x, w, K, N, T, dev):
    import torch
    y = torch.full((T * N,), float("nan"), dtype=torch.float32, device=dev)
    rc = capi.lib().linear_q4_0_forward_device_noalloc(None, _ptr(x), _ptr(w), _ptr(y), K, N, T)
    assert rc == 0, capi.lib().jjo_last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(T, N)


@pytest.mark.parametrize("K,N,T1,T2", [(4096, 1024, 300, 37), (1024, 4096, 64, 5), (4096, 14336, 16, 2),
                                       (11008, 256, 3, 1),
                                       # one token over a row longer than the fused GEMV takes:
                                       # the quantize goes through the static buffer
                                       (20480, 192, 2, 1)])
def test_no_alloc_matches_workspace_entry(K, N, T1, T2, dev):
    import torch
    rng = np.random.default_rng(K + T1)
    w_h = c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    w = torch.from_numpy(w_h).to(dev)
    for T in (T1, T2):  # the second call is smaller
        note(f"no-alloc linear K={K} N={N} T={T}")
        x_h = rng.standard_normal((T, K)).astype(np.float32)
        x = torch.from_numpy(x_h).to(dev)
        ref = _with_workspace(x, w, K, N, T, dev)
        got = _no_alloc(x, w, K, N, T, dev)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        rows = rng.choice(N, min(N, 64), replace=False)
        wsub = np.ascontiguousarray(w_h.reshape(N, -1)[np.sort(rows)]).reshape(-1)
        exp = c_oracle.matmul(wsub, c_oracle.quantize_q8_1(x_h, [K, T]), K, rows.size, T)
        np.testing.assert_allclose(got[:, np.sort(rows)], exp, rtol=RTOL, atol=ATOL)


def test_no_alloc_rejects_oversized_batch(dev):
    import torch
    cap = capi.linear_q4_0_noalloc_max_bytes()
    K, N = 4096, 64
    T = cap // capi.linear_q4_0_workspace_bytes(K, 1) + 1
    note(f"no-alloc linear oversize T={T} (cap {cap} bytes)")
    x = torch.zeros(T * K, dtype=torch.float32, device=dev)
    w = torch.zeros(N * K // 32 * 18, dtype=torch.uint8, device=dev)
    y = torch.full((T * N,), 7.0, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="static buffer"):
        capi.linear_q4_0_noalloc(x, w, y, K, N, T)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    # the largest batch that fits still runs
    Tmax = T - 1
    x2 = torch.randn(Tmax * K, dtype=torch.float32, device=dev)
    y2 = torch.empty(Tmax * N, dtype=torch.float32, device=dev)
    capi.linear_q4_0_noalloc(x2, w, y2, K, N, Tmax)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y2).all())


def test_no_alloc_first_call_under_graph_capture():
    """In a fresh process, the entry's first call on the device (which resolves the
    static buffer's address) is made while the stream is captured into a HIP graph;
    every replay must equal the workspace entry bit for bit."""
    script = Path(__file__).resolve().parent / "gpu_scripts" / "no_alloc_graph.py"
    note("no-alloc linear: first call inside graph capture (fresh process)")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert r.stdout.strip().endswith("ok"), r.stdout[-2000:]
