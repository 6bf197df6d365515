"""Run by tests/test_zz_no_alloc.py in a fresh process: the first call of
linear_q4_0_forward_device_noalloc on the device happens inside a HIP graph capture
(so the static buffer's address is looked up there).  The graph is replayed several
times with eager work and synchronizations between replays; every replay must equal
linear_q4_0_forward_device with a caller workspace, bit for bit.  Prints "ok"."""
import ctypes
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from jjjetson_ops_amd import capi  # noqa: E402

dev = torch.device("cuda:0")
rng = np.random.default_rng(11)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def q4_0_random(N, K):
    w = torch.from_numpy(rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8))
    w.view(-1, 18)[:, 0:2] = torch.tensor([0x66, 0x22], dtype=torch.uint8)  # finite fp16 scale
    return w.to(dev)


lib = capi.lib()
for K, N, T in ((4096, 1024, 5), (20480, 256, 1)):  # batch, and one token past the fused GEMV
    print(f"[case] capture K={K} N={N} T={T}", flush=True)
    w = q4_0_random(N, K)
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(dev)
    ws = torch.empty(capi.linear_q4_0_workspace_bytes(K, T), dtype=torch.uint8, device=dev)
    ref = torch.empty(T * N, dtype=torch.float32, device=dev)
    y = torch.full((T * N,), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.linear_q4_0_forward_device_noalloc(s, ptr(x), ptr(w), ptr(y), K, N, T)
        assert rc == 0, lib.jjo_last_error()
    rc = lib.linear_q4_0_forward_device(None, ptr(ws), ptr(x), ptr(w), ptr(ref), K, N, T)
    assert rc == 0, lib.jjo_last_error()
    torch.cuda.synchronize()
    exp = ref.cpu().numpy().view(np.uint32)
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy().view(np.uint32)
        assert np.array_equal(got, exp), f"replay {rep} differs at K={K} T={T}"
        (x * 2.0).sum().item()  # eager work between replays
    del g
print("ok", flush=True)
