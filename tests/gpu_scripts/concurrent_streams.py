"""Run by tests/test_gpu_concurrency.py in a fresh process: several host threads,
each on its own HIP stream, make their first and later calls into the library at
the same time (one-time per-kernel set-up included).  Every result must equal the
same call made alone beforehand, bit for bit.  Prints "ok"."""
import sys
import threading
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from jjjetson_ops_amd import capi  # noqa: E402

dev = torch.device("cuda:0")
rng = np.random.default_rng(5)
CASES = [  # (K, N, M, algo)
    (4096, 512, 1, capi.ALGO_GEMV),
    (4096, 1024, 4, capi.ALGO_GEMV),
    (4096, 768, 8, capi.ALGO_SKINNY),
    (4096, 1024, 16, capi.ALGO_SKINNY_LDS),
    (2048, 1024, 256, capi.ALGO_MFMA),
    (1024, 640, 100, capi.ALGO_AUTO),
    # split-layout weights (AUTO over the split kernels: GEMV, skinny, GEMM)
    (4096, 512, 1, "split"),
    (4096, 1024, 8, "split"),
    (2048, 512, 200, "split"),
]
data = []
for K, N, M, algo in CASES:
    w = torch.from_numpy(rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8))
    w.view(-1, 18)[:, 0:2] = torch.tensor([0x66, 0x22], dtype=torch.uint8)  # a finite fp16 scale
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev)
    xq = torch.empty(capi.q8_1_output_bytes([K, M]), dtype=torch.uint8, device=dev)
    capi.quantize_q8_1(x, xq, [K, M])
    w = w.to(dev)
    if algo == "split":
        ws = torch.empty_like(w)
        capi.q4_0_to_split(w, ws, N, K)
        w = ws
    data.append((w, xq))
torch.cuda.synchronize()

# Threads start together; each one's first call is also the process's first call of
# its kernel, so one-time set-up runs concurrently.
barrier = threading.Barrier(len(CASES))
results, errors = {}, []


def worker(i):
    K, N, M, algo = CASES[i]
    w, xq = data[i]
    s = torch.cuda.Stream()
    outs = []
    try:
        barrier.wait()
        with torch.cuda.stream(s):
            for _ in range(20):
                y = torch.empty(M * N, dtype=torch.float32, device=dev)
                if algo == "split":
                    capi.mat_mul_split(w, xq, y, K, N, M, stream=s)
                else:
                    capi.mat_mul(w, xq, y, K, N, M, algo=algo, stream=s)
                outs.append(y)
        s.synchronize()
        results[i] = [o.cpu() for o in outs]
    except Exception as e:  # reported by the parent
        errors.append(f"case {i}: {e!r}")


threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(CASES))]
for t in threads:
    t.start()
for t in threads:
    t.join()
if errors:
    sys.exit("; ".join(errors))
for i, (K, N, M, algo) in enumerate(CASES):
    w, xq = data[i]
    y = torch.empty(M * N, dtype=torch.float32, device=dev)
    if algo == "split":
        capi.mat_mul_split(w, xq, y, K, N, M)
    else:
        capi.mat_mul(w, xq, y, K, N, M, algo=algo)
    torch.cuda.synchronize()
    ref = y.cpu()
    for r, o in enumerate(results[i]):
        if not torch.equal(o.view(torch.int32), ref.view(torch.int32)):
            sys.exit(f"case {CASES[i]} call {r}: differs from the lone call")
print("ok", flush=True)
