"""Writes the small golden fixtures under tests/golden/ from the C oracle.

  q8_1_seed24_2048x13.npz : the reference test's input (tests/test_q8_1.py:71-73,
                            np.random.seed(24), randn(2048,13,1,1), Fortran order)
                            and its Q8_1 bytes (208 blocks).
  mmq_small.npz           : a K=256, N=48, M=3 matmul case (Q4_0 bytes, Q8_1 bytes,
                            per-block int32 sums, fp32 y) for GPU smoke checks.

Run:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import c_oracle  # noqa: E402


def main():
    np.random.seed(24)
    x = np.asfortranarray(np.random.randn(2048, 13, 1, 1).astype(np.float32))
    q = c_oracle.quantize_q8_1(x, [2048, 13, 1, 1])
    np.savez_compressed(HERE / "q8_1_seed24_2048x13.npz", q8_1=q)

    K, N, M = 256, 48, 3
    rng = np.random.default_rng(2024)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w = c_oracle.quantize_q4_0(wf)
    xa = rng.standard_normal((M, K)).astype(np.float32)
    xa[:, 5] *= 20
    xq = c_oracle.quantize_q8_1(xa, [K, M, 1, 1])
    np.savez_compressed(HERE / "mmq_small.npz", K=K, N=N, M=M, w=w, x=xa, xq=xq,
                        sumi=c_oracle.block_sums(w, xq, K, N, M), y=c_oracle.matmul(w, xq, K, N, M))


if __name__ == "__main__":
    main()
