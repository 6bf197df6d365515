"""The split Q4_0 weight layout (host side, no GPU): the repackers are exact
inverses, every byte lands where the layout says, and the values a split matrix
dequantizes to are the Q4_0 matrix's own."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import numpy as np
import pytest

from jjjetson_ops_amd import capi, q4_0
from oracle import c_oracle


def test_split_bytes():
    assert capi.lib().q4_0_split_bytes(3, 64) == 3 * 2 * 18
    assert capi.lib().q4_0_split_bytes(3, 48) == -1
    assert capi.lib().q4_0_split_bytes(0, 64) == -1


@pytest.mark.parametrize("N,K", [(1, 32), (7, 96), (33, 4096), (5, 11008)])
def test_split_round_trip_and_placement(N, K):
    rng = np.random.default_rng(N * 7 + K)
    w = rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8)
    s = capi.q4_0_to_split_host(w, N, K)
    assert s.size == w.size
    nbt = N * (K // 32)
    blocks = w.reshape(nbt, 18)
    # qs plane first (16 bytes per block, row-major), then the fp16 scales
    assert np.array_equal(s[: nbt * 16].reshape(nbt, 16), blocks[:, 2:])
    assert np.array_equal(s[nbt * 16:].reshape(nbt, 2), blocks[:, :2])
    assert np.array_equal(capi.q4_0_from_split_host(s, N, K), w)


def test_split_dequantizes_to_the_same_values():
    N, K = 16, 256
    rng = np.random.default_rng(3)
    w = c_oracle.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    s = capi.q4_0_to_split_host(w, N, K)
    nbt = N * (K // 32)
    qs = s[: nbt * 16].reshape(N, K // 32, 16)
    d = s[nbt * 16:].view(np.float16).reshape(N, K // 32).astype(np.float32)
    lo = (qs & 0x0F).astype(np.float32) - 8.0   # elements 0..15 of each block
    hi = (qs >> 4).astype(np.float32) - 8.0     # elements 16..31
    deq = (np.concatenate([lo, hi], axis=2) * d[:, :, None]).reshape(N, K)
    assert np.array_equal(deq, q4_0.dequantize_q4_0_np(w, N, K))


def test_split_rejects_bad_shapes():
    w = np.zeros(18 * 4, np.uint8)
    with pytest.raises(ValueError):
        capi.q4_0_to_split_host(w, 2, 48)
    with pytest.raises(ValueError):
        capi.q4_0_to_split_host(w, 4, 64)  # buffer too small
