"""GPU: the device Q4_0 quantizer against the C oracle (bit-exact), and a Q4_0
checkpoint written by the repacker feeding the GEMV."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import sys

import numpy as np
import pytest

from jjjetson_ops_amd import capi
from jjjetson_ops_amd import weights as W
from oracle import c_oracle
from _ties import q4_tie_matrix

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def device_quantize(w: np.ndarray, dev, offset: int = 0) -> np.ndarray:
    import torch
    rows, cols = w.shape
    n = W.q4_0_bytes(rows, cols)
    wt = torch.from_numpy(np.ascontiguousarray(w)).to(dev)
    buf = torch.full((n + offset + 64,), 0xA5, dtype=torch.uint8, device=dev)
    W.quantize_q4_0_device(wt, buf[offset:offset + n], rows, cols)
    torch.cuda.synchronize()
    b = buf.cpu().numpy()
    assert np.all(b[:offset] == 0xA5) and np.all(b[offset + n:] == 0xA5)   # nothing written outside
    return b[offset:offset + n]


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (64, 4096), (1000, 4160), (11008, 4096), (4096, 14336)])
def test_device_quantizer_matches_oracle(rows, cols, dev):
    note(f"quantize_q4_0_device rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    assert np.array_equal(device_quantize(w, dev), c_oracle.quantize_q4_0(w))


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_device_quantizer_unaligned_output(offset, dev):
    note(f"quantize_q4_0_device output offset {offset}")
    rng = np.random.default_rng(offset)
    w = (rng.standard_normal((33, 2048)) * 0.02).astype(np.float32)
    assert np.array_equal(device_quantize(w, dev, offset), c_oracle.quantize_q4_0(w))


def test_device_quantizer_boundary_and_special_blocks(dev):
    note("quantize_q4_0_device crafted rounding boundaries and special blocks")
    w, idx, nib = q4_tie_matrix(64, 1024, seed=12, per_block=3)
    got = device_quantize(w, dev)
    exp = c_oracle.quantize_q4_0(w)
    assert np.array_equal(got, exp)
    b = got.reshape(-1, 18)
    assert np.array_equal(np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4], 1).reshape(-1)[idx], nib)
    s = np.zeros((6, 64), np.float32)
    s[1, 0:32] = np.linspace(-1, 1, 32)
    s[1, 5], s[1, 9] = -3.0, 3.0
    s[2, 32:64] = 3e5
    s[2, 40] = -7e5
    s[3, 0:32] = 1e-7
    s[3, 3] = -2e-7
    s[4, 0:32] = np.float32(np.nan)
    s[4, 7] = 1.0
    s[5, 0:32] = -0.0
    s[5, 33], s[5, 62] = 0.5, -0.5        # |max| tie across lanes: the first (lane 0) wins
    assert np.array_equal(device_quantize(s, dev), c_oracle.quantize_q4_0(s))


def test_device_quantizer_rejects_bad_args(dev):
    import torch
    w = torch.zeros(64, dtype=torch.float32, device=dev)
    out = torch.zeros(64, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        W.quantize_q4_0_device(w, out, 2, 48)
    with pytest.raises(RuntimeError, match="16-byte"):
        W.quantize_q4_0_device(w[1:33], out, 1, 32)


def test_repacked_checkpoint_drives_the_gemv(tmp_path, dev):
    """F32 checkpoint -> repacker -> reader -> device -> GEMV, against the oracle
    chain; the device quantizer reproduces the file's bytes."""
    import torch
    from safetensors.numpy import save_file
    note("repacked checkpoint -> GEMV")
    rng = np.random.default_rng(7)
    K, N = 4096, 1024
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    src = tmp_path / "f32.safetensors"
    save_file({"layer0.w_up": wf, "layer0.norm": np.ones(K, np.float32)}, str(src))
    out = tmp_path / "q.safetensors"
    W.quantize_file(src, out)
    t = W.read_safetensors(out)["layer0.w_up"]
    assert t.dtype == W.Q4_0 and t.dims == (N, K)
    wq = t.data.reshape(-1)
    assert np.array_equal(device_quantize(wf, dev), wq)
    x = rng.standard_normal((1, K)).astype(np.float32)
    xq_ref = c_oracle.quantize_q8_1(x, [K, 1])
    y = torch.empty(N, dtype=torch.float32, device=dev)
    capi.mat_mul_f32(torch.from_numpy(wq).to(dev), torch.from_numpy(x).to(dev), None, y, K, N, 1)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy().reshape(1, N), c_oracle.matmul(wq, xq_ref, K, N, 1),
                               rtol=1e-3, atol=1e-4)
