"""On-disk Q4_0 weights, host side (no GPU): the host quantizer against the C
oracle, closed-form round trips, the safetensors reader / writer against the stock
`safetensors` package, the streaming repacker and its error paths."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import json
import struct

import numpy as np
import pytest

from jjjetson_ops_amd import weights as W
from oracle import c_oracle, oracle_np
from _ties import q4_tie_matrix, q4_tie_cases


def _nibbles(q: np.ndarray) -> np.ndarray:
    b = q.reshape(-1, 18)
    return np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4], axis=1).reshape(-1)


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("rows,cols,threads", [(1, 32, 1), (7, 96, 1), (64, 4096, 0), (300, 1024, 3)])
def test_host_quantizer_matches_oracle(rows, cols, threads):
    rng = np.random.default_rng(rows * cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    got = W.quantize_q4_0(w, threads)
    assert got.shape == (rows, cols // 32, 18)
    assert np.array_equal(got.reshape(-1), c_oracle.quantize_q4_0(w))
    assert np.array_equal(got.reshape(-1), oracle_np.quantize_q4_0(w))


def test_host_quantizer_special_blocks():
    """All-zero block (d = -0.0, nibbles 8), ties of |max| with opposite signs (the
    first wins), huge values (fp16 d overflows to inf), subnormal scales, NaN."""
    rows, cols = 6, 64
    w = np.zeros((rows, cols), np.float32)
    w[1, 0:32] = np.linspace(-1, 1, 32)
    w[1, 5], w[1, 9] = -3.0, 3.0          # tie: -3 comes first, d = 0.375
    w[2, 32:64] = 3e5                       # mx = -7e5 below: d = 87500 > 65504 -> fp16 +inf
    w[2, 40] = -7e5
    w[3, 0:32] = 1e-7                       # subnormal fp16 scale
    w[3, 3] = -2e-7
    w[4, 0:32] = np.float32(np.nan)
    w[4, 7] = 1.0
    w[5, 0:32] = -0.0
    got = W.quantize_q4_0(w).reshape(-1)
    exp = c_oracle.quantize_q4_0(w)
    assert np.array_equal(got, exp)
    b = got.reshape(rows, 2, 18)
    d = b[..., 0:2].copy().view(np.float16)[..., 0]
    assert d[0, 0] == 0 and np.signbit(d[0, 0])             # 0 / -8 = -0
    assert np.all(_nibbles(b[0]) == 8)
    assert d[1, 0] == np.float16(-3.0 / -8.0)                # first of the |3| tie
    assert np.isinf(d[2, 1]) and d[2, 1] > 0                 # -7e5 / -8 overflows fp16
    assert d[3, 0] == np.float16(np.float32(-2e-7) / np.float32(-8.0))


def test_closed_form_round_trip():
    """Values already on a block's Q4_0 grid, d * (n - 8) with the -8 end present
    (so mx = -8d and the recovered d is d itself), quantize back to exactly n."""
    rng = np.random.default_rng(5)
    rows, cols = 16, 256
    d = (2.0 ** rng.integers(-12, -2, (rows, cols // 32))).astype(np.float32)   # exact in fp16
    n = rng.integers(0, 16, (rows, cols // 32, 32))
    n[:, :, 0] = 0                                              # value -8d: the block's max magnitude
    n[:, :, 1:][n[:, :, 1:] == 0] = 1                           # a single -8d per block
    w = ((n - 8) * d[..., None]).astype(np.float32).reshape(rows, cols)
    got = W.quantize_q4_0(w)
    assert np.array_equal(_nibbles(got), n.reshape(-1))          # element order 0..31 per block
    dd = got[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    assert np.array_equal(dd, d)
    assert np.array_equal(oracle_np.dequantize_q4_0(got.reshape(-1), rows, cols), w)


def test_rounding_boundary_cases():
    """Crafted values where a fused multiply-add would move a nibble down by one:
    the two-rounding rule (product, then + 8.5) is what the quantizer computes."""
    w, idx, nib = q4_tie_matrix(32, 512, seed=11, per_block=2)
    exp = c_oracle.quantize_q4_0(w)
    assert np.array_equal(_nibbles(exp)[idx], nib)               # the oracle pins the rule
    got = W.quantize_q4_0(w, 4).reshape(-1)
    assert np.array_equal(got, exp)


def test_tie_cases_separate_the_two_rules():
    """The crafted cases really distinguish the rules: the fused form gives n - 1."""
    rng = np.random.default_rng(3)
    for mx, v, nt in q4_tie_cases(rng, 50):
        idv = np.float32(1.0) / (mx / np.float32(-8.0))
        two = np.float32(np.float32(v * idv) + np.float32(8.5))
        fused = np.float32(np.float64(v) * np.float64(idv) + 8.5)
        assert int(two) == nt and int(fused) == nt - 1


def test_quantizer_rejects_bad_shapes():
    with pytest.raises(ValueError):
        W.quantize_q4_0(np.zeros((2, 48), np.float32))
    with pytest.raises(ValueError):
        W.quantize_q4_0(np.zeros(64, np.float32))
    assert W.q4_0_bytes(3, 64) == 3 * 2 * 18
    assert W.q4_0_bytes(3, 48) == -1 and W.q4_0_bytes(0, 32) == -1


# ------------------------------------------------------------------ file format
def _sample(rng):
    return {
        "embed": (rng.standard_normal((10, 64)) * 0.1).astype(np.float32),
        "layer0.w_q": (rng.standard_normal((96, 128)) * 0.02).astype(np.float32),
        "layer0.w_input_layernorm": rng.standard_normal(64).astype(np.float32),
        "layer0.w_up": (rng.standard_normal((160, 64)) * 0.02).astype(np.float32),
    }


def test_writer_output_reads_with_stock_safetensors(tmp_path):
    from safetensors import safe_open
    from safetensors.numpy import load_file
    rng = np.random.default_rng(0)
    t = _sample(rng)
    q = W.quantize_q4_0(t["layer0.w_q"])
    mixed = dict(t)
    mixed["layer0.w_q"] = W.WeightTensor(W.Q4_0, (96, 128), q)
    p = tmp_path / "m.safetensors"
    W.write_safetensors(p, mixed)
    stock = load_file(str(p))
    for k, v in t.items():
        if k == "layer0.w_q":
            assert stock[k].dtype == np.uint8 and stock[k].shape == (96, 4, 18)
            assert np.array_equal(stock[k], q)
        else:
            assert np.array_equal(stock[k], v)
    with safe_open(str(p), "np") as f:
        assert f.metadata() == {"q4_0:layer0.w_q": "Q4_0"}
    # data section is 8-byte aligned, as the format recommends
    hs = struct.unpack("<Q", p.read_bytes()[:8])[0]
    assert hs % 8 == 0


def test_reader_reads_stock_files(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(1)
    t = _sample(rng)
    q = W.quantize_q4_0(t["layer0.w_up"])
    stock = dict(t)
    stock["layer0.w_up"] = q
    p = tmp_path / "s.safetensors"
    save_file(stock, str(p), metadata={"q4_0:layer0.w_up": "Q4_0", "format": "np"})
    got = W.read_safetensors(p)
    assert list(sorted(got)) == sorted(t)
    for k, v in t.items():
        g = got[k]
        if k == "layer0.w_up":
            assert g.dtype == W.Q4_0 and g.dims == (160, 64) and np.array_equal(g.data, q)
        else:
            assert g.dtype == W.F32 and g.dims == v.shape and np.array_equal(g.data, v)


def test_unmarked_u8_and_other_dtypes_are_rejected(tmp_path):
    from safetensors.numpy import save_file
    p = tmp_path / "u8.safetensors"
    save_file({"w": np.zeros((4, 2, 18), np.uint8)}, str(p))          # U8 without the Q4_0 marker
    with pytest.raises(RuntimeError, match="unsupported dtype U8"):
        W.read_safetensors(p)
    save_file({"w": np.zeros((4, 32), np.float16)}, str(p))
    with pytest.raises(RuntimeError, match="unsupported dtype F16"):
        W.read_safetensors(p)
    save_file({"w": np.zeros((4, 3, 17), np.uint8)}, str(p), metadata={"q4_0:w": "Q4_0"})
    with pytest.raises(RuntimeError, match=r"\[rows, cols/32, 18\]"):
        W.read_safetensors(p)


def _raw_file(p, header: dict, data: bytes):
    h = json.dumps(header).encode()
    p.write_bytes(struct.pack("<Q", len(h)) + h + data)


def test_malformed_files_are_rejected(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x01\x02")
    with pytest.raises(RuntimeError, match="8-byte"):
        W.read_safetensors(p)
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(RuntimeError, match="header length"):
        W.read_safetensors(p)
    _raw_file(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8)
    with pytest.raises(RuntimeError, match="past the data section"):
        W.read_safetensors(p)
    _raw_file(p, {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, b"\0" * 16)
    with pytest.raises(RuntimeError, match="shape needs"):
        W.read_safetensors(p)
    h = b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]'
    p.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 16)
    with pytest.raises(RuntimeError, match="malformed"):
        W.read_safetensors(p)
    _raw_file(p, {"a": {"dtype": "F32", "shape": [4.5], "data_offsets": [0, 16]}}, b"\0" * 16)
    with pytest.raises(RuntimeError, match="non-integer"):
        W.read_safetensors(p)
    with pytest.raises(RuntimeError, match="cannot open"):
        W.read_safetensors(tmp_path / "missing.safetensors")


def test_json_escapes_and_empty_file(tmp_path):
    p = tmp_path / "e.safetensors"
    name = 'we"ird\\name\té\U0001F600'
    W.write_safetensors(p, {name: np.arange(32, dtype=np.float32).reshape(1, 32)})
    got = W.read_safetensors(p)
    assert list(got) == [name] and np.array_equal(got[name].data, np.arange(32, dtype=np.float32).reshape(1, 32))
    from safetensors.numpy import load_file
    assert list(load_file(str(p))) == [name]
    W.write_safetensors(p, {})
    assert W.read_safetensors(p) == {}


def test_writer_rejects_bad_tensors(tmp_path):
    p = tmp_path / "w.safetensors"
    with pytest.raises(RuntimeError, match="Q4_0 tensor"):
        W.write_safetensors(p, {"x": W.WeightTensor(W.Q4_0, (4, 48), np.zeros(4 * 27, np.uint8))})
    with pytest.raises(RuntimeError, match="nbytes"):
        W.write_safetensors(p, {"x": W.WeightTensor(W.Q4_0, (4, 64), np.zeros(10, np.uint8))})


def test_repacker_streams_and_quantizes(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(2)
    t = _sample(rng)
    src = tmp_path / "f32.safetensors"
    save_file(t, str(src))
    # all eligible 2-D tensors (embed 64 cols, w_q, w_up); the 1-D norm stays F32
    out = tmp_path / "q.safetensors"
    W.quantize_file(src, out, num_threads=2)
    got = W.read_safetensors(out)
    for k, v in t.items():
        if v.ndim == 2:
            assert got[k].dtype == W.Q4_0 and got[k].dims == v.shape
            assert np.array_equal(got[k].data.reshape(-1), c_oracle.quantize_q4_0(v))
        else:
            assert got[k].dtype == W.F32 and np.array_equal(got[k].data, v)
    # only the named ones
    out2 = tmp_path / "q2.safetensors"
    W.quantize_file(src, out2, names=["layer0.w_up"])
    got2 = W.read_safetensors(out2)
    assert got2["layer0.w_up"].dtype == W.Q4_0
    assert got2["layer0.w_q"].dtype == W.F32 and got2["embed"].dtype == W.F32
    # re-running the repacker on its own output keeps Q4_0 tensors as they are
    out3 = tmp_path / "q3.safetensors"
    W.quantize_file(out2, out3, names=["layer0.w_q"])
    got3 = W.read_safetensors(out3)
    assert np.array_equal(got3["layer0.w_up"].data, got2["layer0.w_up"].data)
    assert got3["layer0.w_q"].dtype == W.Q4_0
    with pytest.raises(RuntimeError, match="no tensor named"):
        W.quantize_file(src, out2, names=["nope"])
    with pytest.raises(RuntimeError, match="not a 2-D F32"):
        W.quantize_file(src, out2, names=["layer0.w_input_layernorm"])


def test_overflowing_shapes_are_rejected(tmp_path):
    """A header whose shape overflows the byte count (numel*4 for F32, cols*32 for
    Q4_0) must not wrap around to a size that matches its data_offsets."""
    p = tmp_path / "big.safetensors"
    a, b = 5 * 5581 * 8681, 49477 * 384773   # a*b = 2^62 + 1: a*b*4 wraps to 4 in 64 bits
    assert a * b == (1 << 62) + 1
    _raw_file(p, {"a": {"dtype": "F32", "shape": [a, b], "data_offsets": [0, 4]}}, b"\0" * 4)
    with pytest.raises(RuntimeError, match="too large|unsupported shape"):
        W.read_safetensors(p)
    c = (1 << 58) + 1                      # cols/32 blocks whose cols*32 overflows int64
    _raw_file(p, {"__metadata__": {"q4_0:w": "Q4_0"},
                  "w": {"dtype": "U8", "shape": [1, c, 18], "data_offsets": [0, 18]}}, b"\0" * 18)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        W.read_safetensors(p)


def test_repacker_refuses_in_place_and_leaves_no_partial_file(tmp_path):
    from safetensors.numpy import save_file
    src = tmp_path / "f32.safetensors"
    save_file({"w": np.ones((4, 64), np.float32)}, str(src))
    before = src.read_bytes()
    with pytest.raises(RuntimeError, match="names the input file"):
        W.quantize_file(src, src)
    assert src.read_bytes() == before
    # a failing run (unknown tensor name) writes nothing at out_path
    out = tmp_path / "q.safetensors"
    with pytest.raises(RuntimeError, match="no tensor named"):
        W.quantize_file(src, out, names=["nope"])
    assert not out.exists()
    assert sorted(p.name for p in tmp_path.iterdir()) == ["f32.safetensors"]
    # a successful run replaces an existing output atomically
    out.write_bytes(b"old")
    W.quantize_file(src, out)
    assert W.read_safetensors(out)["w"].dtype == W.Q4_0
    assert sorted(p.name for p in tmp_path.iterdir()) == ["f32.safetensors", "q.safetensors"]
