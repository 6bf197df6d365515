"""The C-ABI library and the pybind11 modules load, export every declared
symbol, and validate arguments — all without a GPU (no compute calls)."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from jjjetson_ops_amd import capi
from oracle import c_oracle

HEADER = Path(__file__).resolve().parents[1] / "include" / "jjjetson_ops_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_what_capi_binds():
    assert declared_functions() == sorted(capi.EXPORTED_SYMBOLS)


def test_header_constants_match_capi():
    """Every JJO_* status, algorithm and weight-dtype constant of the header has the
    same value in capi.py (JJO_ALGO_X -> ALGO_X, JJO_WEIGHT_DTYPE_X -> WEIGHT_DTYPE_X,
    status codes under their own names)."""
    consts = dict(re.findall(r"^#define\s+JJO_([A-Z0-9_]+)\s+(-?\d+)", HEADER.read_text(), flags=re.M))
    assert any(k.startswith("ALGO_") for k in consts)
    for name, value in consts.items():
        if name.startswith(("ALGO_", "WEIGHT_DTYPE_")):
            assert getattr(capi, name) == int(value), name
        elif name.startswith("ERR_") or name == "OK":
            assert getattr(capi, "JJO_" + name) == int(value), name


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(str(capi.LIB_PATH))
    for name in declared_functions():
        assert hasattr(L, name), name
    assert "gfx950" in capi.version()


def test_q8_1_output_bytes():
    assert capi.q8_1_output_bytes([2048, 13, 1, 1]) == 208 * 144
    assert capi.q8_1_output_bytes([4096]) == 32 * 144
    assert capi.q8_1_output_bytes([160, 3]) == 3 * 2 * 144
    assert capi.q8_1_output_bytes([640, 2, 2, 3]) == 6 * 2 * 4 * 2 * 144  # slice stride ne1*4*ceil(K/512)
    for d in ([48, 1], [0, 1], [128, -1], []):
        assert capi.q8_1_output_bytes(d) == -1
    for d in ([2048, 13, 1, 1], [160, 3], [640, 2, 2, 3]):
        assert capi.q8_1_output_bytes(d) == c_oracle.lib().oracle_q8_1_n_blocks(
            c_oracle._p(c_oracle.dims4(d))) * 144


def test_parse_matches_oracle():
    rng = np.random.default_rng(0)
    raw = rng.integers(0, 256, 37 * 144, dtype=np.uint8)
    raw.reshape(37, 144)[:, 0:16] = np.float16(rng.standard_normal((37, 8))).view(np.uint8).reshape(37, 16)
    a = capi.parse_q8_1(raw, 37)
    b = c_oracle.parse_q8_1(raw, 37)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_pybind_parse_matches_oracle():
    import q8_1_me
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 256, 5 * 144, dtype=np.uint8)
    raw.reshape(5, 144)[:, 0:16] = np.float16(rng.standard_normal((5, 8))).view(np.uint8).reshape(5, 16)
    qs, d, s = q8_1_me.parse(raw, 5)
    assert qs.shape == (5, 128) and qs.dtype == np.int8
    assert d.shape == (5, 4) and d.dtype == np.float32 and s.dtype == np.float32
    qr, dr, sr = c_oracle.parse_q8_1(raw, 5)
    assert np.array_equal(qs, qr) and np.array_equal(d, dr) and np.array_equal(s, sr)


def _rc(fn, *args):
    return fn(*args)


def test_device_entries_validate_before_touching_a_device():
    L = capi.lib()
    d = (ctypes.c_int64 * 2)(48, 1)
    assert L.q8_1_device(ctypes.c_void_p(16), ctypes.c_void_p(16), d, 2, None) == capi.JJO_ERR_INVALID_ARG
    assert b"multiple of 32" in L.jjo_last_error()
    d = (ctypes.c_int64 * 2)(128, 1)
    assert L.q8_1_device(ctypes.c_void_p(8), ctypes.c_void_p(16), d, 2, None) == capi.JJO_ERR_INVALID_ARG
    assert b"16-byte aligned" in L.jjo_last_error()
    assert L.mat_mul_q4_0_q8_1_device(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 96, 4, 1,
                                      None) == capi.JJO_ERR_INVALID_ARG
    assert L.mat_mul_q4_0_q8_1_device(ctypes.c_void_p(16), ctypes.c_void_p(16), None, 128, 4, 1,
                                      None) == capi.JJO_ERR_INVALID_ARG
    assert L.mat_mul_q4_0_q8_1_device_algo(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 128,
                                           4, 0, 1, None) == capi.JJO_ERR_INVALID_ARG
    assert L.mat_mul_q4_0_q8_1_grouped_device(ctypes.c_void_p(16), ctypes.c_void_p(16), None, 8, None,
                                              ctypes.c_void_p(16), 128, 4, 4, None) == capi.JJO_ERR_INVALID_ARG


def test_host_matmul_validation_mirrors_reference():
    """src/cuda/mm_q4_0_q8_1.cu:326-340: dims[0]==ncols_k, ncols_k % 32, ncols_k % 128."""
    L = capi.lib()
    buf = np.zeros(1 << 16, np.uint8)
    p = ctypes.c_void_p(buf.ctypes.data)
    for K, nk in ((256, 128), (96, 96), (160, 160)):
        d = (ctypes.c_int64 * 4)(K, 1, 1, 1)
        assert L.mat_mul_q4_0_q8_1(p, p, p, p, d, 4, 8, nk) == capi.JJO_ERR_INVALID_ARG


@pytest.mark.skipif(__import__("conftest").gpu_available(), reason="checks the no-GPU error path")
def test_no_device_is_an_error_not_a_fallback():
    import q8_1_me
    x = np.zeros((128, 1), np.float32)
    out = np.zeros(144, np.uint8)
    with pytest.raises(RuntimeError):
        q8_1_me.quantize(x, out, [128, 1, 1, 1])


def test_pybind_rejects_bad_buffers():
    import mm_q4_0_q8_1_me
    import q8_1_me
    x = np.zeros((128, 2), np.float32, order="F")
    with pytest.raises(ValueError):
        q8_1_me.quantize(x, np.zeros(100, np.uint8), [128, 2, 1, 1])  # too small
    with pytest.raises(ValueError):
        q8_1_me.quantize(x, np.zeros(288, np.int8), [128, 2, 1, 1])  # wrong dtype
    w = np.zeros(8 * 4 * 18, np.uint8)
    with pytest.raises(ValueError):
        mm_q4_0_q8_1_me.mmq(w, x, np.zeros(288, np.uint8), np.zeros(16, np.float64), [128, 2, 1, 1], 8, 128)
    with pytest.raises(ValueError):  # dims[0] != ncols_k
        mm_q4_0_q8_1_me.mmq(w, x, np.zeros(288, np.uint8), np.zeros(16, np.float32), [128, 2, 1, 1], 8, 256)


def test_newer_device_entries_validate_before_touching_a_device():
    """Every device entry beyond the reference's pair rejects a malformed call with
    JJO_ERR_INVALID_ARG before it looks for a GPU (checked here, with none)."""
    L = capi.lib()
    P = ctypes.c_void_p
    a16, a8 = P(16), P(8)
    bad = capi.JJO_ERR_INVALID_ARG
    calls = {
        # split layout: weight must be 16-byte aligned; K a multiple of 128
        "mat_mul_q4_0s_q8_1_device": lambda: L.mat_mul_q4_0s_q8_1_device(a8, a16, a16, 128, 4, 1, None),
        "mat_mul_q4_0s_q8_1_f32_device": lambda: L.mat_mul_q4_0s_q8_1_f32_device(a16, a16, a16, a16, 96, 4, 1,
                                                                                  None),
        "mat_mul_q4_0s_q8_1_grouped_device": lambda: L.mat_mul_q4_0s_q8_1_grouped_device(
            a16, a16, None, 8, None, a16, 128, 4, 4, None),
        "q4_0_to_split_device": lambda: L.q4_0_to_split_device(a16, a16, 4, 100, None),
        # engine linear layers: in_features a multiple of 128, sizes positive
        "linear_q4_0_forward_device": lambda: L.linear_q4_0_forward_device(None, a16, a16, a16, a16, 96, 4, 1),
        "linear_q4_0s_forward_device": lambda: L.linear_q4_0s_forward_device(None, a16, a16, a16, a16, 128, 0, 1),
        "linear_q4_0_forward_device_noalloc": lambda: L.linear_q4_0_forward_device_noalloc(
            None, a16, a16, a16, 4096, 4, 1 << 20),
        # MoE stages
        "moe_top_k_device": lambda: L.moe_top_k_device(None, a16, a16, a16, 4, 8, 0),
        "moe_dispatch_q8_1_device": lambda: L.moe_dispatch_q8_1_device(None, a16, None, 4, 0, 128, 8, a16, a16,
                                                                       a16, None),
        "moe_q4_0_gate_up_device": lambda: L.moe_q4_0_gate_up_device(None, a16, a16, a16, a16, 8, a16, 128, 100,
                                                                     4),
        "moe_q4_0_gate_up_swiglu_q8_1_device": lambda: L.moe_q4_0_gate_up_swiglu_q8_1_device(
            None, a16, a16, a16, a16, 8, a16, 128, 100, 4),
        "swiglu_quantize_q8_1_device": lambda: L.swiglu_quantize_q8_1_device(None, a16, a16, None, 4, 100),
        "moe_combine_device": lambda: L.moe_combine_device(None, a16, a16, a16, a16, 4, 6, 2),
        "moe_q4_0_ffn_forward_device": lambda: L.moe_q4_0_ffn_forward_device(
            None, a16, a16, a16, a16, a16, a16, 4, 128, 128, 8, 2, P(256), 16),
        "moe_q4_0s_ffn_forward_device": lambda: L.moe_q4_0s_ffn_forward_device(
            None, a16, a16, a8, a16, a16, a16, 4, 128, 128, 8, 2, P(256), 1 << 30),
        # weights and diagnostics
        "quantize_q4_0_device": lambda: L.quantize_q4_0_device(None, a16, a16, 4, 100),
        "jjo_read_floor_device": lambda: L.jjo_read_floor_device(a16, -1, a16, None),
    }
    for name, call in calls.items():
        rc = call()
        assert rc == bad, f"{name}: rc {rc}, last error {L.jjo_last_error()!r}"
        assert L.jjo_last_error(), name
