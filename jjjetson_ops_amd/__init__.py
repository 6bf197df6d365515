"""MI355X (gfx950) Q4_0 x Q8_1 quantized matmul path.

Python surfaces:
  * ``q8_1_me`` / ``mm_q4_0_q8_1_me`` — pybind11 modules with the reference's
    op names and buffer layouts (host numpy buffers, synchronous);
  * ``jjjetson_ops_amd.capi`` — device-tensor wrappers of the C ABI
    (asynchronous on torch's current stream).
"""
from pathlib import Path

__all__ = ["capi", "q4_0", "PKG_DIR"]
PKG_DIR = Path(__file__).resolve().parent

from . import capi, q4_0  # noqa: E402
