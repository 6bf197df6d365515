"""The C ABI from a plain C program (gcc, no C++ or Python in between): the
header compiles as C and the Q4_0 weight entries work end to end (no GPU)."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import shutil
import subprocess
from pathlib import Path

import pytest

from jjjetson_ops_amd import capi

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_c_client_weights_roundtrip(tmp_path):
    exe = tmp_path / "weights_roundtrip"
    lib = capi.LIB_PATH
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-O1", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "c" / "weights_roundtrip.c"), "-o", str(exe),
                    f"-L{lib.parent}", "-ljjjetson_ops_amd", f"-Wl,-rpath,{lib.parent}"], check=True)
    r = subprocess.run([str(exe), str(tmp_path / "w.safetensors")], capture_output=True, text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.strip() == "ok"


@pytest.mark.gpu
@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_c_client_linear_q4_0(tmp_path):
    """linear_q4_0_forward_host called from C on a gfx950 GPU."""
    exe = tmp_path / "linear_q4_0"
    lib = capi.LIB_PATH
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-O1", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "c" / "linear_q4_0.c"), "-o", str(exe), "-lm",
                    f"-L{lib.parent}", "-ljjjetson_ops_amd", f"-Wl,-rpath,{lib.parent}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
