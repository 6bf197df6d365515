"""Build recipe of the gfx950 library and its Python modules (in-tree).

Outputs (next to this file):
  libjjjetson_ops_amd.so             HIP kernels + C ABI (hipcc, gfx950 only)
  q8_1_me<ext>.so, mm_q4_0_q8_1_me<ext>.so   pybind11 modules linked to it

Run:  python -m jjjetson_ops_amd.build      (or call build_all()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB = PKG / "libjjjetson_ops_amd.so"

HIP_SOURCES = ["quantize_q8_1.hip", "gemv_q4_0_q8_1.hip", "gemm_skinny_q4_0_q8_1.hip", "gemm_skinny_persist.hip", "gemm_q4_0_q8_1_mfma.hip", "gemm_q4_0_q8_1_mfma64.hip", "moe_route.hip",
               "quantize_q4_0.hip", "q4_0_split.hip", "gemm_q4s_mfma.hip", "weights_q4_0.cpp", "capi.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed-FP32 (v_pk_*_f32) code generation on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # Keep MFMA sources/results in arch VGPRs: the epilogues read every MFMA result
    # with VALU ops, which cannot take AGPR operands (no v_accvgpr copies).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
PYBIND_MODULES = {"q8_1_me": "bind_q8_1.cpp", "mm_q4_0_q8_1_me": "bind_mm_q4_0_q8_1.cpp"}


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    noise = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build_lib(jobs: int = 4) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_pybind() -> list[Path]:
    import pybind11

    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    py_inc = sysconfig.get_paths()["include"]
    outs = []
    for mod, src in PYBIND_MODULES.items():
        out = PKG / f"{mod}{ext}"
        tmp = PKG / f".{mod}.tmp.so"
        _run([
            "g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-fvisibility=hidden",
            f"-I{pybind11.get_include()}", f"-I{py_inc}", f"-I{INCLUDE}",
            str(CSRC / src), "-o", str(tmp),
            f"-L{PKG}", "-ljjjetson_ops_amd", "-Wl,-rpath,$ORIGIN",
        ])
        os.replace(tmp, out)
        outs.append(out)
    return outs


def build_all() -> None:
    build_lib()
    build_pybind()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB}")
