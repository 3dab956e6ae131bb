"""Build the native parts of easy_as_amd in-tree (no GPU needed).

* ``easy_as_amd/libeas_hip.so`` — the C ABI of ``include/eas_hip.h``
  (HIP runtime + hiprtc), compiled with hipcc for gfx950.
* ``easy_as_amd/_hip<EXT_SUFFIX>`` — the CPython binding over that ABI.

Run ``python -m easy_as_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

LIB = PKG / "libeas_hip.so"
EXT = PKG / ("_hip" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

# Packed-FP32 instructions are disabled in every HIP compile of this project.
HIP_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    _run([
        str(ROCM / "bin" / "hipcc"), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-shared",
        *HIP_FLAGS, "-Wall", "-Wno-unused-command-line-argument", f"-I{INCLUDE}",
        str(CSRC / "eas_hip.cpp"), "-o", str(tmp),
        f"-L{ROCM / 'lib'}", "-ldl", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
    ])
    os.replace(tmp, LIB)
    return LIB


def build_ext() -> Path:
    tmp = EXT.with_suffix(".tmp")
    py_inc = sysconfig.get_paths()["include"]
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{py_inc}", f"-I{INCLUDE}",
        str(CSRC / "hip_module.cpp"), "-o", str(tmp), f"-L{PKG}", "-leas_hip", "-Wl,-rpath,$ORIGIN",
    ])
    os.replace(tmp, EXT)
    return EXT


def build() -> None:
    build_lib()
    build_ext()


if __name__ == "__main__":
    build()
    sys.exit(0)
