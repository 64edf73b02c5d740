"""Build the two native artefacts of cufk_amd in place.

* ``libcufk_hip.so``: the HIP kernels and the C ABI (``include/cufk_hip.h``), compiled by
  ``hipcc --offload-arch=gfx950``.
* ``_C.<abi>.so``: the PyTorch-ROCm extension (autograd wrappers + validation), plain C++
  compiled by ``g++`` against torch and linked to ``libcufk_hip.so`` through ``$ORIGIN``.

Run ``python cufk_amd/_build.py`` (or ``__graft_entry__.build()``); it imports nothing from
the package, whose ``__init__`` needs the extension this builds.  Every call recompiles.
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
ARCH = os.environ.get("CUFK_OFFLOAD_ARCH", "gfx950")

HIP_LIB = PKG / "libcufk_hip.so"
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
EXT_LIB = PKG / f"_C{EXT_SUFFIX}"

# Every HIP translation unit is built with packed FP32 disabled: the compiler must not emit
# v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")


def build_hip() -> Path:
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run(
        [str(ROCM / "bin" / "hipcc"), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}", str(CSRC / "cufk_hip.hip"), "-o", str(tmp)]
    )
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_extension() -> Path:
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(cpp_extension.library_paths()[0])
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROCM / "include"), str(INCLUDE)]
    tmp = EXT_LIB.with_suffix(".tmp")
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-w",
        *[f"-I{p}" for p in includes],
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        str(CSRC / "binding.cpp"),
        "-o",
        str(tmp),
        f"-L{PKG}",
        "-lcufk_hip",
        f"-L{torch_lib}",
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        f"-L{ROCM / 'lib'}",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, EXT_LIB)
    return EXT_LIB


def build() -> None:
    build_hip()
    build_extension()


if __name__ == "__main__":
    build()
    print(HIP_LIB)
    print(EXT_LIB)
