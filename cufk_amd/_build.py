"""Build the two native artefacts of cufk_amd in place.

* ``libcufk_hip.so``: the HIP kernels and the C ABI (``include/cufk_hip.h``), compiled by
  ``hipcc --offload-arch=gfx950`` as independent units (the ABI, and ``launchers.hip`` once
  per dtype and kernel family) in parallel, then linked.
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
import tempfile
from concurrent.futures import ThreadPoolExecutor
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
# v_pk_{add,mul,fma}_f32.  A pointer passed where a more strictly aligned type is expected is
# an error: rows sit at any element offset, so only the element-aligned vector types may touch
# them.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Werror=align-mismatch",
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


# launchers.hip is compiled once per (dtype, kernel family); the codes match cufk_dtype
# (include/cufk_hip.h) and the CUFK_FAMILY_* values in launchers.hip.
DTYPES = (0, 1, 2, 3)
FAMILIES = (0, 1, 2, 3, 4, 5, 6)


def _jobs() -> int:
    return max(1, min(16, int(os.environ.get("MAX_JOBS", "0")) or (os.cpu_count() or 1)))


def _compile_hip(src: Path, obj: Path, defines: tuple[str, ...] = ()) -> Path:
    _run([str(ROCM / "bin" / "hipcc"), *HIP_FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)])
    return obj


def _hip_objects(pool: ThreadPoolExecutor, tmp: Path) -> list:
    futures = [pool.submit(_compile_hip, CSRC / "cufk_hip.hip", tmp / "cufk_hip.o")]
    for fam in FAMILIES:
        for dt in DTYPES:
            obj = tmp / f"launchers_f{fam}_d{dt}.o"
            futures.append(pool.submit(_compile_hip, CSRC / "launchers.hip", obj, (f"-DCUFK_FAMILY={fam}", f"-DCUFK_DTYPE={dt}")))
    return futures


def _link_hip(objects: list[Path]) -> Path:
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([str(ROCM / "bin" / "hipcc"), f"--offload-arch={ARCH}", "-shared", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def _extension_flags() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(cpp_extension.library_paths()[0])
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROCM / "include"), str(INCLUDE)]
    compile_flags = [
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-w",
        *[f"-I{p}" for p in includes],
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
    ]
    link_flags = [
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
    return compile_flags, link_flags


def _compile_extension(obj: Path, compile_flags: list[str]) -> Path:
    _run(["g++", *compile_flags, "-c", str(CSRC / "binding.cpp"), "-o", str(obj)])
    return obj


def _link_extension(obj: Path, link_flags: list[str]) -> Path:
    tmp = EXT_LIB.with_suffix(".tmp")
    _run(["g++", "-shared", str(obj), "-o", str(tmp), *link_flags])
    os.replace(tmp, EXT_LIB)
    return EXT_LIB


def build() -> None:
    """Compile every unit in parallel (MAX_JOBS, else the CPU count, at most 16 jobs), then link
    libcufk_hip.so and the extension against it."""
    compile_flags, link_flags = _extension_flags()
    with tempfile.TemporaryDirectory(prefix="cufk_amd_build_") as d, ThreadPoolExecutor(_jobs()) as pool:
        tmp = Path(d)
        ext = pool.submit(_compile_extension, tmp / "binding.o", compile_flags)
        hip = _hip_objects(pool, tmp)
        _link_hip([f.result() for f in hip])
        _link_extension(ext.result(), link_flags)


if __name__ == "__main__":
    build()
    print(HIP_LIB)
    print(EXT_LIB)
