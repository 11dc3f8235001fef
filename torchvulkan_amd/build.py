"""Build recipe for the gfx950 dense-contraction library.

Compiles every HIP source of the C ABI (``csrc/*.hip``) for gfx950 with hipcc
and links them into ``torchvulkan_amd/libtvk_hip.so``, in-tree, so the built
library travels with the source tree. The PrivateUse1 backend extension
(``csrc/backend/*.cpp``) is built by :func:`build_backend` against the
installed torch headers and links to the same library.

Run ``python torchvulkan_amd/build.py`` (or ``__graft_entry__.build()``); the
package itself cannot be imported before its extension exists.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtvk_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 instructions are disabled for every device pass; the host pass
# warns that it does not know the feature, which is harmless. float32 division
# and square root are the correctly rounded ones (hipcc's default, stated so
# that no later flag can change it silently).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


# MFMA results in VGPRs for these files: the attention kernels' softmax and
# rescale steps work on the accumulators with ordinary VALU instructions, and
# in the AGPR form hipcc rotates the GEMM and convolution kernels'
# accumulators through AGPR copies inside their k loops (the 256x256 ring
# GEMM, gemm_dma.hip, and gemm.hip allocate cleanly in the default form). The
# MFMA calibration loop rotates its sixteen accumulators through 88 AGPR
# copies a trip in the AGPR form and issues only MFMAs in the VGPR form.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {
    "attention.hip": VGPR_FORM,
    "calibrate.hip": VGPR_FORM,
    "gemm_dma128.hip": VGPR_FORM,
    "gemm_skinny.hip": VGPR_FORM,
    "conv.hip": VGPR_FORM,
    "conv_nhwc.hip": VGPR_FORM,
    "conv_stem.hip": VGPR_FORM,
}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
    return obj


def build_library(jobs: int | None = None) -> Path:
    """Compile csrc/*.hip for gfx950 and link libtvk_hip.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) - 1), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


BACKEND_SRC = CSRC / "backend"
BACKEND = PKG / "_C.so"


def _torch_flags() -> tuple[list[str], list[str]]:
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = [
        "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-variable", "-Wno-unused-function",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_C",
        *[f"-I{p}" for p in ce.include_paths()], f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
    ]
    libdir = ce.library_paths()[0]
    ldflags = [
        f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-L{PKG}", "-ltvk_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}",
    ]
    return cflags, ldflags


def build_backend(jobs: int | None = None) -> Path:
    """Compile the PrivateUse1 backend (csrc/backend/*.cpp) with g++ into torchvulkan_amd/_C.so."""
    if not LIB.exists():
        raise RuntimeError("build libtvk_hip.so first")
    BUILD.mkdir(exist_ok=True)
    cflags, ldflags = _torch_flags()
    sources = sorted(BACKEND_SRC.glob("*.cpp"))
    cxx = os.environ.get("CXX", "g++")

    def comp(src: Path) -> Path:
        obj = BUILD / ("backend_" + src.stem + ".o")
        _run([cxx, *cflags, "-c", str(src), "-o", str(obj)])
        return obj

    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) - 1), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(comp, sources))
    tmp = BACKEND.with_suffix(".so.tmp")
    _run([cxx, "-shared", *map(str, objs), "-o", str(tmp), *ldflags])
    os.replace(tmp, BACKEND)
    return BACKEND


def main() -> None:
    lib = build_library()
    print(f"built {lib}")
    ext = build_backend()
    print(f"built {ext}")


if __name__ == "__main__":
    main()
