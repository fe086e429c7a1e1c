"""Ahead-of-time build of the MI355X decode library and its PyTorch extension (in-tree).

Produces, next to this file:
  lib/libqwentts_amd.so        C-ABI library (include/qwentts_amd.h): the gfx950 kernels and
                               their extern "C" launchers, built with hipcc.
  _qwentts_amd_C<ext>.so       PyTorch-ROCm extension with the reference's pybind classes
                               (MegakernelTTSDecoder, MegakernelCodePredictorDecoder), built
                               with g++ and linked against the library (rpath $ORIGIN/lib).

Replaces the reference's JIT ``load_inline`` (megakernel_backbone.py:339-353,
megakernel_code_predictor.py:247-260). Run: ``python qwentts-turbo_amd/build.py``.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"
LIB = PKG / "lib" / "libqwentts_amd.so"
EXT_NAME = "_qwentts_amd_C"

# Device-code flags: every HIP translation unit is built with packed-f32 instructions off.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def ext_path() -> Path:
    return PKG / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {cmd[0]}")
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if verbose and err:
        print(err)


def build_library(verbose: bool = False) -> Path:
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    _run([ROCM / "bin" / "hipcc", *HIP_FLAGS, "-shared", f"-I{ROOT / 'include'}", f"-I{PKG / 'csrc'}",
          PKG / "csrc" / "qtts_decode.hip", PKG / "csrc" / "qtts_prefill.hip", PKG / "csrc" / "qtts_shared.hip",
          "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_extension(verbose: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension
    tdir = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROCM / "include"), str(ROOT / "include")]
    out = ext_path()
    tmp = out.with_suffix(".tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{i}" for i in incs], PKG / "csrc" / "bindings.cpp", "-o", tmp,
           f"-L{tdir / 'lib'}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           f"-L{ROCM / 'lib'}", "-lamdhip64", f"-L{LIB.parent}", "-lqwentts_amd",
           "-Wl,-rpath,$ORIGIN/lib", f"-Wl,-rpath,{tdir / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
