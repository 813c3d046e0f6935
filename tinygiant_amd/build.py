"""Builds libtinygiant.so (gfx950) in-tree with hipcc.

Every HIP source is compiled with -ffp-contract=off and correctly rounded
fp32 division/square root (the kernels round exactly as the host definition
of each step), and with the packed-FP32 feature disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtinygiant.so"
SOURCES = ["tg_kernels.hip", "tg_moe.hip", "tg_mfma.hip", "tg_legacy.hip", "tg_sample.hip", "tg_abi.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("TG_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    out = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{out}")
    if out.strip() and verbose:
        print(out)


# Per-source extra flags.  tg_mfma.hip: MFMA results in ordinary VGPRs, so the
# fp32 epilogue reads them without a v_accvgpr_read per element.  Every source:
# the leading scalar and pointer kernel arguments arrive preloaded in SGPRs, so
# a kernel's first loads need no round trip to the argument buffer (the code
# object keeps the argument loads for firmware without the feature).
EXTRA_FLAGS = {"tg_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16"],
               "tg_moe.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
               "tg_kernels.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
               "tg_legacy.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
               "tg_sample.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link libtinygiant.so."""
    BUILD.mkdir(exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", CSRC / src, "-o", obj], verbose)
        objs.append(obj)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


SAN = PKG / "_san"


def build_sanitized(verbose: bool = False) -> Path:
    """The library with AddressSanitizer and UndefinedBehaviorSanitizer on
    its host code only (the gfx950 code is built as usual, without them),
    into _san/.  For tests/test_sanitizers.py, which preloads clang's shared
    ASan runtime.  Rebuilt only when a source is newer than the library."""
    SAN.mkdir(exist_ok=True)
    lib = SAN / "libtinygiant.so"
    deps = [CSRC / f for f in SOURCES] + list(CSRC.glob("*.h")) + [ROOT / "include" / "tinygiant.h", Path(__file__)]
    if lib.exists() and lib.stat().st_mtime > max(d.stat().st_mtime for d in deps):
        return lib
    host = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-g", "-Xarch_host", "-shared-libsan"]
    objs = []
    for src in SOURCES:
        obj = SAN / (Path(src).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), *host, "-c", CSRC / src, "-o", obj], verbose)
        objs.append(obj)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *host, *objs, "-o", lib], verbose)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
