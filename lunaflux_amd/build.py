"""Builds the native artefacts of lunaflux_amd in-tree:

  lunaflux_amd/liblunaflux_hip.so   C-ABI (include/lunaflux_hip.h and
                                    include/lunaflux_fp8.h): host code, plus
                                    the scratch array of the no-allocation
                                    launch (csrc/scratch.hip)
  lunaflux_amd/lunaflux_fp8.hsaco   gfx950 code object with every kernel
  lunaflux_amd/lunaflux_fp8.manifest.json
                                    its v1 artifact manifest (SHA-256, device
                                    target, entry points; lunaflux_amd/manifest.py)

Run ``python -m lunaflux_amd.build``. hipcc cross-compiles for gfx950, so no
GPU is needed.
"""
from __future__ import annotations

import os
import subprocess
import sys

PACKAGE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PACKAGE)
CSRC = os.path.join(PACKAGE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

LIBRARY = os.path.join(PACKAGE, "liblunaflux_hip.so")
CODE_OBJECT = os.path.join(PACKAGE, "lunaflux_fp8.hsaco")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code: hipcc would
# otherwise form them from ordinary float code.
DEVICE_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Werror"]


def _run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_code_object(out=CODE_OBJECT):
    src = os.path.join(CSRC, "kernels", "lunaflux_fp8.hip")
    tmp = out + ".tmp"
    _run([HIPCC, "--genco", *DEVICE_FLAGS, "-I", INCLUDE, src, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_library(out=LIBRARY):
    """Host code (runtime.cpp, pack.cpp) plus scratch.hip, the one source with
    device code of its own: the scratch array and its clearing kernel, built
    for gfx950 into the library's embedded code object."""
    sources = [os.path.join(CSRC, "runtime.cpp"), os.path.join(CSRC, "pack.cpp"),
               os.path.join(CSRC, "scratch.hip")]
    tmp = out + ".tmp"
    _run([HIPCC, *HOST_FLAGS, f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-shared", "-I", INCLUDE, "-I", CSRC, *sources, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_all():
    build_library()
    build_code_object()
    from lunaflux_amd import manifest
    print(manifest.write_manifest(), flush=True)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
