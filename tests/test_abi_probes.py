"""CPU probes of the drop-in boundary, built here with gcc/g++ against a fake
HIP runtime (tests/probes/fake_hip.cpp; the library's CPU test build,
-DLUNAFLUX_HIP_FAKE, routes every HIP call through it):

* abi_probe: the C ABI (include/lunaflux_hip.h) - lifecycle interlocks and
  retryable closes, region and lease checks, transfers, the launch path
  (operands held during the launch, LF_BUSY on close, base + offset
  parameters, limits, injected failures), the symbol grammar, the
  asynchronous launch's deferred release - as the reference's fake-driver
  probes check internal/cuda (launch_probe.c, region_probe.c,
  lifecycle_probe.c, allocation_lease_probe.c, transfer_probe.c);
* moonbit_probe: the MoonBit stub layer
  (lunaflux_amd/csrc/moonbit/lunaflux_hip_moonbit.c), every extern of
  internal/cuda/ffi.mbt:29-240, built against a stand-in moonbit.h
  (tests/probes/moonbit.h) since the MoonBit toolchain is absent.

Each is also built with AddressSanitizer and UndefinedBehaviorSanitizer
(host code only; no GPU is involved).
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBES = os.path.join(ROOT, "tests", "probes")
CSRC = os.path.join(ROOT, "lunaflux_amd", "csrc")
INCLUDE = os.path.join(ROOT, "include")
HIP_INCLUDE = "/opt/rocm/include"

pytestmark = pytest.mark.skipif(
    shutil.which("gcc") is None or shutil.which("g++") is None
    or not os.path.exists(os.path.join(HIP_INCLUDE, "hip", "hip_runtime_api.h")),
    reason="needs gcc, g++ and the HIP headers")


def build(out_dir, name, c_sources, flags):
    cxx = ["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror", *flags,
           "-D__HIP_PLATFORM_AMD__", "-DLUNAFLUX_HIP_FAKE", "-I", HIP_INCLUDE, "-I", INCLUDE,
           "-I", CSRC, "-I", PROBES]
    cc = ["gcc", "-std=c11", "-O1", "-g", "-Wall", "-Wextra", "-Werror", *flags, "-I", INCLUDE,
          "-I", PROBES]
    objects = []
    for src in [os.path.join(CSRC, "runtime.cpp"), os.path.join(PROBES, "fake_hip.cpp")]:
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        subprocess.run(cxx + ["-c", src, "-o", obj], check=True)
        objects.append(obj)
    for src in c_sources:
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        subprocess.run(cc + ["-c", src, "-o", obj], check=True)
        objects.append(obj)
    exe = os.path.join(out_dir, name)
    subprocess.run(["g++", *flags, *objects, "-o", exe], check=True)
    return exe


PROGRAMS = {
    "abi_probe": [os.path.join(PROBES, "abi_probe.c")],
    "moonbit_probe": [os.path.join(CSRC, "moonbit", "lunaflux_hip_moonbit.c"),
                      os.path.join(PROBES, "moonbit_shim.c"),
                      os.path.join(PROBES, "moonbit_probe.c")],
}


@pytest.mark.parametrize("sanitize", [False, True], ids=["plain", "asan-ubsan"])
@pytest.mark.parametrize("program", sorted(PROGRAMS))
def test_probe(tmp_path, program, sanitize):
    flags = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer",
             "-fno-sanitize-recover=undefined"] if sanitize else []
    exe = build(str(tmp_path), program, PROGRAMS[program], flags)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1")
    run = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    print(run.stdout)
    print(run.stderr)
    assert run.returncode == 0, run.stderr
    assert run.stdout.strip().splitlines()[-1] == "ok all"
