"""Build the native parts in-tree (no JIT cache, so the files travel with the source tree):

  lib/libq4hip.so   HIP kernels + C ABI, gfx950      (hipcc)
  lib/q4hip.node    N-API addon over the C ABI       (gcc, against the Node headers)

Usage: python e2e-browser-voice-agent_amd/build.py
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")

# -ffp-contract=off: no multiply-add fusion, so every binary32 operation rounds once as on the CPU.
# Correctly rounded fp32 divide and sqrt (hipcc's default, stated explicitly).
# Packed-FP32 instructions are disabled for all device code.
# -amdgpu-mfma-vgpr-form: matrix-core results in ordinary VGPRs (they feed vector ALU chains at once).
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-fhip-fp32-correctly-rounded-divide-sqrt", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + os.path.join(REPO, "include")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in line)
    if r.returncode:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build_hip() -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libq4hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", tmp, os.path.join(PKG, "csrc", "q4hip.hip")])
    os.replace(tmp, out)
    return out


def build_addon() -> str | None:
    src = os.path.join(PKG, "node", "addon.c")
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return None
    out = os.path.join(LIB, "q4hip.node")
    tmp = out + ".tmp"
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", "-DNAPI_VERSION=8",
          "-I" + NODE_INCLUDE, "-I" + os.path.join(REPO, "include"), "-o", tmp, src,
          "-L" + LIB, "-lq4hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def main() -> None:
    print(build_hip())
    a = build_addon()
    if a:
        print(a)


if __name__ == "__main__":
    sys.exit(main())
