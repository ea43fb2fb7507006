"""Build the HIP backend library in-tree: sanic_amd/libsanic_hip.so (gfx950 only)."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = ["runtime.cpp", "emit_hip.cpp", "skeletons.cpp", "skel_attention.cpp", "skel_flash.cpp", "skel_gemm.cpp", "rtc.cpp"]
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "--offload-arch=gfx950",
         # packed-f32 instruction forms stay disabled for device code
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-result"]


def build(verbose: bool = False) -> str:
    out = os.path.join(HERE, "libsanic_hip.so")
    csrc = os.path.join(HERE, "csrc")
    cmd = ["/opt/rocm/bin/hipcc", *FLAGS, *[os.path.join(csrc, s) for s in SOURCES],
           "-I", os.path.join(HERE, "..", "include"), "-lhiprtc", "-ldl", "-lpthread",
           "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libsanic_hip.so")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
