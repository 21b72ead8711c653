"""Build libcpv.so (HIP for gfx950) in-tree with hipcc.

Flags that are part of the numeric contract:
  -ffp-contract=off                          no implicit a*b+c fusion
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE division and square root
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no packed fp32 instructions
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libcpv.so")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=False):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    tmp = OUT + ".tmp"
    cmd = [hipcc] + HIP_FLAGS + ["-I", os.path.join(HERE, "..", "include"), "-o", tmp] + sources()
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(OUT)
