"""Builds liblifscan_hip.so (the C-ABI HIP library) in-tree with hipcc for gfx950.

The library is compiled from ``csrc/*.hip`` next to this package and written to
``lifscan/_lib/liblifscan_hip.so``.  Flags that fix the numerics:
  -ffp-contract=off                        no FMA contraction (two-rounding LIF step)
  -fno-gpu-flush-denormals-to-zero         IEEE fp32 denormals
  -fhip-fp32-correctly-rounded-divide-sqrt IEEE division for map breakpoints
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 instructions
"""
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)  # hard-resets-compose_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "liblifscan_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: cannot build the HIP extension")


def build_library(verbose=False, extra_flags=()):
    """Compile every csrc/*.hip into lifscan/_lib/liblifscan_hip.so (always recompiles)."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, *extra_flags, "-I", os.path.join(REPO, "include"), *sources(),
           "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        raise RuntimeError(f"hipcc failed (exit {res.returncode})")
    if verbose and res.stdout.strip():
        # host pass warns about the gfx-only target feature; show anything else
        lines = [l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l]
        if lines:
            print("\n".join(lines))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
