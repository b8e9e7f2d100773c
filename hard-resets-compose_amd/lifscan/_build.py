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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        raise RuntimeError(f"hipcc failed (exit {res.returncode}): {' '.join(cmd[-3:])}")
    if verbose and res.stdout.strip():
        # host pass warns about the gfx-only target feature; show anything else
        lines = [l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l]
        if lines:
            print("\n".join(lines))


def _stale(obj, src):
    """True when obj is missing or older than its source or any csrc header."""
    if not os.path.exists(obj):
        return True
    deps = [src] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    deps.append(os.path.join(REPO, "include", "lifscan_hip.h"))
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def build_library(verbose=False, extra_flags=(), out=None, jobs=None, incremental=False):
    """Compile every csrc/*.hip (one hipcc per source, in parallel) and link them into
    lifscan/_lib/liblifscan_hip.so, or into `out`.  Recompiles everything unless
    `incremental`, which skips sources whose object is newer than them and every header."""
    from concurrent.futures import ThreadPoolExecutor
    out = out or LIB_PATH
    obj_dir = os.path.join(os.path.dirname(out), "_obj")
    os.makedirs(obj_dir, exist_ok=True)
    flags = [f for f in HIP_FLAGS if f != "-shared"] + list(extra_flags)
    inc = ["-I", os.path.join(REPO, "include")]
    objs = []
    cmds = []
    for src in sources():
        obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        if incremental and not extra_flags and not _stale(obj, src):
            continue
        cmds.append([hipcc(), *flags, *inc, "-c", src, "-o", obj])
    if cmds:
        jobs = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
        with ThreadPoolExecutor(jobs) as ex:
            list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = out + ".tmp"
    _run([hipcc(), *HIP_FLAGS, *extra_flags, *objs, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


OPS_NAME = "lifscan_ops"
OPS_DIR = os.path.join(LIB_DIR, "_ops")
OPS_PATH = os.path.join(OPS_DIR, OPS_NAME + ".so")


def build_ops(verbose=False):
    """Compile lifscan/_ops.cpp (the C++ autograd function of lif_tuned's recomputing pair) into
    the in-tree lifscan/_lib/_ops/lifscan_ops.so with torch's extension builder (host compiler,
    torch and HIP headers; it calls the HIP library through addresses handed over at load)."""
    import torch  # noqa: F401  (the builder needs torch's headers and libraries)
    from torch.utils import cpp_extension
    os.makedirs(OPS_DIR, exist_ok=True)
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    cpp_extension.load(
        name=OPS_NAME, sources=[os.path.join(PKG_DIR, "_ops.cpp")], build_directory=OPS_DIR,
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"],
        extra_include_paths=["/opt/rocm/include"],
        extra_ldflags=[f"-L{torch_lib}", "-lc10_hip", f"-Wl,-rpath,{torch_lib}"],
        with_cuda=False, is_python_module=True, verbose=verbose)
    return OPS_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv, incremental="-i" in sys.argv))
