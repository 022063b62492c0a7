"""Builds libpixhip.so (HIP kernels for gfx950 + the C ABI + the C++ shim) in
place, next to this file.  hipcc cross-compiles, so this runs without a GPU.

    python -m pixelina_amd.build
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OBJDIR = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libpixhip.so")
SHIM_CHECK = os.path.join(HERE, "shim_check")

SOURCES = [
    "csrc/quantize.hip",
    "csrc/repack.hip",
    "csrc/gemm.hip",
    "csrc/matvec.hip",
    "csrc/fuse.hip",
    "csrc/ops.hip",
    "csrc/api.cpp",
    "host/backend_hip.cpp",
]

ARCH = os.environ.get("PIXHIP_ARCH", "gfx950")

# -ffp-contract=off: every fused multiply-add in the kernels is explicit, so
# the quantizers reproduce the reference's rounding bit for bit.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 are generated.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-I", os.path.join(HERE, "csrc"),
    "-I", os.path.join(HERE, "host"),
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src):
    path = os.path.join(HERE, src)
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *FLAGS, "-c", path, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(OBJDIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    # The shim driver the GPU tests run (host code over the library).
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "host"),
           os.path.join(HERE, "host", "shim_check.cpp"), "-o", SHIM_CHECK + ".tmp", "-L", HERE, "-lpixhip",
           "-Wl,-rpath,$ORIGIN"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"shim_check build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(SHIM_CHECK + ".tmp", SHIM_CHECK)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
