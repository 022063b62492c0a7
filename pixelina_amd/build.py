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
    "csrc/gemm_kq.hip",
    "csrc/matvec.hip",
    "csrc/fuse.hip",
    "csrc/ops.hip",
    "csrc/attention.hip",
    "csrc/tensor_ops.hip",
    "csrc/conv.hip",
    "csrc/api.cpp",
    "csrc/model_file.cpp",
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


# Kernels whose s_waitcnt vmcnt accounting counts only their own DMAs: a
# register spill would add scratch traffic to that counter and break it, so the
# build fails if the compiler spills any (the integer-sum debug variants drain
# the counter completely and are exempt).  The attention kernels drain it
# completely too, but sit at the register limit, where a spill would mean
# scratch traffic in the key loop; they are checked as well.
NO_SPILL = {
    "csrc/attention.hip": ("attn_kernelILi128E", "attn_kernelILi64E", "attn_wide_kernelILi128E", "attn_wide_kernelILi96E",
                           "attn_wide_kernelILi64E"),
    "csrc/gemm_kq.hip": ("gemm_kq_kernelILb1ELb0E", "gemm_kq_kernelILb0ELb0E"),
    "csrc/gemm.hip": ("gemm_kernelILb0E", "gemm_small_kernel"),
}


def _check_no_spill(src, kernels):
    path = os.path.join(HERE, src)
    out = os.path.join(OBJDIR, os.path.basename(src) + ".s")
    cmd = [_hipcc(), *FLAGS, "--cuda-device-only", "-S", path, "-o", out]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{proc.stderr}")
    name, spills = None, {}
    with open(out) as f:
        for line in f:
            line = line.strip()
            if line.startswith(".name:"):
                name = line.split()[-1]
            elif line.startswith(".vgpr_spill_count:") and name:
                spills[name] = int(line.split()[-1])
    for k in kernels:
        hits = [v for n, v in spills.items() if k in n]
        if not hits:
            raise RuntimeError(f"{src}: kernel {k} not found in the device assembly")
        if max(hits) > 0:
            raise RuntimeError(f"{src}: kernel {k} spills {max(hits)} VGPRs (its vmcnt waits assume no scratch traffic)")


def build(verbose=False):
    os.makedirs(OBJDIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(SOURCES) + len(NO_SPILL), os.cpu_count() or 4)) as pool:
        checks = [pool.submit(_check_no_spill, src, ks) for src, ks in NO_SPILL.items() if src in SOURCES]
        objs = list(pool.map(_compile, SOURCES))
        for c in checks:
            c.result()
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
