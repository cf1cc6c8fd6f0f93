"""Build the gfx950 backend in-tree.

    python -m sabrewing_amd.build        # or __graft_entry__.build()

Produces
    sabrewing_amd/libsabrewing_hip.so      HIP kernels + C ABI (include/sabrewing_hip.h)
    sabrewing_amd/libsabrewing_loader.so   lag_cuda_* seam (include/sabrewing_loader.h)

Every HIP translation unit is compiled for gfx950 only, with fused
multiply-add contraction off (the kernels write every fma they mean), IEEE
f32 division/sqrt, and packed-fp32 instructions disabled.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
HIP_SOURCES = ["backend_hip.hip", "k_dot8.hip", "k_mfma.hip", "k_idot.hip", "k_shared.hip", "k_route.hip", "coli_hip.hip",
               "k_gen.hip", "k_glue.hip", "k_lanes.hip"]
HIP_LIB = os.path.join(HERE, "libsabrewing_hip.so")
LOADER_LIB = os.path.join(HERE, "libsabrewing_loader.so")
ARCH = "gfx950"


def hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 backend)")


HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{out}")
    return out


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    cc = hipcc()
    objs = []

    def one(src):
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        out = _run([cc, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose and out.strip():
            print(out)
        return obj

    with ThreadPoolExecutor(max_workers=min(4, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(one, HIP_SOURCES))
    tmp = HIP_LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, HIP_LIB)
    tmp = LOADER_LIB + ".tmp"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
          os.path.join(CSRC, "loader.c"), "-o", tmp, "-ldl"])
    os.replace(tmp, LOADER_LIB)
    return HIP_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
