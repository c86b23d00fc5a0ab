"""Build libfvs.so (the gfx950 HIP kernels behind include/fvs.h) in-tree with hipcc, and the host-only
row tier reader libfvs_tier.so (include/fvs_tier.h) with the host compiler.

Each .hip translation unit is compiled to an object in parallel, then linked into
fanarvse_paper_amd/libfvs.so. Floating-point contraction is disabled (every fma in the kernels is
written explicitly, so results follow the canonical operation order documented in fvs.h), fp32
division and square root are correctly rounded, and packed-fp32 instructions are not generated.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libfvs.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


TIER_SRC = os.path.join(CSRC, "fvs_tier.cpp")
TIER_LIB = os.path.join(HERE, "libfvs_tier.so")
CXX = os.environ.get("CXX", "g++")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_tier():
    """The host-only row tier reader (include/fvs_tier.h) with the host compiler."""
    tmp = TIER_LIB + ".tmp"
    r = subprocess.run([CXX, "-O2", "-std=c++17", "-Wall", "-fPIC", "-shared", TIER_SRC, "-o", tmp, "-lpthread"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed for {TIER_SRC}:\n{r.stderr}")
    os.replace(tmp, TIER_LIB)
    return TIER_LIB


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=False):
    """Compile every kernel source and link libfvs.so; returns the library path."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    build_tier()
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, and {TIER_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
