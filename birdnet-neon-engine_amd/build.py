"""Builds libbnneon_hip.so (hipcc, gfx950) in place, next to this file.

    python birdnet-neon-engine_amd/build.py

Every HIP source is compiled with -ffp-contract=off (no implicit fused
multiply-adds: the int8 epilogues must round exactly as the reference's
-ffp-contract=off build does), fp32 denormals kept, and packed-fp32 code
generation disabled.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbnneon_hip.so")

SOURCES = [
    "device.hip",
    "kern_s8n.hip",
    "pw_s8_static.hip",
    "kern_proto.hip",
    "kern_fproto.hip",
    "kern_dw.hip",
    "kern_wino.hip",
    "kern_f16.hip",
    "kern_gemm_f32.hip",
    "kern_dot.hip",
    "kern_qdot.hip",
    "kern_fe.hip",
    "kern_f32.hip",
    "pkg_file.cpp",
    "rt_contract.cpp",
    "rt_pkg.cpp",
    "ops_table.cpp",
    "ops_s8n.cpp",
    "ops_proto.cpp",
    "ops_f32.cpp",
    "ops_f16.cpp",
    "ops_dot.cpp",
    "bnneon.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++20",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _compile(src):
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, src + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [HIPCC] + FLAGS + lang + ["-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    return obj


def build(verbose=False):
    """Compiles every source that exists and links libbnneon_hip.so."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + \
        objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
