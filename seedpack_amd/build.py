"""Builds libseedpack_amd.so (HIP, gfx950) in-tree from seedpack_amd/csrc/*.hip, plus the host-only
C++ sources seedpack_amd/csrc/*.cpp (built with the host compiler).

Every translation unit is compiled with IEEE float semantics: no FMA contraction, no fast-math,
correctly rounded division and square root, f32 denormals kept, and packed-FP32 instruction
selection disabled. These are the bit-exactness requirements of the quantizers
(seedpack/gpuquant.py:300 and seedpack/ggml/build.sh:7 in the reference).

    python -m seedpack_amd.build [-j N]
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "libseedpack_amd.so")
ARCH = os.environ.get("SPA_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


HOSTCXX = os.environ.get("CXX") or shutil.which("g++") or "c++"
HOST_CFLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall"]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src):
    stem, ext = os.path.splitext(src)
    obj = os.path.join(OBJ, stem + (".o" if ext == ".hip" else "_host.o"))
    if ext == ".hip":
        cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [HOSTCXX, *HOST_CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{os.path.basename(cmd[0])} failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    noise = [ln for ln in r.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln
             and "is not a recognized feature" not in ln]
    return obj, "\n".join(noise)


def build(jobs=None, verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, noise in results:
        if noise and verbose:
            print(f"[build] {os.path.basename(obj)}:\n{noise}", file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] {LIB} ({len(srcs)} sources)")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    build(ap.parse_args().j)
