"""Build the plugin's native libraries for gfx950, in-tree.

    python jax-metallib_amd/build.py            # kernels + plugin
    python jax-metallib_amd/build.py --jobs 8

Outputs (git-ignored, shipped with the tree):
    jax-metallib_amd/lib/libmk_kernels.so   kernel C-ABI (include/mk_kernels.h) and
                                            the plugin runtime (include/mk_runtime.h)

Every HIP translation unit is compiled with hipcc for gfx950 only, with the
packed-FP32 feature disabled (-Xclang -target-feature -Xclang -packed-fp32-ops);
objects go to jax-metallib_amd/lib/obj/ and are linked into one shared library.
"""

import argparse
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(LIB, "obj")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-I", os.path.join(REPO, "include"),
]

# Kernel library sources (order = link order).
KERNEL_SOURCES = [
    "capi.cpp",
    "ew_jit.cpp",
    "kernels/qmatmul.hip",
    "kernels/qgemm.hip",
    "kernels/decoder.hip",
    "kernels/gemm.hip",
    "kernels/dot_general.hip",
    "kernels/rowops.hip",
    "kernels/eltwise.hip",
    "runtime/shlo_parser.cpp",
    "runtime/planner.cpp",
    "runtime/runtime.cpp",
]


def _compile(src):
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src.replace("/", "_") + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC] + COMMON + lang + ["-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    return obj


def _link(objs, target, extra=()):
    tmp = target + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + list(objs) + list(extra)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed for {target}:\n{r.stdout}{r.stderr}")
    os.replace(tmp, target)


def build(jobs=None, verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, KERNEL_SOURCES))
    target = os.path.join(LIB, "libmk_kernels.so")
    _link(objs, target, ["-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"])
    if verbose:
        print(f"built {os.path.relpath(target, REPO)}")
    return target


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    try:
        build(args.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
