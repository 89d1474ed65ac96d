"""Build the plugin's native libraries for gfx950, in-tree.

    python jax-metallib_amd/build.py            # kernels + plugin
    python jax-metallib_amd/build.py --jobs 8

Outputs (git-ignored, shipped with the tree):
    jax-metallib_amd/lib/libmk_kernels.so   kernel C-ABI (include/mk_kernels.h) and
                                            the plugin runtime (include/mk_runtime.h)
    jax-metallib_amd/lib/libmk_pjrt.so      the PJRT plugin: GetPjrtApi
                                            (include/pjrt_c_api_mi355x.h)

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
    "kernels/layout.hip",
    "runtime/shlo_parser.cpp",
    "runtime/mlir_bytecode.cpp",
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


# The PJRT plugin: the GetPjrtApi table over the runtime C-ABI.  Host C++
# only (no device code), linked against libmk_kernels.so next to it; a
# version script leaves GetPjrtApi as its one exported symbol.
PJRT_SOURCE = os.path.join(CSRC, "pjrt", "pjrt_api.cpp")
PJRT_EXPORTS = os.path.join(CSRC, "pjrt", "exports.map")
CXX = os.environ.get("CXX", "g++")


def _build_pjrt():
    obj = os.path.join(OBJ, "pjrt_pjrt_api.cpp.o")
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
           "-I", os.path.join(REPO, "include"), "-c", PJRT_SOURCE, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed for pjrt_api.cpp:\n{r.stdout}{r.stderr}")
    target = os.path.join(LIB, "libmk_pjrt.so")
    tmp = target + ".tmp"
    cmd = [CXX, "-shared", "-fPIC", "-o", tmp, obj, "-L", LIB, "-lmk_kernels", "-Wl,-rpath,$ORIGIN",
           f"-Wl,--version-script={PJRT_EXPORTS}", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed for libmk_pjrt.so:\n{r.stdout}{r.stderr}")
    os.replace(tmp, target)
    return target


# Sanitizer build of the host code (StableHLO parser, planner, runtime,
# MKEX reader, elementwise JIT cache, C-ABI glue, PJRT adapter): the host
# sources compiled by g++ with AddressSanitizer and UndefinedBehaviorSanitizer,
# linked with the uninstrumented device-code objects into lib/asan/.  The C
# test harness tests/pjrt/pjrt_harness.c is built twice: with the sanitizers
# (it drives lib/asan/ on the CPU) and without (for the GPU box).
SAN_HOST_SOURCES = ["capi.cpp", "ew_jit.cpp", "runtime/shlo_parser.cpp", "runtime/mlir_bytecode.cpp",
                    "runtime/planner.cpp", "runtime/runtime.cpp"]
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]
HARNESS_SOURCE = os.path.join(REPO, "tests", "pjrt", "pjrt_harness.c")


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")


def _build_sanitized(kernel_objs):
    san_dir = os.path.join(LIB, "asan")
    os.makedirs(os.path.join(san_dir, "obj"), exist_ok=True)
    inc = ["-I", os.path.join(REPO, "include"), "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]
    host_objs = []
    for src in SAN_HOST_SOURCES + ["pjrt/pjrt_api.cpp"]:
        obj = os.path.join(san_dir, "obj", src.replace("/", "_") + ".o")
        _run([CXX, "-O1", "-std=c++17", "-fPIC"] + SAN_FLAGS + inc + ["-c", os.path.join(CSRC, src), "-o", obj],
             f"sanitizer compile of {src}")
        host_objs.append(obj)
    device_objs = [o for o in kernel_objs if o.endswith(".hip.o")]
    kern = os.path.join(san_dir, "libmk_kernels.so")
    _run([CXX, "-shared", "-fPIC"] + SAN_FLAGS + ["-o", kern] + host_objs[:-1] + device_objs +
         ["-L/opt/rocm/lib", "-lamdhip64", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"], "sanitizer link of libmk_kernels")
    _run([CXX, "-shared", "-fPIC"] + SAN_FLAGS + ["-o", os.path.join(san_dir, "libmk_pjrt.so"), host_objs[-1],
                                                  "-L", san_dir, "-lmk_kernels", "-Wl,-rpath,$ORIGIN",
                                                  f"-Wl,--version-script={PJRT_EXPORTS}"],
         "sanitizer link of libmk_pjrt")
    test_dir = os.path.join(LIB, "test")
    os.makedirs(test_dir, exist_ok=True)
    cc = os.environ.get("CC", "gcc")
    base = [cc, "-std=c11", "-Wall", "-Wextra", "-O1", "-I", os.path.join(REPO, "include"), HARNESS_SOURCE]
    _run(base[:1] + SAN_FLAGS + base[1:] + ["-o", os.path.join(test_dir, "pjrt_harness_asan"), "-ldl"],
         "sanitizer harness build")
    _run(base + ["-o", os.path.join(test_dir, "pjrt_harness"), "-ldl"], "harness build")


def build(jobs=None, verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, KERNEL_SOURCES))
    target = os.path.join(LIB, "libmk_kernels.so")
    _link(objs, target, ["-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"])
    pjrt = _build_pjrt()
    _build_sanitized(objs)
    if verbose:
        print(f"built {os.path.relpath(target, REPO)}, {os.path.relpath(pjrt, REPO)}")
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
