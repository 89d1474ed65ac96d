"""The PJRT plugin library (libmk_pjrt.so) on the CPU, with no GPU.

* It exports exactly one symbol, GetPjrtApi (the reference's plugin does the
  same, src/pjrt_plugin/api/pjrt_api.cc:324-329).
* The C harness tests/pjrt/pjrt_harness.c, built with AddressSanitizer and
  UndefinedBehaviorSanitizer against the sanitizer build of the host code
  (lib/asan/), drives the table the way the reference's own table tests do
  (tests/test_pjrt_required_callbacks.py:118-160, test_pjrt_handle_abi.py:15-25
  under /root/reference): table shape and version, the 107 entries the
  reference sets, error objects and their function table, events (pending,
  OnReady, Set with an error, Await), the topology, argument-struct checks,
  and Client_Create failing with UNAVAILABLE when no device is visible.
* The same harness runs the StableHLO parser and planner (mkrt_compile_check)
  on every program the workload compiles, as text and as MLIR bytecode, and
  on every truncation and a set of byte flips of each, and the serialized-executable reader
  (mkrt_serialized_inspect) on every truncation and header byte flip, all
  under the sanitizers: any out-of-bounds access, leak or undefined behaviour
  aborts the harness.
"""

import os
import shutil
import subprocess

import pytest

from mi355x import programs as P

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "jax-metallib_amd", "lib")
HARNESS_ASAN = os.path.join(LIB, "test", "pjrt_harness_asan")
ASAN_PJRT = os.path.join(LIB, "asan", "libmk_pjrt.so")
ASAN_KERNELS = os.path.join(LIB, "asan", "libmk_kernels.so")


def _need(path):
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: run __graft_entry__.build()")


def _gpu_visible():
    # Device nodes only: the harness decides on its own what Client_Create
    # must return, and initialising HIP here is not needed.
    return os.path.exists("/dev/kfd") and any(n.startswith("renderD") for n in os.listdir("/dev/dri"))\
        if os.path.isdir("/dev/dri") else False


def _harness(args, timeout=600):
    env = dict(os.environ)
    env.setdefault("ASAN_OPTIONS", "detect_leaks=1:abort_on_error=0:halt_on_error=1")
    env.setdefault("UBSAN_OPTIONS", "print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([HARNESS_ASAN] + args, capture_output=True, text=True, timeout=timeout, env=env)
    assert r.returncode == 0, f"harness {args[0]} failed ({r.returncode}):\n{r.stdout[-4000:]}\n{r.stderr[-8000:]}"
    return r.stdout


def test_exactly_one_exported_symbol():
    lib = os.path.join(LIB, "libmk_pjrt.so")
    _need(lib)
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("binutils nm not installed")
    out = subprocess.run([nm, "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    syms = [l.split()[-1] for l in out.splitlines() if l.strip()]
    assert syms == ["GetPjrtApi"], syms


def test_table_errors_events_topology_under_sanitizers():
    _need(HARNESS_ASAN)
    _need(ASAN_PJRT)
    out = _harness(["api", ASAN_PJRT, "gpu" if _gpu_visible() else "nogpu"])
    assert "api ok" in out


def _corpus():
    """Every StableHLO program form the workload and the tests compile."""
    progs = {
        "int4": P.int4_g64_matmul(16, 4096, 14336), "int4_m256": P.int4_g64_matmul(256, 1024, 512),
        "int8": P.int8_pc_matmul(16, 4096, 14336), "gemm_bf16": P.matmul(512, 512, 512),
        "gemm_pref": P.matmul(200, 64, 136, preferred_f32=True), "bmm": P.matmul(128, 64, 256, batch=4),
        "gemm_f32": P.matmul(256, 320, 264, dt="f32"), "softmax": P.softmax(64, 512),
        "softmax_bf16": P.softmax(64, 512, "bf16"), "rmsnorm": P.rmsnorm(64, 512),
        "rmsnorm_bf16": P.rmsnorm(64, 512, "bf16"), "argmax": P.argmax(64, 512),
        "argmax_bf16": P.argmax(64, 512, "bf16"), "sum": P.reduce(64, 512), "max": P.reduce(64, 512, "max"),
        "trailing": P.reduce_trailing((4, 8, 16), 2, "sum"), "chain6": P.chain6(64, 512),
        "chain6_bf16": P.chain6(64, 512, "bf16"), "plumbing": P.plumbing(256),
        "dot_int": P.dot_general((8, 16), (16, 4), "int32"),
        "dot_self_t": P.dot_general((8, 16), None, "float32", self_transpose=True),
    }
    return progs


def test_parser_and_planner_under_sanitizers(tmp_path):
    _need(HARNESS_ASAN)
    _need(ASAN_KERNELS)
    files = []
    for name, text in _corpus().items():
        p = tmp_path / f"{name}.mlir"
        p.write_text(text)
        files.append(str(p))
    out = _harness(["parse", ASAN_KERNELS] + files, timeout=1200)
    assert "parse ok" in out


def test_bytecode_reader_under_sanitizers(tmp_path):
    """The MLIR-bytecode front end on portable artifacts of the corpus (and
    builtin-dialect modules at other bytecode versions): every truncation and
    a spread of byte flips."""
    import _bytecode as B
    _need(HARNESS_ASAN)
    _need(ASAN_KERNELS)
    files = []
    for i, (name, text) in enumerate(sorted(_corpus().items())):
        flavor, version = ("vhlo", 1) if i % 2 == 0 else ("builtin", 2 + i % 5)
        p = tmp_path / f"{name}.mlirbc"
        p.write_bytes(B.to_bytecode(text, flavor, version))
        files.append(str(p))
    out = _harness(["parse", ASAN_KERNELS] + files, timeout=1200)
    assert "parse ok" in out


def test_serialized_executable_reader_under_sanitizers(tmp_path):
    _need(HARNESS_ASAN)
    _need(ASAN_KERNELS)
    from mi355x import runtime as rt
    files = []
    for name in ("chain6_bf16", "softmax", "gemm_bf16"):
        p = tmp_path / f"{name}.mkex"
        p.write_bytes(rt.serialize_program(_corpus()[name]))
        files.append(str(p))
    out = _harness(["inspect", ASAN_KERNELS] + files)
    assert "inspect ok" in out
