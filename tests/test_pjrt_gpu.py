"""The PJRT plugin on the GPU, driven only through GetPjrtApi's table by the C
harness tests/pjrt/pjrt_harness.c (dlopen of libmk_pjrt.so, as jaxlib loads
a plugin): Client_Create -> Client_Compile -> BufferFromHostBuffer ->
LoadedExecutable_Execute -> Event_Await -> ToHostBuffer, plus the output
metadata, the device assignment, CopyRawToHost, Serialize /
DeserializeAndLoad and buffer deletion on the way
(src/pjrt_plugin/api/pjrt_client.cc:178-293, pjrt_executable.cc:245-378,
pjrt_buffer.cc:148-234 under /root/reference).  The outputs are checked
against the CPU oracle at the workload's tolerances."""

import os
import subprocess

import numpy as np
import pytest

import _bytecode as B
from _gpu import BF16_RTOL, F32_RTOL, assert_rel_close
from mi355x import programs as P
from oracle import cport, quant
from oracle.bf16 import bf16_bits_to_f32

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "jax-metallib_amd", "lib")
HARNESS = os.path.join(LIB, "test", "pjrt_harness")
PJRT = os.path.join(LIB, "libmk_pjrt.so")

BF16, U8, F32 = 13, 6, 11  # PJRT_Buffer_Type


def _run(args, timeout=240):
    for p in (HARNESS, PJRT):
        if not os.path.exists(p):
            pytest.fail(f"{p} missing: run __graft_entry__.build()")
    print(f"[pjrt] {' '.join(os.path.basename(a) for a in args[:3])}", flush=True)
    r = subprocess.run([HARNESS] + args, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"harness failed ({r.returncode}):\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    return r.stdout


def _spec(tmp_path, name, arr, ptype):
    path = tmp_path / f"{name}.bin"
    path.write_bytes(np.ascontiguousarray(arr).tobytes())
    return f"{ptype}:{'x'.join(str(d) for d in arr.shape)}:{path}"


def test_table_on_the_gpu():
    """The table checks of the CPU test, with Client_Create succeeding and the
    client's devices, memory, memory stats, device assignment and compile
    errors exercised."""
    out = _run(["api", PJRT, "gpu"])
    assert "api ok" in out


def test_int4_headline_through_the_table(tmp_path):
    M, K, N = 16, 4096, 14336
    x, packed, s, z = quant.make_int4_case(np.random.default_rng(0), M, K, N)
    prog = tmp_path / "int4.mlir"
    prog.write_text(P.int4_g64_matmul(M, K, N))
    out = tmp_path / "y.bin"
    _run(["run", PJRT, str(prog), str(out), _spec(tmp_path, "x", x, BF16), _spec(tmp_path, "w", packed, U8),
          _spec(tmp_path, "s", s, BF16), _spec(tmp_path, "z", z, U8)])
    y = np.frombuffer(out.read_bytes(), dtype=np.uint16).reshape(M, N)
    assert_rel_close(bf16_bits_to_f32(y), cport.int4_g64_matmul(x, packed, s, z), BF16_RTOL, "int4 via PJRT")


def test_plumbing_through_the_table(tmp_path):
    """The workload's plumbing program, tanh(A @ B).sum(axis=1) on f32
    [1024, 1024]: f32 in and out, three kernel steps."""
    n = 1024
    rng = np.random.default_rng(0)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    prog = tmp_path / "plumbing.mlir"
    prog.write_text(P.plumbing(n))
    out = tmp_path / "y.bin"
    _run(["run", PJRT, str(prog), str(out), _spec(tmp_path, "a", a, F32), _spec(tmp_path, "b", b, F32)])
    y = np.frombuffer(out.read_bytes(), dtype=np.float32)
    ref = np.tanh(a.astype(np.float64) @ b.astype(np.float64)).sum(axis=1)
    assert_rel_close(y, ref, F32_RTOL, "plumbing via PJRT", elem=False)


def test_softmax_through_the_table(tmp_path):
    x = (np.random.default_rng(3).standard_normal((256, 8192)) * np.sqrt(2)).astype(np.float32)
    prog = tmp_path / "softmax.mlir"
    prog.write_text(P.softmax(256, 8192))
    out = tmp_path / "y.bin"
    _run(["run", PJRT, str(prog), str(out), _spec(tmp_path, "x", x, F32)])
    y = np.frombuffer(out.read_bytes(), dtype=np.float32).reshape(x.shape)
    from oracle import rowops
    assert_rel_close(y, rowops.softmax(x), F32_RTOL, "softmax via PJRT")


def test_int4_headline_from_a_portable_artifact(tmp_path):
    """The form jaxlib sends (MLIR bytecode of the vhlo dialect,
    pjrt_client.cc:178-244) compiled and run through the table."""
    M, K, N = 16, 4096, 14336
    x, packed, s, z = quant.make_int4_case(np.random.default_rng(1), M, K, N)
    prog = tmp_path / "int4.mlirbc"
    prog.write_bytes(B.to_bytecode(P.int4_g64_matmul(M, K, N)))
    out = tmp_path / "y.bin"
    _run(["run", PJRT, str(prog), str(out), _spec(tmp_path, "x", x, BF16), _spec(tmp_path, "w", packed, U8),
          _spec(tmp_path, "s", s, BF16), _spec(tmp_path, "z", z, U8)])
    y = np.frombuffer(out.read_bytes(), dtype=np.uint16).reshape(M, N)
    assert_rel_close(bf16_bits_to_f32(y), cport.int4_g64_matmul(x, packed, s, z), BF16_RTOL, "int4 via bytecode")


def test_argmax_from_a_portable_artifact(tmp_path):
    from oracle import rowops
    x = np.random.default_rng(4).standard_normal((512, 4096)).astype(np.float32)
    x[7, 100] = np.nan
    x[9, :] = -np.inf
    prog = tmp_path / "argmax.mlirbc"
    prog.write_bytes(B.to_bytecode(P.argmax(512, 4096), "vhlo", 6))
    out = tmp_path / "y.bin"
    _run(["run", PJRT, str(prog), str(out), _spec(tmp_path, "x", x, F32)])
    y = np.frombuffer(out.read_bytes(), dtype=np.int32)
    assert np.array_equal(y, rowops.argmax(x))


def test_timing_modes(tmp_path):
    """The harness's two timing modes (bench.py's C-side figures for the
    decode-shaped call) run and report per-call times."""
    import json
    M, K, N = 16, 4096, 14336
    x, packed, s, z = quant.make_int4_case(np.random.default_rng(2), M, K, N)
    prog = tmp_path / "int4.mlir"
    prog.write_text(P.int4_g64_matmul(M, K, N))
    specs = [_spec(tmp_path, "x", x, BF16), _spec(tmp_path, "w", packed, U8), _spec(tmp_path, "s", s, BF16),
             _spec(tmp_path, "z", z, U8)]
    for args in (["time", PJRT, str(prog), "2", "5"] + specs,
                 ["floor", os.path.join(LIB, "libmk_kernels.so"), "/opt/rocm/lib/libamdhip64.so", "2", "5"]):
        rep = json.loads(_run(args).strip().splitlines()[-1])
        assert rep["iters"] == 5 and 0 < rep["min_us"] <= rep["median_us"] <= rep["p90_us"], rep
