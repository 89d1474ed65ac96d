"""CPU oracle for the MI355X PJRT plugin's hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the plugin library, its
Python registration, its kernels) imports, links or calls this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and there only as the checker or as the timed CPU port.

The reference (erfanzar/jax-metallib) compares its GPU results against JAX's
XLA:CPU backend (``benchmarks/vs_cpu.py:682-721``; every regression test runs
``jax.jit(fn, backend="cpu")``, e.g. ``tests/test_native_softmax.py:66-71``).
JAX is not installed in this image, so this package restates, in numpy
(float64 accumulation) and in a small C library (``oracle/c/``), the
arithmetic XLA:CPU performs for each hot-path op, following the reference's
own statements of those semantics, which each function cites.

Parity pins (what keeps each restatement honest) live in
``tests/test_oracle.py``: the reference tests' known answers, closed forms,
brute-force loops on tiny inputs and invariants.  Every function listed in
``PINS`` below has at least one such check; none is "parity unpinned" except
where ``PINS`` says so.

Modules:
  bf16     -- bfloat16 round-to-nearest-even and widening (numpy bit twiddling)
  quant    -- int4 group-64 / int8 per-channel dequant-matmul, the reference's
              affine quantizer, nibble packing
  gemm     -- dot_general with XLA's dtype rules (bf16 -> f32 accumulate)
  rowops   -- softmax, RMSNorm, argmax, sum/max reductions (last axis)
  eltwise  -- the fused elementwise op set with per-op bf16 rounding
  cport    -- ctypes loader for the C restatement (the bench's CPU baseline)
"""

PINS = {
    "bf16.round_bf16": "closed form: exactly-representable values, RNE ties, NaN/inf, overflow",
    "quant.pack_int4_k/unpack_int4_k": "round trip + brute-force loop + literal byte vectors",
    "quant.int4_g64_matmul": "brute-force loop on tiny inputs; all-ones closed form; reference [[64,64]]",
    "quant.int8_pc_matmul": "brute-force loop; identity-weight closed form",
    "quant.affine_quantize/dequantize": "reference test_quantized.py roundtrip/zeros/shape/[[64,64]] known answers",
    "gemm.dot_general": "identity, all-ones (=K), 7e4 overflow case, K=1 signed zero, brute-force loop",
    "rowops.softmax": "reference special rows (NaN, -inf, +inf, constant 80) + sum-to-one invariant",
    "rowops.rmsnorm": "constant-row closed form, brute-force loop",
    "rowops.argmax": "reference special-value matrices (first NaN, first max, -0 == +0) vs brute force",
    "rowops.reduce": "brute force; NaN propagation; -0/+0 max",
    "eltwise.chain6": "op-by-op closed forms (exp(0)=1, log1p(0)=0, select masks) + bf16 rounding points",
    "cport.int4_g64_matmul": "numpy oracle (M > 64, ragged N, several groups, column slices), brute-force "
                             "loop, nibble-order / zero-point closed form",
    "cport.int8_pc_matmul": "numpy oracle, brute-force loop, identity weight with and without scales",
    "cport.gemm_bf16": "numpy oracle (row slices), A @ I == A, ones (= K), K * m * n index matrices",
    "cport.argmax_f32": "brute-force loop on the reference's special-value matrices, known rows",
}
