"""The benchmark's input generator (mi355x.synthetic, product side) draws the
same values as the tests' generator in oracle.quant, so bench.py times the
inputs the parity tests check; bench.py's timed legs do not import the
oracle."""

import numpy as np

from mi355x import synthetic
from oracle import quant
from oracle.bf16 import f32_to_bf16_bits


def test_int4_case_matches_the_test_generator():
    for (M, K, N) in [(1, 64, 8), (16, 256, 512), (3, 128, 40)]:
        a = synthetic.int4_case(np.random.default_rng(5), M, K, N)
        b = quant.make_int4_case(np.random.default_rng(5), M, K, N)
        for u, v in zip(a, b):
            assert u.dtype == v.dtype and u.shape == v.shape
            assert np.array_equal(u, v)


def test_int8_case_matches_the_test_generator():
    a = synthetic.int8_case(np.random.default_rng(9), 16, 256, 96)
    b = quant.make_int8_case(np.random.default_rng(9), 16, 256, 96)
    for u, v in zip(a, b):
        assert u.dtype == v.dtype and np.array_equal(u, v)


def test_bf16_rounding_is_nearest_even():
    # Ties at the bf16 half-ulp go to the even mantissa; others round to nearest.
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20,
                     -2.5, 3.0e38, 1e-40, -0.0], dtype=np.float32)
    got = synthetic.bf16_bits(vals)
    assert list(got[:4]) == [0x3F80, 0x3F80, 0x3F82, 0x3F81]
    assert np.array_equal(got, f32_to_bf16_bits(vals))


def test_bench_timed_legs_do_not_import_the_oracle():
    import ast
    import os
    src = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")).read()
    tree = ast.parse(src)
    for fn in tree.body:
        if not isinstance(fn, ast.FunctionDef) or fn.name.startswith("cpu_baseline"):
            continue
        for node in ast.walk(fn):
            if isinstance(node, ast.ImportFrom) and node.module and node.module.startswith("oracle"):
                raise AssertionError(f"bench.py:{fn.name} imports {node.module}")
            if isinstance(node, ast.Import):
                for n in node.names:
                    assert not n.name.startswith("oracle"), f"bench.py:{fn.name} imports {n.name}"
