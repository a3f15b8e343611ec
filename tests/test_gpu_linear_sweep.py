"""Seeded sweep of ABI v1 linear shapes through the C-ABI, against the oracle.

Each case draws a weight type (F32, F16, BF16) and a shape from its own seed:
rows 1..16 (the weight-streaming plans, with and without a K split), 17..63,
or 64..160 (bf16 weights with K a multiple of 64 take the tiled product);
columns and outputs either multiples of the 16 x 32 weight tiles or not.
Random inputs are held to the reordered-f32-sum bound of the other linear
tests, |d| <= 1e-5 * sum_c |input * weight| + 1e-4 * |ref|, and
integer-valued inputs (every partial sum exact in f32) must match the oracle
(native/cpu/safetyraise_cpu.c:203-239) bit for bit.
"""
import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_linear import BF16, F16, F32, weight_bits, widened

pytestmark = pytest.mark.gpu

SWEEP = 32


def draw(case_id):
    rng = np.random.default_rng(0x11AE0000 + case_id)
    dtype = int(rng.choice([F32, F16, BF16, BF16]))
    rows = int(rng.choice([rng.integers(1, 17), rng.integers(17, 64), rng.integers(64, 161)]))
    aligned = rng.random() < 0.5
    cols = int(64 * rng.integers(1, 33)) if aligned else int(rng.integers(1, 2049))
    out = int(16 * rng.integers(1, 257)) if aligned else int(rng.integers(1, 4097))
    return rng, dtype, rows, cols, out


@pytest.mark.parametrize("case_id", range(SWEEP))
def test_linear_shape_sweep(backend, case_id):
    rng, dtype, rows, cols, out = draw(case_id)
    print(f"case {case_id}: dtype {dtype} rows {rows} cols {cols} out {out}", flush=True)
    x = (2 * rng.standard_normal((rows, cols))).astype(np.float32)
    bits = weight_bits(rng.standard_normal((out, cols)), dtype)
    got = backend.linear(bits, x, dtype)
    ref = O.linear(x, bits, dtype)
    mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, dtype)).T
    bad = np.abs(got - ref) > 1e-5 * mag + 1e-4 * np.abs(ref)
    assert not bad.any(), (dtype, rows, cols, out, np.abs(got - ref).max())
    # integer-valued inputs: every partial sum is exact, so the order of the
    # sum cannot show
    xi = rng.integers(-8, 9, size=(rows, cols)).astype(np.float32)
    wi = weight_bits(rng.integers(-8, 9, size=(out, cols)).astype(np.float32), dtype)
    assert np.array_equal(backend.linear(wi, xi, dtype), O.linear(xi, wi, dtype))
