"""The GEMV's x format under stress: the quantized types take x as 22-bit
fixed point per 32-element segment (|Y| < 2^22 of the segment's maximum,
three signed-byte digit planes), so small elements that share a segment with
a large one keep few bits.  These tests put such segments in x and check the
device against the reference's sequential f32 loop (oracle.mat_vec_mul,
src/quant.rs:188-205) and against an exact float64 product of the
dequantized weights (oracle.dequantize, bit-exact with quant.rs:356-840),
both within the north-star bound GEMV_TOL (normwise, 1e-4).

Non-finite x: the reference's sequential sum makes a row +-inf or NaN when
x holds an inf or a NaN; the device makes every row that meets such an
element NaN for the quantized types (the segment's 1/k is NaN) and follows
IEEE arithmetic for F16/F32 (x stays f32).  The tests pin exactly that.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

TYPES = [0, 1, 2, 6, 8, 12, 13, 14]
NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
QUANT = (2, 6, 8, 12, 13, 14)
SHAPES = [(896, 896), (4096, 14336)]


def x_outliers(cols, seed):
    """N(0,1) with one element of every 32-element segment scaled by 1e4."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(cols).astype(np.float32)
    idx = np.arange(0, cols, 32) + rng.integers(0, 32, cols // 32)
    x[idx] *= np.float32(1e4)
    return x


def x_loguniform(cols, seed):
    """|x| log-uniform in [1e-6, 1e3], random signs."""
    rng = np.random.default_rng(seed)
    mag = 10.0 ** rng.uniform(-6.0, 3.0, cols)
    return (mag * rng.choice([-1.0, 1.0], cols)).astype(np.float32)


def ref_pair(oracle, raw, dtype, rows, cols, x):
    """(the reference's f32 loop, the exact product in float64)."""
    y32 = (oracle.mat_vec_mul(raw, dtype, rows, cols, x) if rows * cols <= 4_000_000
           else oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x))
    w = oracle.dequantize(raw, dtype, rows * cols)[:rows * cols].reshape(rows, cols).astype(np.float64)
    return y32, w @ x.astype(np.float64)


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
@pytest.mark.parametrize("dist", ["outliers", "loguniform"])
def test_adversarial_x(ctx, oracle, synth, dtype, shape, dist):
    rows, cols = shape
    seed = synth.config_seed(1) + 101 * rows + cols + dtype
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    x = x_outliers(cols, seed) if dist == "outliers" else x_loguniform(cols, seed)
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.full(rows, np.nan, np.float32)
    m.matvec_host(x, y)
    m.free()
    y32, y64 = ref_pair(oracle, raw, dtype, rows, cols, x)
    e_ref, e_exact, e_cpu = normwise_err(y, y32), normwise_err(y, y64), normwise_err(y32, y64)
    print(f"{NAMES[dtype]} {rows}x{cols} {dist}: vs reference {e_ref:.2e}, vs exact {e_exact:.2e} "
          f"(reference vs exact {e_cpu:.2e})", flush=True)
    assert e_ref <= GEMV_TOL
    assert e_exact <= GEMV_TOL


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("bad", ["inf", "-inf", "nan"])
def test_non_finite_x(ctx, oracle, synth, dtype, bad):
    rows, cols = 256, 1024
    raw = synth.gen_blocks(dtype, rows, cols, 77 + dtype)
    x = synth.gen_x(cols, 77)
    x[333] = np.float32(bad)
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.zeros(rows, np.float32)
    m.matvec_host(x, y)
    m.free()
    ref = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
    # every row meets column 333: every output of both sides is non-finite
    assert not np.isfinite(ref).any()
    assert not np.isfinite(y).any()
    if dtype in QUANT:
        assert np.isnan(y).all()                 # the segment's 1/k is NaN
    else:
        # f32 x: IEEE arithmetic as in the reference -- same infinities where
        # the reference's row has one, NaN where it has NaN
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        fin = ~np.isnan(ref)
        assert np.array_equal(np.sign(y[fin]), np.sign(ref[fin]))


@pytest.mark.parametrize("dtype", QUANT, ids=[NAMES[t] for t in QUANT])
def test_clean_call_after_non_finite(ctx, oracle, synth, dtype):
    """A call with an inf in x carries nothing into the next call: the same
    clean x gives bit-identical y before and after it (straddling row groups
    for the K-quants at cols = 896)."""
    rows, cols = 64, 896 if dtype in (12, 13, 14) else 64
    raw = synth.gen_blocks(dtype, rows, cols, 91 + dtype)
    x = synth.gen_x(cols, 91)
    m = ctx.upload(raw, dtype, rows, cols)
    y_clean = np.zeros(rows, np.float32)
    m.matvec_host(x, y_clean)
    xb = x.copy()
    xb[5] = np.inf
    y_bad = np.zeros(rows, np.float32)
    m.matvec_host(xb, y_bad)
    y_again = np.zeros(rows, np.float32)
    m.matvec_host(x, y_again)
    m.free()
    assert np.isnan(y_bad).all()
    assert np.array_equal(y_clean.view(np.uint32), y_again.view(np.uint32))
    assert normwise_err(y_clean, oracle.mat_vec_mul(raw, dtype, rows, cols, x)) <= GEMV_TOL
