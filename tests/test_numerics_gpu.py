"""The GEMV's x format under stress: the quantized types take x as 22-bit
fixed point per 32-element segment (|Y| < 2^22 of the segment's maximum,
three signed-byte digit planes), so small elements that share a segment with
a large one keep few bits.  These tests put such segments in x and check the
device against the reference's sequential f32 loop (oracle.mat_vec_mul,
src/quant.rs:188-205) and against an exact float64 product of the
dequantized weights (oracle.dequantize, bit-exact with quant.rs:356-840),
both within the north-star bound GEMV_TOL (normwise, 1e-4).

Tiny x (every element scaled by 1e-30): the segment scale k is capped at
2^122, which keeps all 22 bits down to a segment maximum of ~7.9e-31.

Non-finite x: the reference's sequential sum makes a row +inf where it meets
+inf (with a positive weight), -inf, or NaN where signs mix, a weight is zero
or x holds a NaN.  The device matches that row by row for every type and
every kernel (stream, LDS ring, wave-private): a workgroup whose x has a
non-finite segment, or one whose maximum exceeds 2^64, recomputes its rows as
f32 sums of rounded products.  Huge finite x (|x| > 2^64) takes the same path
and is compared within GEMV_TOL.
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


def same_classes(y, ref):
    """Row by row: NaN where the reference has NaN, otherwise the same value
    (the reference's +-inf, or for finite rows within the GEMV tolerance)."""
    y, ref = np.asarray(y), np.asarray(ref)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), \
        f"NaN rows differ: device {np.flatnonzero(np.isnan(y))[:8]} ref {np.flatnonzero(np.isnan(ref))[:8]}"
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(y), inf)
    assert np.array_equal(y[inf], ref[inf])
    fin = np.isfinite(ref)
    if fin.any():
        assert normwise_err(y[fin], ref[fin]) <= GEMV_TOL


def ref_mv(oracle, raw, dtype, rows, cols, x):
    return (oracle.mat_vec_mul(raw, dtype, rows, cols, x) if rows * cols <= 4_000_000
            else oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x))


KIND = {0: "generic", 1: "stream", 2: "ring", 3: "wave"}


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("bad", ["inf", "-inf", "nan", "both-infs", "huge"])
def test_non_finite_x(ctx, oracle, synth, dtype, bad):
    """256 x 1024 (stream kernel): one inf, one -inf, one NaN, an inf and a
    -inf in different segments, or one element of 1e30 (finite: diverted)."""
    rows, cols = 256, 1024
    raw = synth.gen_blocks(dtype, rows, cols, 77 + dtype)
    x = synth.gen_x(cols, 77)
    if bad == "both-infs":
        x[333], x[700] = np.inf, -np.inf
    elif bad == "huge":
        x[333] = np.float32(1e30)
    else:
        x[333] = np.float32(bad)
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.zeros(rows, np.float32)
    m.matvec_host(x, y)
    kind = m.kernel_kind
    m.free()
    ref = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
    if bad == "huge":
        assert np.isfinite(ref).all()
    else:
        assert not np.isfinite(ref).any()        # every row meets the column
    print(f"{NAMES[dtype]} {bad} ({KIND.get(kind)}): ref NaN rows {int(np.isnan(ref).sum())}, "
          f"+inf {int((ref == np.inf).sum())}, -inf {int((ref == -np.inf).sum())}", flush=True)
    same_classes(y, ref)


# every kernel family on a non-finite x: Q4_K rows of 14336 (wave-private at
# 4096 rows, stream at 4000), 18944 (stream), the LDS ring's types at 14336,
# straddling row groups (896)
BIG = [(12, 4096, 14336), (12, 4000, 14336), (12, 3584, 18944), (13, 4096, 14336), (14, 4096, 14336),
       (8, 4096, 14336), (2, 4096, 14336), (12, 512, 896), (14, 512, 896)]


@pytest.mark.parametrize("dtype,rows,cols", BIG, ids=[f"{NAMES[t]}-{r}x{c}" for t, r, c in BIG])
def test_non_finite_x_every_kernel(ctx, oracle, synth, dtype, rows, cols):
    """+inf and -inf in two segments (rows mix to NaN or keep one sign), a
    NaN, then one element of 1e30 (finite, but past the fixed-point range:
    the f32 path), through the kernel each shape plans."""
    raw = synth.gen_blocks(dtype, rows, cols, 7 + dtype + cols)
    m = ctx.upload(raw, dtype, rows, cols)
    kind = m.kernel_kind
    for case in ("infs", "nan", "huge"):
        x = synth.gen_x(cols, 7 + cols)
        if case == "infs":
            x[cols // 3], x[cols // 3 + 97] = np.inf, -np.inf
        elif case == "nan":
            x[cols - 5] = np.nan
        else:
            x[cols // 2] = np.float32(1e30)
        y = np.zeros(rows, np.float32)
        m.matvec_host(x, y)
        ref = ref_mv(oracle, raw, dtype, rows, cols, x)
        print(f"{NAMES[dtype]} {rows}x{cols} {case} ({KIND.get(kind)}): NaN {int(np.isnan(ref).sum())}, "
              f"+inf {int((ref == np.inf).sum())}, -inf {int((ref == -np.inf).sum())}", flush=True)
        same_classes(y, ref)
    # and a clean x afterwards: the fast path again
    x = synth.gen_x(cols, 8 + cols)
    y = np.zeros(rows, np.float32)
    m.matvec_host(x, y)
    m.free()
    assert normwise_err(y, ref_mv(oracle, raw, dtype, rows, cols, x)) <= GEMV_TOL


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_tiny_x(ctx, oracle, synth, dtype, shape):
    """x ~ N(0,1) * 1e-30: every segment keeps its 22 bits (k <= 2^122)."""
    rows, cols = shape
    seed = synth.config_seed(1) + 7 * rows + cols + dtype
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    x = (synth.gen_x(cols, seed).astype(np.float64) * 1e-30).astype(np.float32)
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.zeros(rows, np.float32)
    m.matvec_host(x, y)
    m.free()
    y32, y64 = ref_pair(oracle, raw, dtype, rows, cols, x)
    e_ref, e_exact = normwise_err(y, y32), normwise_err(y, y64)
    print(f"{NAMES[dtype]} {rows}x{cols} x*1e-30: vs reference {e_ref:.2e}, vs exact {e_exact:.2e}", flush=True)
    assert e_ref <= GEMV_TOL
    assert e_exact <= GEMV_TOL


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
    same_classes(y_bad, oracle.mat_vec_mul(raw, dtype, rows, cols, xb))
    assert np.array_equal(y_clean.view(np.uint32), y_again.view(np.uint32))
    assert normwise_err(y_clean, oracle.mat_vec_mul(raw, dtype, rows, cols, x)) <= GEMV_TOL


def zero_weight_columns(raw, dtype, rows, cols, cidx):
    """Set the weight of column cidx[s] of every row to exactly zero (Q8_0:
    code 0; Q4_0: nibble 8, byte 2 + j/2 of its block, low nibble for even
    j -- quant.rs:106-121)."""
    raw = raw.copy()
    bb = 34 if dtype == 8 else 18
    for r in range(rows):
        f = r * cols + cidx                               # flat element index
        b, j = f // 32, f % 32
        if dtype == 8:
            raw[b * bb + 2 + j] = 0
        else:
            byte = b * bb + 2 + j // 2
            lo = (j % 2) == 0
            raw[byte] = np.where(lo, (raw[byte] & 0xF0) | 0x08, (raw[byte] & 0x0F) | 0x80)
    return raw


@pytest.mark.parametrize("dtype", [8, 2], ids=["Q8_0", "Q4_0"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_outlier_at_zero_weight(ctx, oracle, synth, dtype, shape):
    """The case the normwise gate above cannot see: one element of every
    segment scaled 1e4x, and every row's weight at that column zero, so no
    product with a segment maximum enters y and the small elements' 22-bit
    fixed-point error is all there is.  Checked against the guarantee of the
    format, per row: |y - exact| <= 2^-22 sum_i |w_i| m_seg(i) (each
    element's error is at most half a step of 2^-22 of its segment's maximum)
    plus 2^-20 sum_i |w_i x_i| for the f32 rounding of the scaled terms.  The
    normwise error this leaves is printed (it is not within GEMV_TOL here:
    the reference's f32 loop keeps 24 bits of every small element)."""
    rows, cols = shape
    seed = synth.config_seed(1) + 7 * rows + cols + dtype
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(cols).astype(np.float32)
    cidx = np.arange(0, cols, 32) + rng.integers(0, 32, cols // 32)
    x[cidx] *= np.float32(1e4)
    raw = zero_weight_columns(synth.gen_blocks(dtype, rows, cols, seed), dtype, rows, cols, cidx)
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.full(rows, np.nan, np.float32)
    m.matvec_host(x, y)
    m.free()
    y32, y64 = ref_pair(oracle, raw, dtype, rows, cols, x)
    w = np.abs(oracle.dequantize(raw, dtype, rows * cols)[:rows * cols].reshape(rows, cols).astype(np.float64))
    assert np.all(w[:, cidx] == 0.0)
    mseg = np.repeat(np.abs(x.astype(np.float64)).reshape(-1, 32).max(axis=1), 32)
    bound = 2.0 ** -22 * (w @ mseg) + 2.0 ** -20 * (w @ np.abs(x.astype(np.float64)))
    err = np.abs(y.astype(np.float64) - y64)
    print(f"{NAMES[dtype]} {rows}x{cols} outliers at zero weights: normwise vs exact "
          f"{normwise_err(y, y64):.2e} (reference {normwise_err(y32, y64):.2e}), "
          f"max err / bound {np.max(err / bound):.3f}", flush=True)
    assert np.all(np.isfinite(y))
    assert np.all(err <= bound)


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
def test_precision_f32_mode(rinf, oracle, synth, dtype):
    """qg_set_precision(QG_PRECISION_F32): every product rounded to f32 and
    summed in f32, as the reference's loop does (quant.rs:195-204), in a
    lane-parallel order.  The zero-weight outlier case above comes within
    1e-4 of the exact product (the reference's own distance, ~1e-6), and
    plain N(0,1) x matches the reference for every type: uploaded (the
    repacked layout for Q8_0 and the K-quants, two-row groups at cols = 896;
    the GGUF layout for the others), wrapped in device memory (the GGUF
    layout, K-quant rows straddling blocks at cols = 896) and through the
    keyed drop-in; non-finite x gives the reference's +-inf / NaN row by
    row."""
    c = rinf.GpuContext(0)
    try:
        with pytest.raises(rinf.QgemvError) as e:
            c.set_precision(2)
        assert e.value.status == 1
        c.set_precision(rinf.PRECISION_F32)
        for rows, cols in ((256, 896), (512, 3584)):
            seed = 300 + rows + dtype
            raw = synth.gen_blocks(dtype, rows, cols, seed)
            x = synth.gen_x(cols, seed)
            m = c.upload(raw, dtype, rows, cols)
            y = np.full(rows, np.nan, np.float32)
            m.matvec_host(x, y)
            m.free()
            ref = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
            assert normwise_err(y, ref) <= 1e-5, (rows, cols, normwise_err(y, ref))
            y2 = np.full(rows, np.nan, np.float32)
            c.mat_vec_mul(raw, dtype, x, y2, rows, cols)
            assert np.array_equal(y2, y)
            import torch
            buf = torch.zeros(raw.nbytes + 4096, dtype=torch.uint8, device="cuda")
            buf[:raw.nbytes] = torch.from_numpy(raw).cuda()
            w = c.wrap_device(buf, dtype, rows, cols)
            y3 = np.full(rows, np.nan, np.float32)
            w.matvec_host(x, y3)
            w.free()
            assert normwise_err(y3, ref) <= 1e-5, (rows, cols, "wrapped", normwise_err(y3, ref))
        if dtype in (8, 2):
            for rows, cols in SHAPES:
                seed = synth.config_seed(1) + 7 * rows + cols + dtype
                rng = np.random.default_rng(seed)
                x = rng.standard_normal(cols).astype(np.float32)
                cidx = np.arange(0, cols, 32) + rng.integers(0, 32, cols // 32)
                x[cidx] *= np.float32(1e4)
                raw = zero_weight_columns(synth.gen_blocks(dtype, rows, cols, seed), dtype, rows, cols, cidx)
                m = c.upload(raw, dtype, rows, cols)
                y = np.full(rows, np.nan, np.float32)
                m.matvec_host(x, y)
                m.free()
                y32, y64 = ref_pair(oracle, raw, dtype, rows, cols, x)
                e_exact, e_ref = normwise_err(y, y64), normwise_err(y32, y64)
                print(f"{NAMES[dtype]} {rows}x{cols} outliers at zero weights, f32 mode: vs exact {e_exact:.2e} "
                      f"(reference {e_ref:.2e})", flush=True)
                assert e_exact <= GEMV_TOL
        # non-finite x: the reference's +-inf / NaN row by row (the f32 sum of
        # rounded products decides these classes whatever its order)
        rows, cols = 256, 1024
        raw = synth.gen_blocks(dtype, rows, cols, 77 + dtype)
        for bad in ("inf", "-inf", "nan", "both-infs"):
            x = synth.gen_x(cols, 77)
            if bad == "both-infs":
                x[333], x[700] = np.inf, -np.inf
            else:
                x[333] = np.float32(bad)
            y = np.zeros(rows, np.float32)
            c.mat_vec_mul(raw, dtype, x, y, rows, cols)
            same_classes(y, oracle.mat_vec_mul(raw, dtype, rows, cols, x))
    finally:
        c.close()
