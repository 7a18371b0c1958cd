"""GPU parity of the mat-vecs with an input prologue (include/qgemv.h):
qg_matvec_norm_dev, RmsNorm of xa + xb then the mat-vec (src/math.rs:237-257,
src/transformer.rs:31-46, src/quant.rs:178-206), against the oracle's rmsnorm
+ mat_vec_mul; qg_matvec_silu_dev, silu(g) * u then the mat-vec
(src/mlp.rs:36-45, src/math.rs:137-146), against the oracle's silu + product
+ mat_vec_mul.

y within GEMV_TOL normwise of the oracle; sum_out (xa + xb) bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

TYPES = [0, 1, 2, 6, 8, 12, 13, 14]
NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
EPS = 1e-6

# Qwen2-0.5B / 7B projection shapes (cols = embed), the lm_head of the tied
# 0.5B model, small matrices, and row-group counts of 1025..1792 with short
# teams (5..7 teams of 16 lanes per CU: workgroups that are not whole waves
# unless the planner rounds them up).
SHAPES = [(896, 896), (128, 896), (4864, 896), (600, 256), (256, 256), (3584, 3584), (1200, 256),
          (1500, 512), (1700, 256)]


def run(ctx, rinf, m, xa, xb, nw, rows, cols, with_sum=True, offset=0):
    import torch
    dev = lambda a: torch.from_numpy(a).cuda()
    pad = torch.zeros(cols + offset, dtype=torch.float32, device="cuda")
    pad[offset:] = dev(xa)
    dxa = pad[offset:]
    dxb = dev(xb) if xb is not None else None
    dnw = dev(nw)
    dy = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    ds = torch.full((cols,), float("nan"), dtype=torch.float32, device="cuda") if with_sum else None
    torch.cuda.synchronize()
    m.matvec_norm_dev(dxa, dxb, dnw, EPS, dy, ds, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return dy.cpu().numpy(), (ds.cpu().numpy() if with_sum else None)


def inputs(synth, rows, cols, seed):
    rng = np.random.default_rng(seed)
    xa = (rng.standard_normal(cols) * 3).astype(np.float32)
    xb = rng.standard_normal(cols).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    return xa, xb, nw


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_norm_matvec_parity(ctx, rinf, oracle, synth, dtype, shape):
    rows, cols = shape
    seed = synth.config_seed(1) + 31 * rows + cols
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    xa, xb, nw = inputs(synth, rows, cols, seed)
    m = ctx.upload(raw, dtype, rows, cols)
    y, s = run(ctx, rinf, m, xa, xb, nw, rows, cols)
    kind = m.kernel_kind
    m.free()
    x = (xa + xb).astype(np.float32)
    ref = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, oracle.rmsnorm(x, nw, EPS))
    err = normwise_err(y, ref)
    print(f"{NAMES[dtype]} {rows}x{cols} kernel={kind} err={err:.2e}", flush=True)
    assert np.array_equal(s.view(np.uint32), x.view(np.uint32))
    assert err <= GEMV_TOL


@pytest.mark.parametrize("dtype", [12, 14, 8], ids=["Q4_K", "Q6_K", "Q8_0"])
def test_norm_matvec_variants(ctx, rinf, oracle, synth, dtype):
    """No xb, no sum_out, and an x that is not 16-byte aligned (the
    two-kernel path) give the same values as the fused kernel."""
    rows, cols = 896, 896
    seed = synth.config_seed(1) + dtype
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    xa, xb, nw = inputs(synth, rows, cols, seed)
    m = ctx.upload(raw, dtype, rows, cols)
    fused, _ = run(ctx, rinf, m, xa, xb, nw, rows, cols, with_sum=False)
    x = (xa + xb).astype(np.float32)
    shifted, s = run(ctx, rinf, m, x, None, nw, rows, cols, offset=1)
    alone, _ = run(ctx, rinf, m, x, None, nw, rows, cols)
    m.free()
    ref = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, oracle.rmsnorm(x, nw, EPS))
    for y in (fused, shifted, alone):
        assert normwise_err(y, ref) <= GEMV_TOL
    assert np.array_equal(s, x)


@pytest.mark.parametrize("dtype", [12, 14, 8], ids=["Q4_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("scale", [1e-15, 1e15], ids=["1e-15", "1e15"])
def test_norm_matvec_input_scale(ctx, rinf, oracle, synth, dtype, scale):
    """RmsNorm removes the scale of xa + xb (eps negligible here), so inputs
    at 1e-15 and 1e15 stay within GEMV_TOL of the oracle and of the unscaled
    result.  The kernel converts (xa + xb) * nw to fixed point before the
    1/rms factor; at 1e-15 the segment maxima (about 1e-14) need 1/k below
    2^-64 for full precision."""
    rows, cols = 1024, 3584
    eps = 1e-37
    seed = synth.config_seed(1) + 5 * dtype + 3
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    xa, xb, nw = inputs(synth, rows, cols, seed)
    m = ctx.upload(raw, dtype, rows, cols)
    outs = {}
    for s in (1.0, scale):
        xas, xbs = (xa * np.float32(s)).astype(np.float32), (xb * np.float32(s)).astype(np.float32)
        import torch
        dev = lambda a: torch.from_numpy(a).cuda()
        dy = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        m.matvec_norm_dev(dev(xas), dev(xbs), dev(nw), eps, dy, None, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        y = dy.cpu().numpy()
        x = (xas + xbs).astype(np.float32)
        ref = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, oracle.rmsnorm(x, nw, eps))
        err = normwise_err(y, ref)
        print(f"{NAMES[dtype]} scale {s:g} err={err:.2e}", flush=True)
        assert err <= GEMV_TOL
        outs[s] = y
    m.free()
    assert normwise_err(outs[scale], outs[1.0]) <= GEMV_TOL


def test_norm_matvec_errors(ctx, rinf, synth):
    import torch
    rows, cols = 64, 256
    m = ctx.upload(synth.gen_blocks(12, rows, cols, 5), 12, rows, cols)
    xa = torch.zeros(cols, dtype=torch.float32, device="cuda")
    nw = torch.ones(cols, dtype=torch.float32, device="cuda")
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    with pytest.raises(rinf.QgemvError) as e:
        m.matvec_norm_dev(xa, None, nw, EPS, y, xa)            # sum_out overlaps xa
    assert e.value.status == 1                                 # QG_ERR_INVALID_ARG
    m.free()


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", [(3584, 18944), (896, 4864), (256, 512), (1200, 256)],
                         ids=["3584x18944", "896x4864", "256x512", "1200x256"])
def test_silu_matvec_parity(ctx, rinf, oracle, synth, dtype, shape):
    import torch
    rows, cols = shape
    seed = synth.config_seed(1) + 17 * rows + cols
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(cols) * 4).astype(np.float32)
    u = rng.standard_normal(cols).astype(np.float32)
    m = ctx.upload(raw, dtype, rows, cols)
    dg, du = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    dy = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    m.matvec_silu_dev(dg, du, dy, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    m.free()
    x = np.array([oracle.silu(float(v)) for v in g], np.float32) * u
    ref = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x.astype(np.float32))
    err = normwise_err(y, ref)
    print(f"silu {NAMES[dtype]} {rows}x{cols} err={err:.2e}", flush=True)
    assert err <= GEMV_TOL


# (4864, 896): two rows per group for the K-quants; (64, 288) and (1000, 288):
# eight rows per group (rows of 9 segments of 32)
GLU_SHAPES = [(t, s) for t in TYPES for s in [(600, 256), (1200, 256), (4864, 896), (40, 512), (64, 288),
                                            (1000, 288)]] + \
    [(t, s) for t in (12, 13, 14, 8, 2, 6) for s in [(18944, 3584), (14336, 4096)]]


def glu_inputs(synth, dtype, H, cols, seed):
    gate = synth.gen_blocks(dtype, H, cols, seed)
    up = synth.gen_blocks(dtype, H, cols, seed + 1)
    return gate, up


@pytest.mark.parametrize("dtype,shape", GLU_SHAPES, ids=[f"{NAMES[t]}-{h}x{c}" for t, (h, c) in GLU_SHAPES])
def test_norm_glu_matvec_parity(ctx, rinf, oracle, synth, dtype, shape):
    """qg_matvec_norm_glu_dev on qg_mat_stack([gate, up]): h = silu(gate.x) *
    (up.x) with x = rmsnorm(xa + xb) * nw (mlp.rs:31-43) within GEMV_TOL of
    the oracle; within a few ulp of silu applied to the stacked matrix's own
    norm mat-vec (the pairing kernel forms the same dot products); sum_out
    bit-exact."""
    import torch
    H, cols = shape
    seed = synth.config_seed(1) + 7 * H + cols + dtype
    gate, up = glu_inputs(synth, dtype, H, cols, seed)
    xa, xb, nw = inputs(synth, H, cols, seed)
    mg, mu = ctx.upload(gate, dtype, H, cols), ctx.upload(up, dtype, H, cols)
    gu = ctx.stack([mg, mu])
    mg.free()
    mu.free()
    assert (gu.rows, gu.cols) == (2 * H, cols)
    dev = lambda a: torch.from_numpy(a).cuda()
    dxa, dxb, dnw = dev(xa), dev(xb), dev(nw)
    dh = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    ds = torch.full((cols,), float("nan"), dtype=torch.float32, device="cuda")
    dy = torch.full((2 * H,), float("nan"), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    gu.matvec_norm_glu_dev(dxa, dxb, dnw, EPS, dh, ds, stream)
    gu.matvec_norm_dev(dxa, dxb, dnw, EPS, dy, None, stream)
    torch.cuda.synchronize()
    h, s, y = dh.cpu().numpy(), ds.cpu().numpy(), dy.cpu().numpy().astype(np.float64)
    kind = gu.kernel_kind
    gu.free()
    x = (xa + xb).astype(np.float32)
    assert np.array_equal(s.view(np.uint32), x.view(np.uint32))
    xn = oracle.rmsnorm(x, nw, EPS)
    g_ref = oracle.mat_vec_mul_rows(gate, dtype, H, cols, xn)
    u_ref = oracle.mat_vec_mul_rows(up, dtype, H, cols, xn)
    ref = np.array([oracle.silu(float(v)) for v in g_ref], np.float32) * u_ref
    err = normwise_err(h, ref)
    # silu in float64 of the device's own gate/up values
    g64, u64 = y[:H], y[H:]
    own = g64 / (1.0 + np.exp(-g64)) * u64
    ulp = np.abs(h - own) / np.maximum(np.abs(own), 1e-30)
    print(f"glu {NAMES[dtype]} {H}x{cols} kernel={kind} err={err:.2e} max rel vs own {ulp.max():.1e}", flush=True)
    assert err <= GEMV_TOL
    assert ulp.max() <= 6e-7


@pytest.mark.parametrize("dtype", [12, 14, 13, 8], ids=["Q4_K", "Q6_K", "Q5_K", "Q8_0"])
@pytest.mark.parametrize("shape", [(1024, 3584), (4864, 896)], ids=["1024x3584", "4864x896"])
def test_glu_wrapped_layout_matches(ctx, rinf, synth, dtype, shape):
    """The paired [gate; up] kernel over GGUF-layout bytes wrapped from device
    memory gives the same h, bit for bit, as over the uploaded (for Q4_K/Q6_K
    repacked) stacked matrix."""
    import torch
    H, cols = shape
    seed = 99 + H + dtype
    gate, up = glu_inputs(synth, dtype, H, cols, seed)
    both = np.concatenate([gate.view(np.uint8).reshape(-1), up.view(np.uint8).reshape(-1)])
    xa, xb, nw = inputs(synth, H, cols, seed)
    buf = torch.zeros(both.nbytes + 1024, dtype=torch.uint8, device="cuda")
    buf[:both.nbytes] = torch.from_numpy(both).cuda()
    wr = ctx.wrap_device(buf, dtype, 2 * H, cols)
    mg, mu = ctx.upload(gate, dtype, H, cols), ctx.upload(up, dtype, H, cols)
    gu = ctx.stack([mg, mu])
    dev = lambda a: torch.from_numpy(a).cuda()
    dxa, dxb, dnw = dev(xa), dev(xb), dev(nw)
    h1 = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    h2 = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    gu.matvec_norm_glu_dev(dxa, dxb, dnw, EPS, h1, None, st)
    wr.matvec_norm_glu_dev(dxa, dxb, dnw, EPS, h2, None, st)
    torch.cuda.synchronize()
    a, b = h1.cpu().numpy(), h2.cpu().numpy()
    for m in (wr, gu, mg, mu):
        m.free()
    del buf
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_glu_and_stack_errors(ctx, rinf, synth):
    import torch
    m = ctx.upload(synth.gen_blocks(8, 65, 256, 3), 8, 65, 256)
    xa = torch.zeros(256, dtype=torch.float32, device="cuda")
    h = torch.zeros(65, dtype=torch.float32, device="cuda")
    with pytest.raises(rinf.QgemvError) as e:
        m.matvec_norm_glu_dev(xa, xa, xa, EPS, h)              # odd row count
    assert e.value.status == 7                                 # QG_ERR_SHAPE
    # a first part that does not end on a block boundary
    a = ctx.upload(synth.gen_blocks(12, 1, 288, 4), 12, 1, 288)
    b = ctx.upload(synth.gen_blocks(12, 1, 288, 5), 12, 1, 288)
    c = ctx.upload(synth.gen_blocks(8, 1, 288, 6), 8, 1, 288)
    with pytest.raises(rinf.QgemvError) as e:
        ctx.stack([a, b])
    assert e.value.status == 7
    with pytest.raises(rinf.QgemvError) as e:
        ctx.stack([c, a])                                      # types differ
    assert e.value.status == 7
    for x in (m, a, b, c):
        x.free()


@pytest.mark.parametrize("dtype", [12, 14, 8, 1], ids=["Q4_K", "Q6_K", "Q8_0", "F16"])
def test_stacked_matvec_bit_exact(ctx, rinf, synth, dtype):
    """qg_mat_stack([A, B, C]) · x is A · x, B · x, C · x one after the other,
    bit for bit (rows are formed by the same per-row code)."""
    import torch
    cols, rows = 1024, (512, 128, 300)
    parts = [synth.gen_blocks(dtype, r, cols, 60 + i) for i, r in enumerate(rows)]
    mats = [ctx.upload(p, dtype, r, cols) for p, r in zip(parts, rows)]
    st = ctx.stack(mats)
    x = torch.from_numpy(np.random.default_rng(9).standard_normal(cols).astype(np.float32)).cuda()
    ys = [torch.zeros(r, dtype=torch.float32, device="cuda") for r in rows]
    y = torch.zeros(sum(rows), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    for m, yy in zip(mats, ys):
        m.matvec_dev(x, yy, stream)
    st.matvec_dev(x, y, stream)
    torch.cuda.synchronize()
    cat = torch.cat(ys).cpu().numpy()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), cat.view(np.uint32))
    for m in mats + [st]:
        m.free()
