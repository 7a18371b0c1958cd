"""qg_matvec_norm_glu_dev_noalloc (include/qgemv.h): the no-allocation variant
of qg_matvec_norm_glu_dev, whose unfused path keeps the normalised x and the
[gate; up] outputs in a static per-GPU device array instead of hipMalloc'd
context buffers.  Checked through the C ABI against the allocating entry
point (same kernels: bit-identical h and residual sum) and against the
oracle (GEMV_TOL), on two calls in a row, the second with a smaller matrix,
on the unfused path (xb NULL; an F16 matrix, whose stream kernels have no
RMSNorm prologue) and on the fused path; and the size limit.  The no-allocation
calls run first, on a fresh context whose every allocation is made to fail
after the upload (qg_test_fail_allocations), so any allocation on that path
would fail the test; the allocating entry runs on another context."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

LIMIT = 262144          # floats in the static scratch array


def ref_h(oracle, raw, dtype, rows2, cols, xa, xb, nw, eps):
    """silu(gate . x) * (up . x) with x = rmsnorm(xa + xb) * nw on the CPU
    (math.rs:237-257 then quant.rs:188-205 and mlp.rs:36-43)."""
    x = xa if xb is None else (xa + xb).astype(np.float32)
    xn = oracle.rmsnorm(x, nw, eps)
    gu = oracle.mat_vec_mul(raw, dtype, rows2, cols, xn)
    half = rows2 // 2
    g, u = gu[:half].astype(np.float64), gu[half:].astype(np.float64)
    return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)


CASES = [  # (type, rows of [gate; up], cols, xb given)
    ((12, 2 * 4864, 896, False), (12, 2 * 128, 256, False)),    # Q4_K, unfused (xb NULL)
    ((1, 2 * 2048, 1024, True), (1, 2 * 64, 512, True)),        # F16: unfused with xb
    ((12, 2 * 1024, 2048, True), (12, 2 * 256, 512, True)),     # Q4_K, fused path
]


@pytest.mark.parametrize("pair", CASES, ids=["q4k-xb-null", "f16", "q4k-fused"])
def test_noalloc_matches_allocating_entry(rinf, ctx, oracle, synth, pair):
    import torch
    fresh = rinf.GpuContext(0)
    try:
        for i, (dtype, rows2, cols, with_xb) in enumerate(pair):
            seed = 500 + 17 * i + rows2 + cols + dtype
            raw = synth.gen_weights(dtype, rows2, cols, seed)
            rng = np.random.default_rng(seed)
            xa = rng.standard_normal(cols).astype(np.float32)
            xb = rng.standard_normal(cols).astype(np.float32) if with_xb else None
            nw = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
            mn = fresh.upload(raw, dtype, rows2, cols)
            ma = ctx.upload(raw, dtype, rows2, cols)
            d = lambda a: torch.from_numpy(a).cuda()
            dxa, dnw = d(xa), d(nw)
            dxb = d(xb) if xb is not None else None
            h = [torch.full((rows2 // 2,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(2)]
            s = [torch.full((cols,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(2)]
            st = torch.cuda.current_stream().cuda_stream
            torch.cuda.synchronize()
            fresh.fail_allocations(1 << 30)             # any allocation from here on fails
            try:
                mn.matvec_norm_glu_dev_noalloc(dxa, dxb, dnw, 1e-6, h[1], s[1], st)
                torch.cuda.synchronize()
            finally:
                fresh.fail_allocations(0)
            ma.matvec_norm_glu_dev(dxa, dxb, dnw, 1e-6, h[0], s[0], st)
            torch.cuda.synchronize()
            ha, hn = h[0].cpu().numpy(), h[1].cpu().numpy()
            sa, sn = s[0].cpu().numpy(), s[1].cpu().numpy()
            mn.free()
            ma.free()
            err = normwise_err(hn, ref_h(oracle, raw, dtype, rows2, cols, xa, xb, nw, 1e-6))
            print(f"call {i}: type {dtype} {rows2}x{cols} xb={'yes' if with_xb else 'NULL'}: "
                  f"err vs oracle {err:.2e}", flush=True)
            assert np.array_equal(ha.view(np.uint32), hn.view(np.uint32))
            assert np.array_equal(sa.view(np.uint32), sn.view(np.uint32))
            assert err <= GEMV_TOL
    finally:
        fresh.close()


def test_noalloc_size_limit(rinf, ctx, synth):
    """round_up(cols, 64) + rows beyond the static array: QG_ERR_SHAPE, h untouched."""
    import torch
    cols = 256
    rows2 = LIMIT - cols + 2            # one [gate; up] pair too many
    raw = synth.gen_weights(12, rows2, cols, 3)
    m = ctx.upload(raw, 12, rows2, cols)
    xa = torch.ones(cols, dtype=torch.float32, device="cuda")
    h = torch.full((rows2 // 2,), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(rinf.QgemvError) as e:
        m.matvec_norm_glu_dev_noalloc(xa, None, xa, 1e-6, h)
    assert e.value.status == 7
    torch.cuda.synchronize()
    assert bool((h == 7.0).all())
    m.free()
