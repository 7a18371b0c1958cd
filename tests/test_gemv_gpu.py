"""GPU parity: the HIP path through the C ABI vs the CPU oracle.

Dequantized values must match bit for bit; mat-vec outputs within the
north-star tolerance, max|y - y_ref| / max|y_ref| <= 1e-4 (GEMV_TOL), where
y_ref is the reference's sequential f32 CPU loop (src/quant.rs:188-205).
"""
from __future__ import annotations

import ctypes
import json
import pathlib

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

TYPES = [0, 1, 2, 6, 8, 12, 13, 14]
NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "kat_blocks.json").read_text())
FAST = (1, 2, 3)       # stream kernel, with the LDS ring or the wave-private kernel (kind 0: per-element fallback)


def gpu_gemv(ctx, raw, dtype, rows, cols, x):
    m = ctx.upload(raw, dtype, rows, cols)
    y = np.full(rows, np.nan, np.float32)
    m.matvec_host(x, y)
    kind = m.kernel_kind
    m.free()
    return y, kind


def ref_gemv(oracle, raw, dtype, rows, cols, x):
    if rows * cols <= 4_000_000:
        return oracle.mat_vec_mul(raw, dtype, rows, cols, x)       # faithful loop
    return oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x)      # bit-identical, threaded


# BASELINE.json configs[1] (per-type sweep at Qwen2-0.5B shapes) plus the
# row-group cases: cols % 256 in {32, 64, 128} and cols % 64 == 32.
# Multi-wave teams (rows of more than 64 items: 14336 and 18944 columns),
# rows that do not fill the last batch; 1200 and 1700 row groups of short
# teams (5 and 7 teams of 16 lanes per CU).
SHAPES = [(896, 896), (128, 896), (896, 4864), (33, 96), (40, 160), (24, 192), (10, 640),
          (7, 4096), (3, 14336), (37, 18944), (129, 3584), (70, 14336), (21, 8320), (1200, 256),
          (1700, 256)]


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_gemv_parity(ctx, oracle, synth, dtype, shape):
    rows, cols = shape
    seed = synth.config_seed(1) + rows * 7 + cols
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    x = synth.gen_x(cols, seed)
    y, kind = gpu_gemv(ctx, raw, dtype, rows, cols, x)
    ref = ref_gemv(oracle, raw, dtype, rows, cols, x)
    err = normwise_err(y, ref)
    print(f"{NAMES[dtype]} {rows}x{cols} kernel={kind} err={err:.2e}", flush=True)
    assert kind in FAST
    assert err <= GEMV_TOL


# (37, 14336), (1030, 8448), (9000, 8448), (3584, 18944): the LDS ring kernel
# (uploaded Q5_K, Q6_K, Q8_0 where their rows make several-wave teams; Q4_K
# rows take the stream kernel) against the stream kernel (wrapped), with
# partial stages, the narrowest ring row, nine stages per team and the 7B
# down projection
WRAP_SHAPES = [(896, 896), (128, 896), (4096, 14336), (37, 18944), (1200, 256), (21, 8320), (64, 288),
               (37, 14336), (1030, 8448), (9000, 8448), (3584, 18944)]


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", WRAP_SHAPES, ids=[f"{r}x{c}" for r, c in WRAP_SHAPES])
def test_wrapped_bytes_match_upload(ctx, oracle, synth, dtype, shape):
    """qg_wrap_device keeps the GGUF layout (its kernels read the file's
    blocks), qg_upload of Q8_0/Q4_K/Q5_K/Q6_K also keeps a repacked copy for the
    stream kernels: both give the same y, bit for bit, and the oracle's within
    GEMV_TOL; the plain and the RMSNorm-prologue kernels of both layouts.  An
    uploaded matrix on the wave-private kernel (kind 3) adds the same item sums
    in another order: its plain y is held to GEMV_TOL of the oracle instead."""
    import torch
    rows, cols = shape
    seed = synth.config_seed(1) + rows * 13 + cols + dtype
    raw = synth.gen_blocks(dtype, rows, cols, seed)
    x = synth.gen_x(cols, seed)
    buf = torch.zeros(raw.nbytes + 1024, dtype=torch.uint8, device="cuda")
    buf[:raw.nbytes] = torch.from_numpy(raw.view(np.uint8).reshape(-1)).cuda()
    up = ctx.upload(raw, dtype, rows, cols)
    wr = ctx.wrap_device(buf, dtype, rows, cols)
    dx = torch.from_numpy(x).cuda()
    nw = torch.from_numpy((1 + 0.1 * np.random.default_rng(seed).standard_normal(cols)).astype(np.float32)).cuda()
    ys = [torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(4)]
    st = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    up.matvec_dev(dx, ys[0], st)
    wr.matvec_dev(dx, ys[1], st)
    up.matvec_norm_dev(dx, dx, nw, 1e-6, ys[2], None, st)
    wr.matvec_norm_dev(dx, dx, nw, 1e-6, ys[3], None, st)
    torch.cuda.synchronize()
    y = [t.cpu().numpy() for t in ys]
    kind = up.kernel_kind
    wr.free()
    up.free()
    del buf
    ref = ref_gemv(oracle, raw, dtype, rows, cols, x)
    if kind == 3:
        assert normwise_err(y[1], ref) <= GEMV_TOL
    else:
        assert np.array_equal(y[0].view(np.uint32), y[1].view(np.uint32))
    assert np.array_equal(y[2].view(np.uint32), y[3].view(np.uint32))
    assert normwise_err(y[0], ref) <= GEMV_TOL


def test_config1_q4k_straddle(ctx, oracle, synth):
    """Q4_K 4864x896 (superblocks straddle row pairs)."""
    rows, cols, dtype = 4864, 896, 12
    raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(0))
    x = synth.gen_x(cols, synth.config_seed(0))
    y, kind = gpu_gemv(ctx, raw, dtype, rows, cols, x)
    ref = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
    assert kind in FAST and normwise_err(y, ref) <= GEMV_TOL
    b = oracle.fallback_cpu(raw, dtype, rows, cols, x)              # config 1 names this path
    assert np.array_equal(b, ref)


def test_lm_head_q6k(ctx, oracle, synth):
    rows, cols, dtype = 151936, 896, 14
    raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(1))
    x = synth.gen_x(cols, 1)
    y, _ = gpu_gemv(ctx, raw, dtype, rows, cols, x)
    ref = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x)
    assert normwise_err(y, ref) <= GEMV_TOL


@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096)])
def test_q4k_target_shapes(ctx, oracle, synth, shape):
    rows, cols = shape
    raw = synth.gen_blocks(12, rows, cols, synth.config_seed(4))
    x = synth.gen_x(cols, 4)
    y, kind = gpu_gemv(ctx, raw, 12, rows, cols, x)
    ref = oracle.mat_vec_mul_rows(raw, 12, rows, cols, x)
    assert kind in FAST and normwise_err(y, ref) <= GEMV_TOL


# The wave-private kernel: Q4_K rows of 12288 / 14336 columns with at least one
# 16-row workgroup per CU (workgroup b of G takes rows b + G i); 4100 rows leave
# 12 of the 257 x 16 row slots past the end (clamped loads, no stores), 8192 rows
# run two workgroups per CU.  Narrower or shorter matrices keep the ring /
# stream kernels.
WAVE_SHAPES = [((4096, 14336), 3), ((4096, 12288), 3), ((4100, 14336), 3), ((8192, 14336), 3),
               ((4000, 14336), 1), ((4096, 16384), 1)]


@pytest.mark.parametrize("shape,want", WAVE_SHAPES, ids=[f"{r}x{c}" for (r, c), _ in WAVE_SHAPES])
def test_wave_kernel(ctx, oracle, synth, shape, want):
    """Parity of the wave-private kernel against the oracle, under the
    adversarial x of tests/test_numerics_gpu.py too (one element per segment
    scaled 1e4), against the LDS-ring/stream result of the same bytes through
    qg_wrap_device, and bit-identical repetition."""
    import torch
    rows, cols = shape
    raw = synth.gen_blocks(12, rows, cols, synth.config_seed(4) + rows + cols)
    rng = np.random.default_rng(rows + cols)
    x = synth.gen_x(cols, 7)
    xo = x.copy()
    idx = np.arange(0, cols, 32) + rng.integers(0, 32, cols // 32)
    xo[idx] *= np.float32(1e4)
    m = ctx.upload(raw, 12, rows, cols)
    assert m.kernel_kind == want
    buf = torch.zeros(raw.nbytes + 1024, dtype=torch.uint8, device="cuda")
    buf[:raw.nbytes] = torch.from_numpy(raw.view(np.uint8).reshape(-1)).cuda()
    wr = ctx.wrap_device(buf, 12, rows, cols)
    for xv in (x, xo):
        ref = oracle.mat_vec_mul_rows(raw, 12, rows, cols, xv)
        ys = []
        for _ in range(3):
            y = np.full(rows, np.nan, np.float32)
            m.matvec_host(xv, y)
            ys.append(y)
        yw = np.full(rows, np.nan, np.float32)
        wr.matvec_host(xv, yw)
        err = normwise_err(ys[0], ref)
        print(f"Q4_K {rows}x{cols} kind={m.kernel_kind}: err vs oracle {err:.2e}, "
              f"vs wrapped {normwise_err(ys[0], yw):.2e}", flush=True)
        assert err <= GEMV_TOL
        assert normwise_err(yw, ref) <= GEMV_TOL
        assert all(np.array_equal(ys[0].view(np.uint32), y.view(np.uint32)) for y in ys[1:])
    wr.free()
    m.free()
    del buf


def test_full_size_linearity_and_determinism(ctx, synth):
    rows, cols = 4096, 14336
    raw = synth.gen_blocks(12, rows, cols, 77)
    m = ctx.upload(raw, 12, rows, cols)
    x1, x2 = synth.gen_x(cols, 1), synth.gen_x(cols, 2)
    ys = []
    for x in (x1, x2, np.float32(2.0) * x1 + x2, x1):
        y = np.zeros(rows, np.float32)
        m.matvec_host(x, y)
        ys.append(y)
    m.free()
    assert normwise_err(ys[2], 2.0 * ys[0] + ys[1]) <= 1e-5
    assert np.array_equal(ys[0].view(np.uint32), ys[3].view(np.uint32))   # same order every run


def test_many_batches_per_team(ctx, oracle, synth):
    """More than 64 batches per several-wave team: the partial sums are
    flushed in several chunks."""
    rows, cols, dtype = 100_000, 4160, 2
    raw = synth.gen_blocks(dtype, rows, cols, 4242)
    x = synth.gen_x(cols, 17)
    y, kind = gpu_gemv(ctx, raw, dtype, rows, cols, x)
    assert kind == 1
    assert normwise_err(y, oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x)) <= GEMV_TOL


def test_interleaved_launches_are_bit_identical(ctx, oracle, synth):
    """Matrices with several-wave teams and several batches per team launched
    in turn, again and again: every repetition gives the same bits (the
    partial-sum slots of one launch never leak into the next)."""
    cases = [(12, 70, 14336), (14, 300, 18944), (8, 129, 3584 * 2)]
    mats, xs, refs = [], [], []
    for i, (t, rows, cols) in enumerate(cases):
        raw = synth.gen_blocks(t, rows, cols, 900 + i)
        mats.append(ctx.upload(raw, t, rows, cols))
        xs.append(synth.gen_x(cols, 40 + i))
        refs.append(oracle.mat_vec_mul(raw, t, rows, cols, xs[-1]))
    assert [m.kernel_kind for m in mats] == [1, 2, 1]       # the Q6_K rows take the LDS ring kernel
    first = [None] * len(cases)
    for rep in range(4):
        for i, m in enumerate(mats):
            y = np.full(cases[i][1], np.nan, np.float32)
            m.matvec_host(xs[i], y)
            if first[i] is None:
                first[i] = y
                assert normwise_err(y, refs[i]) <= GEMV_TOL
            else:
                assert np.array_equal(y.view(np.uint32), first[i].view(np.uint32))
    for m in mats:
        m.free()


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("shape", [(896, 896), (3, 896), (3, 96), (5, 33), (1, 1), (2, 4864)])
def test_dequant_bit_exact(ctx, oracle, synth, dtype, shape):
    rows, cols = shape
    raw = synth.gen_blocks(dtype, rows, cols, rows + 31 * cols)
    m = ctx.upload(raw, dtype, rows, cols)
    out = np.full(rows * cols, np.nan, np.float32)
    m.dequant_host(out)
    m.free()
    ref = oracle.dequantize(raw, dtype, rows * cols)[: rows * cols]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kat", KAT, ids=[k["name"] for k in KAT])
def test_known_answer_blocks_gpu(ctx, kat):
    raw = np.frombuffer(bytes.fromhex(kat["raw"]), np.uint8).copy()
    t = kat["type"]
    n = len(kat["expected"])
    m = ctx.upload(raw, t, 1, n)
    out = np.zeros(n, np.float32)
    m.dequant_host(out)
    m.free()
    exp = np.array([np.nan if v is None else (np.inf if v == "inf" else (-np.inf if v == "-inf" else v))
                    for v in kat["expected"]], np.float32)
    nan = np.isnan(exp)
    assert np.all(out[nan].view(np.uint32) == 0x7FC00000)      # canonical NaN (quant.rs:328)
    assert np.array_equal(out[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f16_all_patterns_bit_exact(ctx, oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    raw = bits.view(np.uint8).copy()
    m = ctx.upload(raw, 1, 256, 256)
    out = np.zeros(65536, np.float32)
    m.dequant_host(out)
    m.free()
    ref = oracle.dequantize(raw, 1, 65536)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
def test_generic_kernel_for_ragged_cols(ctx, oracle, synth, dtype):
    """cols % 32 != 0: elements of one block fall in several rows at arbitrary
    offsets; the generic per-element kernel handles it."""
    for rows, cols in ((7, 33), (3, 100), (1, 1), (5, 257)):
        raw = synth.gen_blocks(dtype, rows, cols, rows * cols)
        x = synth.gen_x(cols, cols)
        y, kind = gpu_gemv(ctx, raw, dtype, rows, cols, x)
        assert kind == 0
        assert normwise_err(y, oracle.mat_vec_mul(raw, dtype, rows, cols, x)) <= GEMV_TOL


@pytest.mark.parametrize("dtype", [12, 14, 8])
def test_partial_last_block_and_group(ctx, oracle, synth, dtype):
    """rows not a multiple of the row group, rows*cols not a multiple of the block."""
    for rows, cols in ((3, 896), (3, 96), (5, 160), (1, 64)):
        raw = synth.gen_blocks(dtype, rows, cols, 5 * rows + cols)
        x = synth.gen_x(cols, 9)
        y, _ = gpu_gemv(ctx, raw, dtype, rows, cols, x)
        assert normwise_err(y, oracle.mat_vec_mul(raw, dtype, rows, cols, x)) <= GEMV_TOL


def test_zero_cols_gives_zeros_and_zero_rows_is_noop(ctx, rinf):
    raw = np.zeros(0, np.uint8)
    m = ctx.upload(raw, 12, 5, 0)
    y = np.full(5, 3.0, np.float32)
    m.matvec_host(np.zeros(0, np.float32), y)
    assert np.all(y == 0.0)                                         # out.fill(0.0), quant.rs:189
    m.free()
    m = ctx.upload(raw, 12, 0, 896)
    m.matvec_host(np.zeros(896, np.float32), np.zeros(0, np.float32))
    m.free()


def test_errors_are_status_codes(ctx, rinf, synth):
    raw = synth.gen_blocks(12, 2, 256, 1)
    with pytest.raises(rinf.QgemvError) as e:
        ctx.upload(raw[:-1], 12, 2, 256)
    assert e.value.status == 3                                      # QG_ERR_SHORT_DATA
    with pytest.raises(rinf.QgemvError) as e:
        ctx.upload(raw, 3, 2, 256)                                  # Q4_1
    assert e.value.status == 2
    lib = ctx.lib
    m = ctx.upload(raw, 12, 2, 256)
    assert lib.qg_dequantize_row_dev(ctx.h, m.h, 2, ctypes.c_void_p(16), None) == 7
    m.free()


def test_device_resident_path_matches_host_path(ctx, oracle, synth):
    import torch
    rows, cols = 896, 4864
    raw = synth.gen_blocks(14, rows, cols, 3)
    x = synth.gen_x(cols, 3)
    m = ctx.upload(raw, 14, rows, cols)
    y_host = np.zeros(rows, np.float32)
    m.matvec_host(x, y_host)
    dx = torch.from_numpy(x).cuda()
    dy = torch.zeros(rows, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    m.matvec_dev(dx, dy, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(dy.cpu().numpy().view(np.uint32), y_host.view(np.uint32))
    # x at a 4-byte (not 16-byte) offset takes the generic kernel, same result range
    buf = torch.zeros(cols + 1, dtype=torch.float32, device="cuda")
    buf[1:] = dx
    dy2 = torch.zeros(rows, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    m.matvec_dev(buf[1:], dy2, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert normwise_err(dy2.cpu().numpy(), oracle.mat_vec_mul(raw, 14, rows, cols, x)) <= GEMV_TOL
    m.free()


def test_gpu_context_drop_in_signature(rinf, oracle, synth):
    """GpuContext::mat_vec_mul(weight_data, dtype, x, out, rows, cols) and
    QuantizedMatrix::mat_vec_mul(x, out, Some(gpu))."""
    gpu = rinf.GpuContext.try_init()
    assert gpu is not None
    rows, cols = 128, 896
    raw = synth.gen_blocks(13, rows, cols, 8)
    x = synth.gen_x(cols, 8)
    qm = rinf.QuantizedMatrix(raw, 13, rows, cols)
    out1 = np.zeros(rows, np.float32)
    out2 = np.zeros(rows, np.float32)
    qm.mat_vec_mul(x, out1, gpu)
    qm.mat_vec_mul(x, out2, gpu)                                    # cached upload reused
    assert np.array_equal(out1, out2)
    assert normwise_err(out1, oracle.mat_vec_mul(raw, 13, rows, cols, x)) <= GEMV_TOL
    with pytest.raises(rinf.QgemvError):
        qm.mat_vec_mul(x[:-1], out1, gpu)
    gpu.close()


@pytest.mark.parametrize("dtype", TYPES, ids=[NAMES[t] for t in TYPES])
def test_dequantize_row_device_quirk(ctx, oracle, synth, dtype):
    import torch
    rows, cols = 6, 896
    raw = synth.gen_blocks(dtype, rows, cols, 41)
    m = ctx.upload(raw, dtype, rows, cols)
    for row in range(rows):
        d = torch.zeros(cols, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        m.dequantize_row_dev(row, d, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref = oracle.dequantize_row(raw, dtype, rows, cols, row, np.zeros(cols, np.float32))
        assert np.array_equal(d.cpu().numpy().view(np.uint32), ref.view(np.uint32)), row
    m.free()
