"""Pins the CPU oracle (oracle/qref.c) against checks that do not restate it:
exhaustive f16 conversion vs numpy, the K-quant scale pack's bit structure,
hand-encoded known-answer blocks with closed-form values, f64 brute force,
one-hot columns, linearity, and agreement of the reference's two CPU paths.
"""
from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest

KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "kat_blocks.json").read_text())
TYPES = [0, 1, 2, 6, 8, 12, 13, 14]


def kat_expected(e):
    out = []
    for v in e:
        out.append(np.nan if v is None else (np.inf if v == "inf" else (-np.inf if v == "-inf" else v)))
    return np.array(out, np.float32)


def test_fp16_exhaustive_matches_ieee(oracle):
    """quant.rs:302-342 vs numpy's IEEE half->single for all 65,536 patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_fp32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # every NaN input becomes the canonical quiet NaN f32::NAN
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)
    assert nan.sum() == 2046


def test_scale_min_k4_is_a_bit_permutation(oracle):
    """get_scale_min_k4 (quant.rs:606-615) maps the 96 bits of the 12-byte pack
    one-to-one onto the 16 six-bit fields: each single input bit sets exactly
    one output bit, and no two input bits land on the same output bit."""
    seen = set()
    for byte in range(12):
        for bit in range(8):
            s = np.zeros(12, np.uint8)
            s[byte] = 1 << bit
            hits = []
            for j in range(8):
                sc, m = oracle.get_scale_min_k4(j, s)
                for kind, v in (("sc", int(sc)), ("m", int(m))):
                    if v:
                        assert v & (v - 1) == 0
                        hits.append((kind, j, v.bit_length() - 1))
            assert len(hits) == 1, (byte, bit, hits)
            seen.add(hits[0])
    assert len(seen) == 96


def test_scale_min_k4_ggml_packing(oracle):
    """Known values: low-6-bit fields for j<4, nibble+2-bit splice for j>=4."""
    s = np.array([0xC1, 0x3F, 0x80, 0x07, 0x42, 0x00, 0xFF, 0x15, 0xA5, 0x0F, 0xF0, 0x3C], np.uint8)
    assert oracle.get_scale_min_k4(0, s) == (0x01, 0x02)
    assert oracle.get_scale_min_k4(1, s) == (0x3F, 0x00)
    assert oracle.get_scale_min_k4(3, s) == (0x07, 0x15)
    # j=4: sc = (s[8]&15) | (s[0]>>6)<<4 = 5 | 3<<4 ; m = (s[8]>>4) | (s[4]>>6)<<4 = 10 | 1<<4
    assert oracle.get_scale_min_k4(4, s) == (0x35, 0x1A)
    # j=7: sc = (s[11]&15) | (s[3]>>6)<<4 = 12 ; m = (s[11]>>4) | (s[7]>>6)<<4 = 3
    assert oracle.get_scale_min_k4(7, s) == (12, 3)


@pytest.mark.parametrize("kat", KAT, ids=[k["name"] for k in KAT])
def test_known_answer_blocks(oracle, kat):
    raw = np.frombuffer(bytes.fromhex(kat["raw"]), np.uint8).copy()
    exp = kat_expected(kat["expected"])
    t = kat["type"]
    if t == 1:
        got = np.array([oracle.dequantize_block(raw, t, i)[0] for i in range(exp.size)], np.float32)
    else:
        got = oracle.dequantize_block(raw, t, 0)[: exp.size]
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(exp[~nan]))


@pytest.mark.parametrize("dtype", TYPES)
def test_dequantize_matches_block_decode(oracle, synth, dtype):
    rows, cols = 3, 96
    raw = synth.gen_blocks(dtype, rows, cols, 11)
    v = oracle.dequantize(raw, dtype, rows * cols)
    bs = {0: 1, 1: 1, 2: 32, 6: 32, 8: 32, 12: 256, 13: 256, 14: 256}[dtype]
    nblk = -(-(rows * cols) // bs)
    blocks = np.concatenate([oracle.dequantize_block(raw, dtype, b).copy()[:bs] for b in range(nblk)])
    # Q4_K / Q5_K keep whole blocks in the Vec (quant.rs:640-666, 714-749)
    assert v.size == (nblk * bs if dtype in (12, 13) else rows * cols)
    assert np.array_equal(v.view(np.uint32), blocks[: v.size].view(np.uint32))


def test_dequantize_short_data_is_err(oracle, synth):
    raw = synth.gen_blocks(12, 2, 256, 1)
    assert oracle.dequantize(raw[:-1], 12, 512) is None
    assert oracle.dequantize(raw, 3, 512) is None        # Q4_1 unsupported (quant.rs:370)


def brute_f64(oracle, raw, dtype, rows, cols, x):
    w = oracle.dequantize(raw, dtype, rows * cols)[: rows * cols].astype(np.float64)
    return w.reshape(rows, cols) @ x.astype(np.float64)


@pytest.mark.parametrize("dtype", TYPES)
@pytest.mark.parametrize("shape", [(5, 64), (7, 96), (3, 896), (4, 256), (2, 33)])
def test_gemv_vs_f64_bruteforce(oracle, synth, dtype, shape):
    rows, cols = shape
    raw = synth.gen_blocks(dtype, rows, cols, rows * 1000 + cols)
    x = synth.gen_x(cols, cols)
    y = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
    ref = brute_f64(oracle, raw, dtype, rows, cols, x)
    w = oracle.dequantize(raw, dtype, rows * cols)[: rows * cols].reshape(rows, cols).astype(np.float64)
    # sequential f32 summation bound: |err| <= n*eps*sum|w*x|
    bound = cols * 2.0 ** -23 * (np.abs(w) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y - ref) <= bound)


@pytest.mark.parametrize("dtype", TYPES)
def test_one_hot_column_is_exact(oracle, synth, dtype):
    """x = e_c returns column c of the dequantized matrix exactly."""
    rows, cols = 6, 896
    raw = synth.gen_blocks(dtype, rows, cols, 7)
    w = oracle.dequantize(raw, dtype, rows * cols)[: rows * cols].reshape(rows, cols)
    for c in (0, 1, 255, 256, 511, 895):
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        y = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
        assert np.array_equal(y, w[:, c])


@pytest.mark.parametrize("dtype", TYPES)
def test_two_cpu_paths_bit_identical(oracle, synth, dtype):
    """quant.rs:188-205 (--cpu) and gpu_backend.rs:556-567 (fallback_cpu)
    sum in the same order, so they agree bit for bit."""
    for rows, cols in ((4864 // 16, 896), (128, 896), (16, 4864 // 4)):
        raw = synth.gen_blocks(dtype, rows, cols, rows + cols)
        x = synth.gen_x(cols, 3)
        a = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
        b = oracle.fallback_cpu(raw, dtype, rows, cols, x)
        assert b is not None
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fallback_cpu_panics_on_partial_kquant_block(oracle, synth):
    """Q4_K with rows*cols % 256 != 0: dequantize returns whole blocks, so the
    length assert of math.rs:198 fires; the --cpu loop still works."""
    raw = synth.gen_blocks(12, 3, 96, 5)
    x = synth.gen_x(96, 5)
    assert oracle.fallback_cpu(raw, 12, 3, 96, x) is None
    assert np.all(np.isfinite(oracle.mat_vec_mul(raw, 12, 3, 96, x)))


@pytest.mark.parametrize("dtype", TYPES)
def test_row_ordered_loop_bit_identical(oracle, synth, dtype):
    for rows, cols in ((37, 896), (9, 4864), (5, 96)):
        raw = synth.gen_blocks(dtype, rows, cols, 99)
        x = synth.gen_x(cols, 4)
        a = oracle.mat_vec_mul(raw, dtype, rows, cols, x)
        b = oracle.mat_vec_mul_rows(raw, dtype, rows, cols, x)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_linearity(oracle, synth):
    rows, cols = 64, 896
    raw = synth.gen_blocks(14, rows, cols, 3)
    x1, x2 = synth.gen_x(cols, 1), synth.gen_x(cols, 2)
    y = oracle.mat_vec_mul(raw, 14, rows, cols, np.float32(2.0) * x1 + x2)
    z = 2.0 * oracle.mat_vec_mul(raw, 14, rows, cols, x1) + oracle.mat_vec_mul(raw, 14, rows, cols, x2)
    assert np.max(np.abs(y - z)) <= 1e-5 * np.max(np.abs(z))


def test_dequantize_row_straddle_quirk(oracle, synth):
    """quant.rs:152-174 at cols=896, Q4_K, row 1: the row starts half-way into
    block 3 (offset 128).  Block 3's tail lands at [0,128); blocks 4..6 are
    written at bi*256+k, i.e. buf[256+k] = block(3+bi)[k] for k < 256 and
    dst < 896; buf[128..256) keeps its prior contents."""
    rows, cols = 2, 896
    raw = synth.gen_blocks(12, rows, cols, 21)
    w = oracle.dequantize(raw, 12, rows * cols).reshape(-1)
    buf = np.full(cols, -7.0, np.float32)
    oracle.dequantize_row(raw, 12, rows, cols, 1, buf)
    true_row = w[896:1792]
    assert np.array_equal(buf[:128], true_row[:128])
    assert np.all(buf[128:256] == -7.0)
    blocks = w.reshape(-1, 256)               # 7 blocks
    for bi in (1, 2, 3):
        lim = min(256, cols + 128 - bi * 256)
        for k in range(lim):
            dst = bi * 256 + k
            if dst < cols:
                assert buf[dst] == blocks[3 + bi][k]
    wrong = np.sum(buf != true_row)
    assert wrong >= 640          # most of the row is displaced, as the quirk implies
    # row 0 (block-aligned) is correct
    buf0 = np.zeros(cols, np.float32)
    oracle.dequantize_row(raw, 12, rows, cols, 0, buf0)
    assert np.array_equal(buf0, w[:896])


def test_rmsnorm_softmax_silu_argmax(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(896).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(896)).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-6)
    r = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(y - r)) < 1e-5
    a = rng.standard_normal(300).astype(np.float32) * 5
    s = a.copy()
    oracle.softmax_inplace(s)
    e = np.exp(a.astype(np.float64) - a.max())
    assert np.max(np.abs(s - e / e.sum())) < 1e-6
    for v in (-30.0, -1.5, 0.0, 0.7, 12.0):
        assert abs(oracle.silu(v) - v / (1 + np.exp(-v))) < 1e-6 * max(1, abs(v))
    b = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert oracle.argmax(b) == 1                       # first maximum wins


def test_rope_rotates_pairs(oracle):
    dim, base, P = 64, 1e6, 40
    c, s = oracle.rope_tables(dim, base, P)
    x = np.random.default_rng(1).standard_normal(dim).astype(np.float32)
    for pos in (0, 1, 39, 45):
        y = x.copy()
        oracle.rope_apply(y, pos, c, s, P)
        b = base if pos < P else 10000.0                 # rope.rs:71-86 fallback base
        th = 1.0 / b ** (np.arange(0, dim, 2) / dim)
        ang = pos * th
        ref = np.empty(dim)
        ref[0::2] = x[0::2] * np.cos(ang) - x[1::2] * np.sin(ang)
        ref[1::2] = x[0::2] * np.sin(ang) + x[1::2] * np.cos(ang)
        assert np.max(np.abs(y - ref)) < 2e-4 * max(1, pos / 8)
        # rotation preserves each pair's norm
        assert np.allclose(np.hypot(y[0::2], y[1::2]), np.hypot(x[0::2], x[1::2]), rtol=1e-5)


def test_repetition_penalty(oracle):
    lg = np.array([2.0, -2.0, 1.0, 0.0], np.float32)
    oracle.repetition_penalty(lg, [0, 1, 0], 1.1, 64)
    assert np.isclose(lg[0], 2.0 / 1.1 / 1.1) and np.isclose(lg[1], -2.2)
    assert lg[2] == 1.0
    lg = np.ones(4, np.float32)
    oracle.repetition_penalty(lg, [3] + [0] * 64, 1.1, 64)   # token 3 is outside the window
    assert lg[3] == 1.0
