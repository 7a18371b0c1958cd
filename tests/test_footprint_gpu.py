"""Device memory of a decode-step model (qg_model_resident_bytes,
include/qgmodel.h): every uploaded Q8_0/Q4_K/Q5_K/Q6_K matrix is held once,
in the repacked layout; the layer parts the model owns are views into the
stacked [Q;K;V] / [gate; up] matrices of the decode step; token_embd is held
in the GGUF layout.  So the weights resident on the device are the file's
quantized bytes plus one 512-byte tail pad per matrix.  Also: the stacked
views hand their bytes back when a part is replaced, and the model then
still follows the oracle; a whole-matrix dequant and a dequantize_row of a
repacked-only matrix equal those of its GGUF bytes."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import normwise_err
from test_decode_gpu import DEEP_TOL, SMALL, build, run_and_compare

pytestmark = pytest.mark.gpu

PAD = 512


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k", "q8_0"])
def test_weights_held_once(rinf, synth, oracle, ctx, mix):
    """Two layers of the Qwen2-7B shape (3584 columns, [Q;K] + V or [Q;K;V]
    stacks, [gate; up]), a 2048-token vocabulary: resident weight bytes <=
    the slots' file bytes + one tail pad per matrix, after the first forward
    pass has built the stacks; the tokens still follow the oracle."""
    cfg = dict(SMALL, n_layers=2, embed_dim=3584, n_heads=28, n_kv_heads=4, hidden_dim=1024, vocab_size=2048)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, mix, 71, 32)
    prompt = np.random.default_rng(71).integers(0, cfg["vocab_size"], 6)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 4)
    rb = dev.resident_bytes()
    n_mats = 2 + 7 * cfg["n_layers"] + 2 * cfg["n_layers"]          # slots + the stacks
    print(f"{mix}: weights {rb['weights']} B, file {rb['file_bytes']} B "
          f"({rb['weights'] / rb['file_bytes']:.4f}x), total {rb['total']} B", flush=True)
    assert rb["weights"] <= rb["file_bytes"] + n_mats * PAD
    assert rb["total"] > rb["weights"]
    assert max(errs) <= DEEP_TOL
    dev.close()


def test_replace_a_stacked_part(rinf, synth, oracle, ctx):
    """After the stacks exist, replace layer 0's wq and layer 1's up (views
    into them): the stacks are rebuilt from the parts' own copies and the
    logits follow the oracle with the new weights."""
    cfg = dict(SMALL, n_layers=2)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", 73, 40)
    prompt = np.random.default_rng(73).integers(0, cfg["vocab_size"], 5)
    run_and_compare(dev, ref, oracle, cfg, prompt, 3)
    t = synth.gen_model(cfg, "q4_k_m", 74)
    for slot, which, layer in (("wq", rinf.M_WQ, 0), ("up", rinf.M_UP, 1)):
        raw, dtype, rows, cols = t["mats"][(slot, layer)]
        dev.set_matrix(which, layer, raw, dtype, rows, cols)
        ref.set_mat(slot, layer, raw, dtype, rows, cols)
    dev.reset()
    ref.reset()
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 6)
    assert max(errs) <= DEEP_TOL
    rb = dev.resident_bytes()
    assert rb["weights"] <= rb["file_bytes"] + (2 + 9 * cfg["n_layers"]) * PAD
    dev.close()


@pytest.mark.parametrize("dtype, cols", [(8, 896), (12, 896), (13, 3584), (14, 4864)],
                         ids=["q8_0", "q4_k-straddle", "q5_k", "q6_k"])
def test_dequant_of_repacked_only_matrix(rinf, synth, oracle, ctx, dtype, cols):
    """An uploaded matrix keeps only its repacked copy: qg_dequant and
    qg_dequantize_row rebuild the GGUF layout (the inverse of the repack) and
    give the oracle's dequantized values bit for bit."""
    import torch
    rows = 64
    raw = synth.gen_blocks(dtype, rows, cols, 5)
    m = ctx.upload(raw, dtype, rows, cols)
    full = np.zeros(rows * cols, np.float32)
    m.dequant_host(full)
    want = oracle.dequantize(raw, dtype, rows * cols)
    assert np.array_equal(full.view(np.uint32), want.view(np.uint32))
    d = torch.zeros(cols, dtype=torch.float32, device="cuda")
    for r in (0, 1, 37, rows - 1):
        # zeros first: rows that straddle blocks leave positions unwritten
        # (quant.rs:152-174), as in the oracle's fresh buffer
        d.zero_()
        m.dequantize_row_dev(r, d)
        ctx.synchronize()
        got = d.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), oracle.dequantize_row(raw, dtype, rows, cols, r).view(np.uint32))
    m.free()


def test_failed_restore_keeps_the_stack(rinf, synth, oracle, ctx):
    """Replacing a part re-copies every view part out of its stack first.
    When one of those copies cannot be allocated (injected failures, every
    allocation index in turn), set_matrix reports out-of-memory and the
    stack whose parts could not all be restored stays alive: the model keeps
    following the oracle (the replacement has the same bytes, so the oracle
    holds either way)."""
    cfg = dict(SMALL, n_layers=2)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", 75, 40)
    prompt = np.random.default_rng(75).integers(0, cfg["vocab_size"], 4)
    run_and_compare(dev, ref, oracle, cfg, prompt, 2)            # builds the stacks and views
    t = synth.gen_model(cfg, "q4_k_m", 75)
    raw, dtype, rows, cols = t["mats"][("up", 1)]
    restore_failures = 0
    for skip in range(16):
        ctx.fail_allocations(1, skip)
        try:
            dev.set_matrix(rinf.M_UP, 1, raw, dtype, rows, cols)
        except rinf.QgemvError as e:
            assert e.status == 6, e
            restore_failures += "matrix copy" in str(e)
        finally:
            ctx.fail_allocations(0)
        dev.reset()
        ref.reset()
        out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 2)
        assert max(errs) <= DEEP_TOL, (skip, max(errs))
    assert restore_failures > 0
    dev.close()
