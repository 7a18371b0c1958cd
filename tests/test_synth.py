"""Pins the synthetic model weights (synth.gen_weights) on the CPU: the
dequantized values (through the oracle's dequantize, bit-exact with
quant.rs:356-840) are centred with standard deviation near 1/sqrt(cols) for
every type, the 6-bit scale pack inverts get_scale_min_k4 (quant.rs:606-615),
and a whole random-init model keeps its activations O(1) over many layers
(the property the long decode parity runs rely on)."""
from __future__ import annotations

import numpy as np
import pytest

TYPES = [0, 1, 2, 6, 8, 12, 13, 14]


@pytest.mark.parametrize("dtype", TYPES)
@pytest.mark.parametrize("cols", [896, 4096, 18944])
def test_weights_centred_and_scaled(oracle, synth, dtype, cols):
    rows = 64
    raw = synth.gen_weights(dtype, rows, cols, 1234 + cols + dtype)
    w = oracle.dequantize(raw, dtype, rows * cols)[: rows * cols].astype(np.float64)
    assert np.all(np.isfinite(w))
    sd = w.std()
    target = 1.0 / np.sqrt(cols)
    assert 0.6 * target < sd < 1.6 * target, (sd, target)
    # the mean of 64 * cols weights of sd ~ target: a few target / sqrt(n) at most
    assert abs(w.mean()) < 8 * target / np.sqrt(w.size) + 0.02 * target, (w.mean(), target)


def test_k_scale_pack_inverts_get_scale_min_k4(oracle, synth):
    rng = np.random.default_rng(5)
    sc = rng.integers(0, 64, size=(200, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(200, 8), dtype=np.uint8)
    packed = synth._pack_k_scales(sc, mn)
    for b in range(200):
        for j in range(8):
            assert oracle.get_scale_min_k4(j, packed[b]) == (sc[b, j], mn[b, j])


def test_random_init_model_stays_bounded(oracle, synth):
    """24 layers of the Qwen2-0.5B layer shape (vocabulary cut to 512):
    the residual stream stays O(1) per layer and attention is not one-hot."""
    import test_oracle_model as tom
    cfg = dict(synth.ARCH["qwen2-0.5b"], vocab_size=512)
    t = synth.gen_model(cfg, "q4_k_m", 77)
    t["mats"][("lm_head", 0)] = t["mats"][("token_embd", 0)]
    npm = tom.NumpyModel(oracle, cfg, t)
    logits = None
    for pos, tok in enumerate([3, 141, 59, 265, 358, 97]):
        logits = npm.forward(tok, pos)
    assert np.all(np.isfinite(logits))
    assert np.max(np.abs(logits)) < 1e3
