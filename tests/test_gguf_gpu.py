"""qg_model_load_gguf (include/qggguf.h, Model::load src/model.rs:136-329) on
files of the synthetic writer: the loaded engine gives the same logits, bit
for bit, as one built slot by slot from the same tensors, and follows the
oracle step by step; the tied lm_head, non-F32 norms (zeros, model.rs:211-216),
missing biases (zeros) and a missing tensor behave as the reference's loader."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

from test_decode_gpu import LOGIT_TOL, SMALL, build, run_and_compare

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gw(rinf):
    return importlib.import_module(rinf.__name__ + ".gguf_writer")


def steps(dev, toks, vocab):
    out = []
    for p, t in enumerate(toks):
        lg = np.zeros(vocab, np.float32)
        dev.forward(int(t), p, lg)
        out.append(lg)
    return out


@pytest.mark.parametrize("name,cfg,mix", [
    ("small", SMALL, "q4_k_m"),
    ("tied896", dict(SMALL, embed_dim=896, n_heads=14, n_kv_heads=2, hidden_dim=1024, vocab_size=700,
                     tied=True), "q4_k_m"),
    ("nobias", dict(SMALL, bias=False), "q8_0"),
])
def test_loaded_model_matches(rinf, synth, oracle, ctx, gw, tmp_path, name, cfg, mix):
    p = tmp_path / f"{name}.gguf"
    gw.write_model(p, synth, cfg, mix, 41, context_length=64)
    dev = rinf.DeviceModel.load_gguf(ctx, p, 32)
    assert dev.cfg.max_seq_len == 32 and dev.cfg.vocab_size == cfg["vocab_size"]
    man, ref, shared = build(rinf, synth, oracle, ctx, cfg, mix, 41, 32)
    toks = np.random.default_rng(3).integers(0, cfg["vocab_size"], 10)
    a, b = steps(dev, toks, cfg["vocab_size"]), steps(man, toks, cfg["vocab_size"])
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    dev.reset()
    out, errs = run_and_compare(dev, ref, oracle, cfg, toks[:5], 6)
    print(f"{name}: max logits err {max(errs):.2e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    dev.close()
    man.close()
    if shared is not None:
        shared.free()


def test_non_f32_norm_loads_as_zeros(rinf, synth, ctx, gw, tmp_path):
    cfg = dict(SMALL, n_layers=1)
    tensors, t = gw.model_tensors(synth, cfg, "q8_0", 43)
    f16 = []
    for n, dims, ty, raw in tensors:
        if n == "blk.0.ffn_norm.weight":
            raw, ty = raw.astype(np.float16), 1
        f16.append((n, dims, ty, raw))
    p = tmp_path / "f16norm.gguf"
    gw.write_gguf(p, gw.model_metadata(cfg, context_length=16), f16)
    dev = rinf.DeviceModel.load_gguf(ctx, p)
    t["vecs"][("ffn_norm", 0)] = np.zeros(cfg["embed_dim"], np.float32)
    man = rinf.DeviceModel(ctx, cfg["embed_dim"], 1, cfg["n_heads"], cfg["n_kv_heads"], cfg["hidden_dim"],
                           cfg["vocab_size"], 16, cfg["rope_base"], cfg["norm_eps"])
    slots = {"token_embd": rinf.M_TOKEN_EMBD, "lm_head": rinf.M_LM_HEAD, "wq": rinf.M_WQ, "wk": rinf.M_WK,
             "wv": rinf.M_WV, "wo": rinf.M_WO, "gate": rinf.M_GATE, "up": rinf.M_UP, "down": rinf.M_DOWN}
    vslots = {"final_norm": rinf.V_FINAL_NORM, "attn_norm": rinf.V_ATTN_NORM, "ffn_norm": rinf.V_FFN_NORM,
              "bq": rinf.V_BQ, "bk": rinf.V_BK, "bv": rinf.V_BV}
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        man.set_matrix(slots[slot], layer, raw, dtype, rows, cols)
    for (nm, layer), v in t["vecs"].items():
        man.set_vector(vslots[nm], layer, v)
    toks = [3, 9, 27]
    for x, y in zip(steps(dev, toks, cfg["vocab_size"]), steps(man, toks, cfg["vocab_size"])):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    dev.close()
    man.close()


def test_missing_tensor_is_an_error(rinf, synth, ctx, gw, tmp_path):
    cfg = dict(SMALL, n_layers=1)
    tensors, _ = gw.model_tensors(synth, cfg, "q8_0", 44)
    tensors = [x for x in tensors if x[0] != "blk.0.ffn_up.weight"]
    p = tmp_path / "missing.gguf"
    gw.write_gguf(p, gw.model_metadata(cfg, context_length=16), tensors)
    with pytest.raises(rinf.QgemvError) as e:
        rinf.DeviceModel.load_gguf(ctx, p)
    assert e.value.status == 7
    assert "blk.0.ffn_up.weight" in str(e.value)


def test_wrapped_dims_return_a_status(rinf, synth, ctx, gw, tmp_path):
    """A norm whose dims multiply past 2^64 -- wrapping to a 32 MiB byte count
    that lies inside the file -- is refused with QG_ERR_SHAPE: no attempt to
    build a vector of ne0 = 2^40 + 1 floats, no exception out of the C ABI."""
    cfg = dict(SMALL, n_layers=1)
    tensors, _ = gw.model_tensors(synth, cfg, "q8_0", 45)
    bad = []
    for n, dims, ty, raw in tensors:
        if n == "blk.0.ffn_norm.weight":
            n, dims, ty, raw = n, [(1 << 40) + 1, 1 << 24], 1, np.zeros(1 << 24, np.float16)
        bad.append((n, dims, ty, raw))
    p = tmp_path / "wrapped.gguf"
    gw.write_gguf(p, gw.model_metadata(cfg, context_length=16), bad)
    with pytest.raises(rinf.QgemvError) as e:
        rinf.DeviceModel.load_gguf(ctx, p)
    assert e.value.status == 7
    assert "ffn_norm" in str(e.value)
