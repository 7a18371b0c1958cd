"""Pins oracle/qref_model.c (the restatement of Transformer::forward,
src/transformer.rs:63-98) without the GPU:

* against an independent float64 numpy forward pass written from the
  reference's definitions (attention.rs:54-124 with GQA head mapping
  h // n_rep, rope.rs:42-96 pairs (2i, 2i+1) per head, kv_cache.rs:52-73,
  mlp.rs:31-46, rmsnorm math.rs:237-257, silu math.rs:137-146, residuals of
  transformer.rs:20-48), on matrices decoded by the already pinned
  qref_dequantize / qref_dequantize_row;
* against closed forms: with wo and down zero the hidden state stays the
  embedding row, so the logits are lm_head · (rmsnorm(embedding) * final_norm);
  at position 0 attention returns v, so with down zero the final hidden state
  is embedding + wo · (wv · xn + bv).

A wrong head index, RoPE pairing, residual wiring, norm or cache order makes
the multi-step comparison fail by orders of magnitude more than the f32 vs
f64 rounding it allows (1e-3 normwise).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import normwise_err

CFG = dict(embed_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=512, vocab_size=300,
           rope_base=1e4, norm_eps=1e-6, tied=False, bias=True)


def dense(oracle, mats, slot, layer):
    raw, dtype, rows, cols = mats[(slot, layer)]
    return oracle.dequantize(raw, dtype, rows * cols)[: rows * cols].astype(np.float64).reshape(rows, cols)


def rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def silu(x):
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


def rope(x, pos, hd, base):
    out = x.copy()
    for h in range(x.size // hd):
        for i in range(hd // 2):
            a = pos / base ** (2 * i / hd)
            x0, x1 = x[h * hd + 2 * i], x[h * hd + 2 * i + 1]
            out[h * hd + 2 * i] = x0 * np.cos(a) - x1 * np.sin(a)
            out[h * hd + 2 * i + 1] = x0 * np.sin(a) + x1 * np.cos(a)
    return out


class NumpyModel:
    """float64 forward pass from the reference's definitions."""

    def __init__(self, oracle, cfg, t):
        self.c = cfg
        m, v = t["mats"], t["vecs"]
        L = cfg["n_layers"]
        self.emb = m[("token_embd", 0)]
        self.oracle = oracle
        self.W = {s: [dense(oracle, m, s, l) for l in range(L)]
                  for s in ("wq", "wk", "wv", "wo", "gate", "up", "down")}
        self.lm = dense(oracle, m, "lm_head", 0)
        E = cfg["embed_dim"]
        kv = cfg["n_kv_heads"] * (E // cfg["n_heads"])
        z = lambda n: np.zeros(n)
        self.V = {k: [np.asarray(v.get((k, l), z(n)), np.float64) for l in range(L)]
                  for k, n in (("attn_norm", E), ("ffn_norm", E), ("bq", E), ("bk", kv), ("bv", kv))}
        self.fn = np.asarray(v[("final_norm", 0)], np.float64)
        self.kc = [[] for _ in range(L)]
        self.vc = [[] for _ in range(L)]

    def embed(self, tok):
        raw, dtype, rows, cols = self.emb
        return self.oracle.dequantize_row(raw, dtype, rows, cols, tok).astype(np.float64)

    def forward(self, tok, pos):
        c = self.c
        E, H, KV = c["embed_dim"], c["n_heads"], c["n_kv_heads"]
        hd, eps = E // H, c["norm_eps"]
        n_rep = H // KV
        x = self.embed(tok)
        for l in range(c["n_layers"]):
            xn = rms(x, self.V["attn_norm"][l], eps)
            q = rope(self.W["wq"][l] @ xn + self.V["bq"][l], pos, hd, c["rope_base"])
            k = rope(self.W["wk"][l] @ xn + self.V["bk"][l], pos, hd, c["rope_base"])
            v = self.W["wv"][l] @ xn + self.V["bv"][l]
            self.kc[l].append(k)
            self.vc[l].append(v)
            K, Vv = np.array(self.kc[l]), np.array(self.vc[l])
            ao = np.zeros(E)
            for h in range(H):
                g = h // n_rep
                s = K[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                ao[h * hd:(h + 1) * hd] = p @ Vv[:, g * hd:(g + 1) * hd]
            x = x + self.W["wo"][l] @ ao
            xn2 = rms(x, self.V["ffn_norm"][l], eps)
            x = x + self.W["down"][l] @ (silu(self.W["gate"][l] @ xn2) * (self.W["up"][l] @ xn2))
        return self.lm @ rms(x, self.fn, eps)


def oracle_model(oracle, cfg, t, max_seq=16):
    ref = oracle.Model(dict(cfg, max_seq_len=max_seq))
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        ref.set_mat(slot, layer, raw, dtype, rows, cols)
    for (name, layer), v in t["vecs"].items():
        ref.set_vec(name, layer, v)
    return ref


@pytest.mark.parametrize("mix", ["q8_0", "q4_k_m"])
def test_oracle_forward_matches_numpy_f64(oracle, synth, mix):
    t = synth.gen_model(CFG, mix, 31)
    ref = oracle_model(oracle, CFG, t)
    npm = NumpyModel(oracle, CFG, t)
    toks = np.random.default_rng(3).integers(0, CFG["vocab_size"], 6)
    for pos, tok in enumerate(toks):
        a = ref.forward(int(tok), pos)
        b = npm.forward(int(tok), pos)
        err = normwise_err(a, b)
        assert err <= 1e-3, f"{mix} pos {pos}: {err:.2e}"


def zero_f32(rows, cols):
    return np.zeros(rows * cols, np.float32).view(np.uint8), 0, rows, cols


def test_oracle_closed_form_without_wo_and_down(oracle, synth):
    t = synth.gen_model(CFG, "q8_0", 32)
    E, Hd = CFG["embed_dim"], CFG["hidden_dim"]
    for l in range(CFG["n_layers"]):
        t["mats"][("wo", l)] = zero_f32(E, E)
        t["mats"][("down", l)] = zero_f32(E, Hd)
    ref = oracle_model(oracle, CFG, t)
    raw, dtype, rows, cols = t["mats"][("token_embd", 0)]
    lm = dense(oracle, t["mats"], "lm_head", 0)
    fn = t["vecs"][("final_norm", 0)].astype(np.float64)
    for pos, tok in enumerate([5, 17, 5, 299]):
        e = oracle.dequantize_row(raw, dtype, rows, cols, tok).astype(np.float64)
        want = lm @ rms(e, fn, CFG["norm_eps"])
        assert normwise_err(ref.forward(tok, pos), want) <= 1e-5


def test_oracle_first_position_attention_is_v(oracle, synth):
    cfg = dict(CFG, n_layers=1)
    t = synth.gen_model(cfg, "q8_0", 33)
    E, Hd = cfg["embed_dim"], cfg["hidden_dim"]
    t["mats"][("down", 0)] = zero_f32(E, Hd)
    ref = oracle_model(oracle, cfg, t)
    m, v = t["mats"], t["vecs"]
    raw, dtype, rows, cols = m[("token_embd", 0)]
    e = oracle.dequantize_row(raw, dtype, rows, cols, 42).astype(np.float64)
    xn = rms(e, v[("attn_norm", 0)].astype(np.float64), cfg["norm_eps"])
    vv = dense(oracle, m, "wv", 0) @ xn + v[("bv", 0)]
    n_rep = cfg["n_heads"] // cfg["n_kv_heads"]
    hd = E // cfg["n_heads"]
    ao = np.concatenate([vv[(h // n_rep) * hd:(h // n_rep + 1) * hd] for h in range(cfg["n_heads"])])
    hid = e + dense(oracle, m, "wo", 0) @ ao
    want = dense(oracle, m, "lm_head", 0) @ rms(hid, v[("final_norm", 0)].astype(np.float64), cfg["norm_eps"])
    assert normwise_err(ref.forward(42, 0), want) <= 1e-5
