"""GPU parity of the batched prefill (qg_model_prefill, include/qgmodel.h):
the prompt's tokens through each layer together, every projection a GEMM on
the matrix cores (x as two f16 pieces under a power-of-two scale per
256-element group, the K-quant weights as integer f16 operands held exactly,
f32 accumulation).  Checked against the oracle's token-by-token
forward pass (oracle/qref_model.c, transformer.rs:63-98 as model.rs:361-365
calls it): the last prompt token's logits, then greedy decode steps on the
caches the prefill wrote (every cached position's K/V enters those steps),
within DEEP_TOL, identical tokens.  Also: chunks of 64 tokens, a prefill that
continues a cache, the token-by-token fallback for a mix without an MFMA
path (F16), generate with the batched prefill, and layer matrices wrapped
in the GGUF layout (qg_wrap_device) so that the GEMM's GGUF-layout loaders
run: rows straddling superblocks (cols = 896) and whole-block rows."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import normwise_err
from test_decode_gpu import DEEP_TOL, SMALL, build

pytestmark = pytest.mark.gpu


def decode_compare(dev, ref, oracle, cfg, ids, ref_l, n_new, pos):
    """n_new greedy steps on both sides after a prompt: logits errors, tokens."""
    V = cfg["vocab_size"]
    logits = np.zeros(V, np.float32)
    errs, out = [], []
    for _ in range(n_new):
        recent = ids[-64:]
        rl = ref_l.copy()
        oracle.repetition_penalty(rl, recent, 1.1, 64)
        t_ref = oracle.argmax(rl)
        t_dev = dev.sample_greedy(recent, 1.1, 64)
        assert t_dev == t_ref
        out.append(t_ref)
        dev.forward(t_ref, pos, logits)
        ref_l = ref.forward(t_ref, pos)
        errs.append(normwise_err(logits, ref_l))
        ids.append(t_ref)
        pos += 1
    return errs, out


def prefill_and_compare(rinf, synth, oracle, ctx, cfg, mix, seed, n_prompt, n_new, max_seq, split=None):
    dev, ref, shared = build(rinf, synth, oracle, ctx, cfg, mix, seed, max_seq)
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab_size"], n_prompt)
    logits = np.zeros(cfg["vocab_size"], np.float32)
    parts = [prompt] if split is None else [prompt[:split], prompt[split:]]
    for p in parts:
        dev.prefill(p, logits)
    ref_l = None
    for pos, tok in enumerate(prompt):
        ref_l = ref.forward(int(tok), pos)
    assert dev.seq_len == n_prompt
    e0 = normwise_err(logits, ref_l)
    errs, out = decode_compare(dev, ref, oracle, cfg, [int(t) for t in prompt], ref_l, n_new, n_prompt)
    dev.close()
    if shared is not None:
        shared.free()
    return e0, errs, out


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k", "q8_0", "q5_k_m"])
def test_small_model_prefill(rinf, synth, oracle, ctx, mix):
    e0, errs, out = prefill_and_compare(rinf, synth, oracle, ctx, SMALL, mix, 41, 20, 10, 64)
    print(f"{mix}: prefill logits err {e0:.2e}, decode max {max(errs):.2e}, tokens {out}", flush=True)
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL


def test_prefill_chunks_and_continuation(rinf, synth, oracle, ctx):
    """150 prompt tokens (chunks of 64, 64, 22), fed as 37 + 113 (the second
    call continues the caches at position 37)."""
    cfg = dict(SMALL, n_layers=2)
    e0, errs, out = prefill_and_compare(rinf, synth, oracle, ctx, cfg, "q4_k_m", 43, 150, 6, 200, split=37)
    print(f"chunks: prefill logits err {e0:.2e}, decode max {max(errs):.2e}", flush=True)
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k_m"])
def test_qwen2_7b_layer_shape_prefill(rinf, synth, oracle, ctx, mix):
    """One layer of the Qwen2-7B shape (head_dim 128, 7 query heads per kv
    head, 3584 columns), 40-token prompt."""
    cfg = dict(SMALL, n_layers=1, embed_dim=3584, n_heads=28, n_kv_heads=4, hidden_dim=1024)
    e0, errs, out = prefill_and_compare(rinf, synth, oracle, ctx, cfg, mix, 47, 40, 6, 64)
    print(f"7b layer {mix}: prefill logits err {e0:.2e}, decode max {max(errs):.2e}", flush=True)
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_attention_head_dims(rinf, synth, oracle, ctx, hd):
    """The prefill attention (f32 MFMA, tiles of 64 cached positions) at
    head_dim 64, 128 and 256, two query heads per kv head: 100 prompt tokens
    fed as 30 + 70 (the second call continues the caches; up to 100
    positions, two tiles), then greedy steps."""
    heads = 1024 // hd
    cfg = dict(SMALL, n_layers=1, embed_dim=1024, n_heads=heads, n_kv_heads=max(1, heads // 2), hidden_dim=512)
    e0, errs, out = prefill_and_compare(rinf, synth, oracle, ctx, cfg, "q4_k_m", 53, 100, 4, 128, split=30)
    print(f"head_dim {hd}: prefill logits err {e0:.2e}, decode max {max(errs):.2e}", flush=True)
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL


def test_qwen2_05b_prefill_then_decode(rinf, synth, oracle, ctx):
    """BASELINE.json configs[2]'s model (24 layers, tied Q4_K embedding at
    cols = 896, two-row groups) with its 32-token prompt through the batched
    prefill, then 32 greedy steps."""
    cfg = synth.ARCH["qwen2-0.5b"]
    e0, errs, out = prefill_and_compare(rinf, synth, oracle, ctx, cfg, "q4_k_m", synth.config_seed(2), 32, 32, 80)
    print(f"qwen2-0.5b: prefill logits err {e0:.2e}, decode max {max(errs):.2e}, tokens {out[:8]}", flush=True)
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL


def test_prefill_fallback_matches_forward(rinf, synth, oracle, ctx):
    """F16 matrices have no MFMA path: qg_model_prefill runs one forward pass
    per token, bit-identical to qg_model_forward calls; the batched path can
    be switched off for a supported mix with the same result as forward."""
    for mix, batched in (("f16", True), ("q4_k_m", False)):
        dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, mix, 53, 40)
        dev.use_batched_prefill(batched)
        prompt = np.random.default_rng(53).integers(0, SMALL["vocab_size"], 9)
        a = np.zeros(SMALL["vocab_size"], np.float32)
        dev.prefill(prompt, a)
        dev.reset()
        b = np.zeros_like(a)
        for pos, tok in enumerate(prompt):
            dev.forward(int(tok), pos, b)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        dev.close()


def test_generate_with_batched_prefill(rinf, synth, oracle, ctx):
    """qg_model_generate's tokens with the batched prefill equal those of the
    token-by-token prompt loop and of the oracle."""
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q4_k_m", 59, 64)
    prompt = np.random.default_rng(59).integers(0, SMALL["vocab_size"], 24)
    toks_b, _, _ = dev.generate(prompt, 12)
    dev.use_batched_prefill(False)
    toks_t, _, _ = dev.generate(prompt, 12)
    ref_l = None
    for pos, tok in enumerate(prompt):
        ref_l = ref.forward(int(tok), pos)
    ids = [int(t) for t in prompt]
    want = []
    for _ in range(12):
        rl = ref_l.copy()
        oracle.repetition_penalty(rl, ids[-64:], 1.1, 64)
        t = oracle.argmax(rl)
        want.append(t)
        ref_l = ref.forward(t, len(ids))
        ids.append(t)
    assert list(toks_b) == list(toks_t) == want
    dev.close()


def test_prefill_errors(rinf, synth, oracle, ctx):
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q4_k_m", 61, 16)
    with pytest.raises(rinf.QgemvError) as e:
        dev.prefill(np.arange(17) % SMALL["vocab_size"])          # more than max_seq_len
    assert e.value.status == 7
    with pytest.raises(rinf.QgemvError) as e:
        dev.prefill([1, SMALL["vocab_size"]])                      # token >= vocab
    assert e.value.status == 7
    assert dev.seq_len == 0
    dev.close()


def build_wrapped(rinf, synth, oracle, ctx, cfg, mix, seed, max_seq):
    """As test_decode_gpu.build, but every layer matrix is GGUF-layout bytes
    in device memory wrapped with qg_wrap_device and shared into its slot
    (never repacked), so the prefill GEMM reads the GGUF layout."""
    import torch
    t = synth.gen_model(cfg, mix, seed)
    dev = rinf.DeviceModel(ctx, cfg["embed_dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                           cfg["hidden_dim"], cfg["vocab_size"], max_seq, cfg["rope_base"], cfg["norm_eps"])
    ref = oracle.Model(dict(cfg, max_seq_len=max_seq))
    slots = {"token_embd": rinf.M_TOKEN_EMBD, "lm_head": rinf.M_LM_HEAD, "wq": rinf.M_WQ,
             "wk": rinf.M_WK, "wv": rinf.M_WV, "wo": rinf.M_WO, "gate": rinf.M_GATE,
             "up": rinf.M_UP, "down": rinf.M_DOWN}
    vslots = {"final_norm": rinf.V_FINAL_NORM, "attn_norm": rinf.V_ATTN_NORM,
              "ffn_norm": rinf.V_FFN_NORM, "bq": rinf.V_BQ, "bk": rinf.V_BK, "bv": rinf.V_BV}
    keep, layouts = [], set()
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        if slot in ("token_embd", "lm_head"):
            dev.set_matrix(slots[slot], layer, raw, dtype, rows, cols)
        else:
            buf = torch.zeros(raw.size + 512, dtype=torch.uint8, device="cuda")
            buf[:raw.size] = torch.from_numpy(np.ascontiguousarray(raw))
            h = ctx.wrap_device(buf, dtype, rows, cols)
            dev.share_matrix(slots[slot], layer, h)
            keep += [buf, h]
            layouts.add((dtype, "whole blocks" if cols % 256 == 0 or dtype == 8 else "straddling"))
        ref.set_mat(slot, layer, raw, dtype, rows, cols)
    for (name, layer), v in t["vecs"].items():
        dev.set_vector(vslots[name], layer, v)
        ref.set_vec(name, layer, v)
    return dev, ref, keep, layouts


@pytest.mark.parametrize("embed,hidden,mix", [(896, 1024, "q4_k_m"), (3584, 1024, "q4_k_m"), (3584, 1024, "q8_0")],
                         ids=["straddle-896", "whole-3584", "q8_0-3584"])
def test_prefill_gguf_layout_matrices(rinf, synth, oracle, ctx, embed, hidden, mix):
    """Wrapped (GGUF-layout) layer matrices through the batched prefill:
    Q4_K rows of 896 columns straddle superblocks (the general loader), Q4_K,
    Q6_K and Q8_0 rows of 3584 / 1024 columns hold whole blocks (the
    whole-block loader); 2 layers, a 40-token prompt, then 6 greedy steps,
    against the oracle."""
    heads = embed // 64 if embed == 896 else 28
    cfg = dict(SMALL, n_layers=2, embed_dim=embed, n_heads=heads, n_kv_heads=2 if embed == 896 else 4,
               hidden_dim=hidden)
    dev, ref, keep, layouts = build_wrapped(rinf, synth, oracle, ctx, cfg, mix, 83, 64)
    prompt = np.random.default_rng(83).integers(0, cfg["vocab_size"], 40)
    logits = np.zeros(cfg["vocab_size"], np.float32)
    dev.prefill(prompt, logits)
    ref_l = None
    for pos, tok in enumerate(prompt):
        ref_l = ref.forward(int(tok), pos)
    e0 = normwise_err(logits, ref_l)
    errs, out = decode_compare(dev, ref, oracle, cfg, [int(t) for t in prompt], ref_l, 6, len(prompt))
    print(f"wrapped {mix} {embed}: layouts {sorted(layouts)}, prefill logits err {e0:.2e}, "
          f"decode max {max(errs):.2e}", flush=True)
    dev.close()
    for k in keep:
        if hasattr(k, "free"):
            k.free()
    assert e0 <= DEEP_TOL and max(errs) <= DEEP_TOL
