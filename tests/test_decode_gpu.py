"""GPU parity of the on-device decode step (include/qgmodel.h) against the
oracle's restatement of Transformer::forward (oracle/qref_model.c,
src/transformer.rs:63-98) and of the greedy sampler with repetition penalty
(src/sampler.rs:72-83, 109-127; src/math.rs:328-339).

Per step, the device logits must agree with the oracle's within normwise
max|Δ| / max|logits_ref| <= LOGIT_TOL (2 layers) or DEEP_TOL (full-depth
models, long contexts), and the greedily sampled token ids must be
identical.  The models are synth.gen_model's random-init weights (centred,
~1/sqrt(cols)), whose activations stay O(1) at any depth; the device and the
oracle then differ only by reduction order and the GEMV's exact integer
accumulation (measured: at most 9.4e-6 over every test here, Qwen2-0.5B at
32 + 128 steps 6.0e-6).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import normwise_err

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-4
DEEP_TOL = 1e-4

SMALL = dict(embed_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=512, vocab_size=600,
             rope_base=1e6, norm_eps=1e-6, tied=False, bias=True)


def build(rinf, synth, oracle, ctx, cfg, mix, seed, max_seq):
    t = synth.gen_model(cfg, mix, seed)
    dev = rinf.DeviceModel(ctx, cfg["embed_dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                           cfg["hidden_dim"], cfg["vocab_size"], max_seq, cfg["rope_base"],
                           cfg["norm_eps"])
    ocfg = dict(cfg, max_seq_len=max_seq)
    ref = oracle.Model(ocfg)
    slots = {"token_embd": rinf.M_TOKEN_EMBD, "lm_head": rinf.M_LM_HEAD, "wq": rinf.M_WQ,
             "wk": rinf.M_WK, "wv": rinf.M_WV, "wo": rinf.M_WO, "gate": rinf.M_GATE,
             "up": rinf.M_UP, "down": rinf.M_DOWN}
    vslots = {"final_norm": rinf.V_FINAL_NORM, "attn_norm": rinf.V_ATTN_NORM,
              "ffn_norm": rinf.V_FFN_NORM, "bq": rinf.V_BQ, "bk": rinf.V_BK, "bv": rinf.V_BV}
    shared = None
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        if slot == "token_embd" and cfg.get("tied"):
            shared = ctx.upload(raw, dtype, rows, cols)
            dev.share_matrix(rinf.M_TOKEN_EMBD, 0, shared)
            dev.share_matrix(rinf.M_LM_HEAD, 0, shared)
            ref.set_mat("lm_head", 0, raw, dtype, rows, cols)           # tied (model.rs:221-226)
        else:
            dev.set_matrix(slots[slot], layer, raw, dtype, rows, cols)
        ref.set_mat(slot, layer, raw, dtype, rows, cols)
    for (name, layer), v in t["vecs"].items():
        dev.set_vector(vslots[name], layer, v)
        ref.set_vec(name, layer, v)
    return dev, ref, shared


def run_and_compare(dev, ref, oracle, cfg, prompt, n_new, penalty=1.1, window=64, tie_tol=0.0):
    """Prompt then greedy decode, step by step on both sides.  A different
    greedy choice is accepted only as a near-tie: the reference's penalised
    logits of the two tokens differ by at most tie_tol * max|logits|; both
    sides then continue with the reference's token."""
    V = cfg["vocab_size"]
    logits = np.zeros(V, np.float32)
    all_ids, errs, out = [], [], []
    pos = 0
    for tok in prompt:
        dev.forward(int(tok), pos, logits)
        ref_l = ref.forward(int(tok), pos)
        errs.append(normwise_err(logits, ref_l))
        all_ids.append(int(tok))
        pos += 1
    for _ in range(n_new):
        recent = all_ids[-64:]
        t_dev = dev.sample_greedy(recent, penalty, window)
        rl = ref_l.copy()
        oracle.repetition_penalty(rl, recent, penalty, window)
        t_ref = oracle.argmax(rl)
        if t_dev != t_ref:
            gap = abs(float(rl[t_ref]) - float(rl[t_dev])) / float(np.max(np.abs(rl)))
            print(f"step {len(out)}: near-tie {t_dev} vs {t_ref}, relative gap {gap:.2e}", flush=True)
            assert gap <= tie_tol, f"step {len(out)}: device token {t_dev} != reference {t_ref} (gap {gap:.2e})"
        out.append(t_ref)
        dev.forward(t_ref, pos, logits)
        ref_l = ref.forward(t_ref, pos)
        errs.append(normwise_err(logits, ref_l))
        all_ids.append(t_ref)
        pos += 1
    return out, errs


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k", "q8_0", "f16"])
def test_small_model_logits_and_tokens(rinf, synth, oracle, ctx, mix):
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, mix, 11, 40)
    prompt = np.random.default_rng(5).integers(0, SMALL["vocab_size"], 8)
    out, errs = run_and_compare(dev, ref, oracle, SMALL, prompt, 16)
    print(f"{mix}: max logits err {max(errs):.2e}, tokens {out}", flush=True)
    assert max(errs) <= LOGIT_TOL
    assert dev.seq_len == 24
    dev.close()


def test_head_dim_96_general_attention(rinf, synth, oracle, ctx):
    """head_dim 96 (not a multiple of 64) takes the general attention kernel."""
    cfg = dict(SMALL, embed_dim=384, hidden_dim=768)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q8_0", 13, 24)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab_size"], 5)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 6)
    assert max(errs) <= LOGIT_TOL
    dev.close()


@pytest.mark.parametrize("embed,heads,kv", [(512, 4, 2), (512, 2, 1), (448, 7, 1)],
                         ids=["hd128", "hd256", "hd64-rep7"])
def test_head_layouts(rinf, synth, oracle, ctx, embed, heads, kv):
    """Split attention for head_dim 64 / 128 / 256 and 7 query heads per kv head."""
    cfg = dict(SMALL, embed_dim=embed, n_heads=heads, n_kv_heads=kv, hidden_dim=2 * embed)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q8_0", 17, 32)
    prompt = np.random.default_rng(8).integers(0, cfg["vocab_size"], 9)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 12)
    print(f"{embed}/{heads}/{kv}: max logits err {max(errs):.2e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    dev.close()


def test_long_sequence(rinf, synth, oracle, ctx):
    """~100 cached positions: every attention range holds several of them."""
    cfg = dict(SMALL, n_layers=1)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", 19, 512)
    prompt = np.random.default_rng(9).integers(0, cfg["vocab_size"], 90)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 12)
    print(f"long: max logits err {max(errs):.2e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    dev.close()


@pytest.mark.parametrize("embed", [256, 512], ids=["hd64", "hd128"])
def test_long_ranges(rinf, synth, oracle, ctx, embed):
    """~600 cached positions over 64 ranges of 10: a wave runs two chunks of
    positions, and the appended slot sits in a later chunk of its range.  At
    this length the maximum is held to DEEP_TOL and the typical step to
    1e-5."""
    cfg = dict(SMALL, n_layers=1, embed_dim=embed, hidden_dim=2 * embed)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q8_0", 23, 640)
    prompt = np.random.default_rng(10).integers(0, cfg["vocab_size"], 590)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 12)
    print(f"ranges {embed}: max logits err {max(errs):.2e}, median {np.median(errs):.2e}", flush=True)
    assert max(errs) <= DEEP_TOL
    assert np.median(errs) <= 1e-5
    dev.close()


@pytest.mark.parametrize("path", [1, 2, 3], ids=["whole-heads", "split", "two-range"])
@pytest.mark.parametrize("embed", [256, 512, 1024], ids=["hd64", "hd128", "hd256"])
def test_attention_paths(rinf, synth, oracle, ctx, path, embed):
    """The attention kernels of the decode step (qg_model_set_attention_path:
    whole query heads in one launch; position ranges then a merge kernel; two
    workgroups per head merged in the wo GEMV's input) against the oracle at
    the same lengths, for head_dim 64, 128 and 256: 70 prompt positions, then
    10 greedy steps."""
    cfg = dict(SMALL, n_layers=1, embed_dim=embed, hidden_dim=2 * embed)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q8_0", 29, 96)
    dev.set_attention_path(path)
    prompt = np.random.default_rng(14).integers(0, cfg["vocab_size"], 70)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 10)
    print(f"path {path} hd {embed // 4}: max logits err {max(errs):.2e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    dev.close()


def test_attention_path_switch_in_generate(rinf, synth, oracle, ctx):
    """A generation across the 512-position boundary (505 prompt tokens, 14
    new): the decode graph changes from two-range to split attention
    mid-run.  The tokens equal those of the step-by-step run, which follows
    the oracle within DEEP_TOL."""
    cfg = dict(SMALL, n_layers=1)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", 31, 540)
    prompt = np.random.default_rng(13).integers(0, cfg["vocab_size"], 505)
    toks, _, _ = dev.generate(prompt, 14)
    dev.reset()
    ref.reset()
    step, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 14)
    print(f"switch: max logits err {max(errs):.2e}", flush=True)
    assert list(toks) == step
    assert max(errs) <= DEEP_TOL
    dev.close()


@pytest.mark.parametrize("path", [1, 3], ids=["whole-heads", "two-range"])
def test_attention_paths_qwen2_7b_heads(rinf, synth, oracle, ctx, path):
    """28 query heads on 4 kv heads of dim 128 (wo Q4_K, 3584 columns): the
    two-range attention, its merge in the wo GEMV's input and the one-launch
    kernel against the oracle over 150 positions, including a position range
    with no positions (the first token of the prompt)."""
    cfg = dict(SMALL, n_layers=1, embed_dim=3584, n_heads=28, n_kv_heads=4, hidden_dim=1024)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", 33, 160)
    dev.set_attention_path(path)
    prompt = np.random.default_rng(15).integers(0, cfg["vocab_size"], 140)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 10)
    print(f"7b heads path {path}: max logits err {max(errs):.2e}, median {np.median(errs):.2e}", flush=True)
    assert max(errs) <= DEEP_TOL
    dev.close()


@pytest.mark.parametrize("mix", ["q4_k_m", "q5_k_m"])
def test_qwen2_7b_layer_shape(rinf, synth, oracle, ctx, mix):
    """One layer of the Qwen2-7B shape: [Q;K] (Q4_K or Q5_K) and V (Q6_K) in
    one launch, gate/up paired at 3584 cols, 7 query heads per kv head of dim
    128."""
    cfg = dict(SMALL, n_layers=1, embed_dim=3584, n_heads=28, n_kv_heads=4, hidden_dim=1024)
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, mix, 29, 64)
    prompt = np.random.default_rng(12).integers(0, cfg["vocab_size"], 12)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 8)
    print(f"7b layer {mix}: max logits err {max(errs):.2e}, median {np.median(errs):.2e}", flush=True)
    assert max(errs) <= DEEP_TOL
    assert np.median(errs) <= 1e-5
    dev.close()


def test_graph_replay_matches_eager(rinf, synth, oracle, ctx):
    """Graph replays give the logits of one-launch-per-kernel execution, bit for
    bit, with other GPU work and synchronisations between the replays."""
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q4_k_m", 21, 40)
    raw = synth.gen_blocks(12, 64, 256, 3)
    other = ctx.upload(raw, 12, 64, 256)
    x = synth.gen_x(256, 3)
    y = np.zeros(64, np.float32)
    toks = np.random.default_rng(10).integers(0, SMALL["vocab_size"], 10)
    runs = []
    for graphs in (False, True):
        dev.use_graphs(graphs)
        dev.reset()
        steps = []
        for p, t in enumerate(toks):
            lg = np.zeros(SMALL["vocab_size"], np.float32)
            dev.forward(int(t), p, lg)
            other.matvec_host(x, y)                 # eager work between replays
            steps.append(lg)
        runs.append(steps)
    for a, b in zip(*runs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    other.free()
    dev.close()


def test_generate_graph_and_eager(rinf, synth, oracle, ctx):
    """generate's on-device sample + forward loop: same tokens with and without graphs."""
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q5_k", 23, 40)
    prompt = np.random.default_rng(11).integers(0, SMALL["vocab_size"], 7)
    dev.use_graphs(False)
    eager, _, _ = dev.generate(prompt, 14)
    dev.use_graphs(True)
    graph, _, _ = dev.generate(prompt, 14)
    again, _, _ = dev.generate(prompt, 14)
    assert list(eager) == list(graph) == list(again)
    assert dev.seq_len == 21
    dev.close()


def test_generate_matches_stepwise(rinf, synth, oracle, ctx):
    """qg_model_generate (Model::generate's loop) gives the tokens of the
    step-by-step run and of the reference sampler."""
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q4_k_m", 12, 40)
    prompt = np.random.default_rng(6).integers(0, SMALL["vocab_size"], 6)
    toks, t_pre, t_dec = dev.generate(prompt, 12)
    dev.reset()
    ref.reset()
    step, _ = run_and_compare(dev, ref, oracle, SMALL, prompt, 12)
    assert list(toks) == step
    assert t_pre > 0 and t_dec > 0
    dev.close()


def test_sampler_repeats_ties_and_nan(rinf, synth, oracle, ctx):
    """The one-launch sampler against the reference's sequential penalty loop
    and first-maximum scan: a token listed k times is penalised k times (the
    penalty is chosen so that 2 and 3 occurrences give different winners),
    only the last `window` entries count, equal logits go to the smaller index
    across workgroup ranges, and a NaN logit at index 0 returns token 0."""
    V = SMALL["vocab_size"]
    t = synth.gen_model(SMALL, "q8_0", 31)
    raw, dtype, rows, cols = t["mats"][("lm_head", 0)]
    dev, ref, _ = build(rinf, synth, oracle, ctx, SMALL, "q8_0", 31, 8)
    lg = np.zeros(V, np.float32)

    def sample(recent, penalty, window=64):
        dev.reset()
        dev.forward(3, 0, lg)
        base = lg.copy()
        tok = dev.sample_greedy(recent, penalty, window)
        rl = base.copy()
        oracle.repetition_penalty(rl, recent, penalty, window)
        assert tok == oracle.argmax(rl), (recent, penalty, window)
        return tok, base

    _, base = sample([], 1.0)
    order = np.argsort(-base, kind="stable")
    a, b = int(order[0]), int(order[1])
    assert base[b] > 0
    p = float((base[a] / base[b]) ** (1 / 2.5))     # a/p^2 > b > a/p^3
    others = [int(v) for v in order[5:12]]
    two = [others[0], a, others[1], a, others[2]]
    three = [a, others[3], a, others[4], a]
    assert sample(two, p)[0] == a
    assert sample(three, p)[0] == b
    assert sample(others[:2] + three, p, window=5)[0] == b
    assert sample(three + others[:2], p, window=4)[0] == a      # one occurrence left
    # a tie: row c (another workgroup's range) holds row a's bytes
    c = next(i for i in range(V) if abs(i - a) > 8)
    tied = np.array(raw, np.uint8, copy=True).reshape(rows, -1)      # whole Q8_0 blocks per row
    tied[c] = tied[a]
    dev.set_matrix(rinf.M_LM_HEAD, 0, tied, dtype, rows, cols)
    tok, base = sample([], 1.0)
    assert base[c] == base[a] and tok == min(a, c)
    assert sample([min(a, c)], 1.1)[0] == max(a, c)
    # NaN at index 0 (an F32 lm_head row of NaNs)
    f = np.full((rows, cols), 0.01, np.float32)
    f[0] = np.nan
    dev.set_matrix(rinf.M_LM_HEAD, 0, f, rinf.F32, rows, cols)
    tok, base = sample([5, 6], 1.1)
    assert np.isnan(base[0]) and tok == 0
    dev.close()


def test_qwen2_05b_config3_as_stated(rinf, synth, oracle, ctx):
    """BASELINE.json configs[2] exactly: Qwen2-0.5B architecture, Q4_K_M, tied
    lm_head, token_embd Q4_K at cols = 896 (rows straddle superblocks: the
    dequantize_row placement of quant.rs:152-174 is in the loop), a 32-token
    random-id prompt then 128 greedy steps, the logits of every one of the
    160 steps against the oracle's CPU forward pass and every greedy token
    against the reference's sampler."""
    cfg = synth.ARCH["qwen2-0.5b"]
    dev, ref, shared = build(rinf, synth, oracle, ctx, cfg, "q4_k_m", synth.config_seed(2), 161)
    prompt = np.random.default_rng(synth.config_seed(2)).integers(0, cfg["vocab_size"], 32)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 128)
    print(f"qwen2-0.5b 32+128: max logits err {max(errs):.2e}, median {np.median(errs):.2e}, "
          f"last {errs[-1]:.2e}, tokens {out[:16]}...", flush=True)
    assert len(errs) == 160
    assert max(errs) <= DEEP_TOL
    dev.close()
    shared.free()


@pytest.mark.parametrize("arch,mix,cidx", [("qwen2-7b", "q4_k_m", 3), ("llama3-8b", "q4_k_m", 4),
                                           ("llama3-8b", "q5_k", 4), ("llama3-8b", "q8_0", 4)])
def test_full_size_models(rinf, synth, oracle, ctx, arch, mix, cidx):
    """BASELINE.json configs[3] and [4] at full size: the 28-layer Qwen2-7B
    model of the bench (Q4_K_M, same seed) and the 32-layer Llama-3-8B in the
    Q4_K_M, Q5_K and Q8_0 mixes; 16 prompt tokens then 16 greedy steps
    (32 positions: several attention ranges per head), logits and tokens
    against the oracle's CPU forward pass."""
    cfg = synth.ARCH[arch]
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, mix, synth.config_seed(cidx), 40)
    prompt = np.random.default_rng(synth.config_seed(cidx)).integers(0, cfg["vocab_size"], 16)
    out, errs = run_and_compare(dev, ref, oracle, cfg, prompt, 16)
    print(f"{arch} {mix} 16+16: max logits err {max(errs):.2e}, median {np.median(errs):.2e}, "
          f"tokens {out}", flush=True)
    assert len(errs) == 32
    assert max(errs) <= DEEP_TOL
    dev.close()


def test_errors(rinf, synth, ctx):
    dev = rinf.DeviceModel(ctx, 256, 1, 4, 2, 512, 100, 4, 1e6, 1e-6)
    with pytest.raises(rinf.QgemvError) as e:
        dev.forward(0, 0)                                   # matrices not set
    assert e.value.status == 1
    t = synth.gen_model(dict(SMALL, n_layers=1, vocab_size=100), "q4_k_m", 3)
    slots = {"token_embd": rinf.M_TOKEN_EMBD, "lm_head": rinf.M_LM_HEAD, "wq": rinf.M_WQ,
             "wk": rinf.M_WK, "wv": rinf.M_WV, "wo": rinf.M_WO, "gate": rinf.M_GATE,
             "up": rinf.M_UP, "down": rinf.M_DOWN}
    with pytest.raises(rinf.QgemvError) as e:
        raw, dtype, rows, cols = t["mats"][("wq", 0)]
        dev.set_matrix(rinf.M_WQ, 0, raw, dtype, rows, cols + 256)   # wrong shape
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        dev.set_matrix(slots[slot], layer, raw, dtype, rows, cols)
    dev.set_vector(rinf.V_FINAL_NORM, 0, np.ones(256, np.float32))
    with pytest.raises(rinf.QgemvError) as e:
        dev.forward(100, 0)                                 # token >= vocab
    assert e.value.status == 7
    for p in range(4):
        dev.forward(1, p)
    with pytest.raises(rinf.QgemvError) as e:
        dev.forward(1, 4)                                   # KV cache full (kv_cache.rs:54-59)
    assert e.value.status == 7
    dev.reset()
    dev.forward(1, 0)
    dev.close()
