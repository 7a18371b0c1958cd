"""Full-depth parity on the path bench.py times
(the 28-layer Qwen2-7B Q4_K_M model of the bench, same seed, its 64-token
random prompt, 256 greedy steps) and configs[4] (32-layer Llama-3-8B Q4_K_M,
64-token prompt, 64 greedy steps).

The prompt goes through the batched prefill (qg_model_prefill: one 64-token
chunk per layer on the matrix cores), as qg_model_generate runs it for the
bench; the reference feeds it token by token (src/model.rs:361-365), so the
oracle runs its token-by-token forward pass (oracle/qref_model.c) over the
same prompt.  Then every greedy step (src/model.rs:376-438: repetition
penalty 1.1 over the last 64 tokens, first maximum) is compared: the device
logits within DEEP_TOL (normwise 1e-4) of the oracle's, and the device's
greedy token equal to the reference's (a different choice is accepted only
as a near-tie, penalised logits within 1e-5 of max|logits|, after which both
sides continue with the reference's token).  Finally qg_model_generate --
the bench's own call, graph replays with the sampler on device -- must give
the device's stepwise tokens up to the first near-tie (all of them when
there is none)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import normwise_err
from test_decode_gpu import DEEP_TOL, build

pytestmark = pytest.mark.gpu

TIE_TOL = 1e-5


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("arch,mix,cidx,n_new", [("qwen2-7b", "q4_k_m", 3, 256), ("llama3-8b", "q4_k_m", 4, 64)],
                         ids=["qwen2-7b-64+256", "llama3-8b-64+64"])
def test_prefill_then_greedy_full_depth(rinf, synth, oracle, ctx, arch, mix, cidx, n_new):
    cfg = synth.ARCH[arch]
    seed = synth.config_seed(cidx)
    n_prompt = 64
    dev, ref, _ = build(rinf, synth, oracle, ctx, cfg, mix, seed, n_prompt + n_new + 1)
    V = cfg["vocab_size"]
    prompt = np.random.default_rng(seed).integers(0, V, n_prompt)      # bench.py decode_run's prompt
    logits = np.zeros(V, np.float32)
    dev.prefill(prompt, logits)
    assert dev.seq_len == n_prompt
    ref_l = None
    for pos, tok in enumerate(prompt):
        ref_l = ref.forward(int(tok), pos)
    e_prefill = normwise_err(logits, ref_l)
    print(f"{arch} {mix}: prefill (64 tokens, one chunk) last-token logits err {e_prefill:.2e}", flush=True)
    assert e_prefill <= DEEP_TOL

    ids = [int(t) for t in prompt]
    errs, dev_toks, ref_toks = [], [], []
    pos = n_prompt
    for step in range(n_new):
        recent = ids[-64:]
        t_dev = dev.sample_greedy(recent, 1.1, 64)
        rl = ref_l.copy()
        oracle.repetition_penalty(rl, recent, 1.1, 64)
        t_ref = oracle.argmax(rl)
        if t_dev != t_ref:
            gap = abs(float(rl[t_ref]) - float(rl[t_dev])) / float(np.max(np.abs(rl)))
            print(f"step {step}: near-tie {t_dev} vs {t_ref}, relative gap {gap:.2e}", flush=True)
            assert gap <= TIE_TOL, f"step {step}: device token {t_dev} != reference {t_ref} (gap {gap:.2e})"
        dev_toks.append(t_dev)
        ref_toks.append(t_ref)
        dev.forward(t_ref, pos, logits)
        ref_l = ref.forward(t_ref, pos)
        errs.append(normwise_err(logits, ref_l))
        ids.append(t_ref)
        pos += 1
        if step % 32 == 31:
            print(f"  step {step + 1}: max logits err so far {max(errs):.2e}", flush=True)
    print(f"{arch} {mix} {n_prompt}+{n_new}: decode logits err max {max(errs):.2e}, median "
          f"{np.median(errs):.2e}, last {errs[-1]:.2e}; tokens {ref_toks[:12]}...", flush=True)
    assert len(errs) == n_new
    assert max(errs) <= DEEP_TOL

    # the bench's call: prefill + greedy steps on device (graph replays)
    gen, _, _ = dev.generate(prompt, n_new)
    gen = [int(t) for t in gen]
    first = next((i for i, (a, b) in enumerate(zip(dev_toks, ref_toks)) if a != b), n_new - 1)
    assert gen[:first + 1] == dev_toks[:first + 1]
    if first == n_new - 1:
        assert gen == ref_toks
    dev.close()
