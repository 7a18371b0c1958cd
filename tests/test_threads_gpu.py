"""One context per thread (include/qgemv.h, the reference's !Sync GpuContext,
src/gpu_backend.rs:14-18): several host threads, each with its own context,
upload and multiply -- or build and run decode-step models -- at the same
time (ctypes releases the GIL for every call, so the calls overlap inside the
library), and every result matches the oracle's, or the same model's run
alone.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, Q5_0 = 12, 14, 8, 6

# (type, rows, cols): stream, ring and generic kernels among them
CASES = [(Q4_K, 1024, 3584), (Q6_K, 512, 3584), (Q8_0, 768, 896), (Q5_0, 256, 1000)]


def test_contexts_in_parallel_threads(rinf, oracle, synth):
    jobs = []
    for k, (t, rows, cols) in enumerate(CASES):
        raw = synth.gen_blocks(t, rows, cols, 50 + k)
        xs = [synth.gen_x(cols, 60 + 4 * k + i) for i in range(4)]
        refs = [oracle.mat_vec_mul(raw, t, rows, cols, x) for x in xs]
        jobs.append((t, rows, cols, raw, xs, refs))
    errors, outs = [], {}

    def work(k):
        t, rows, cols, raw, xs, refs = jobs[k]
        try:
            c = rinf.GpuContext(0)
            try:
                m = c.upload(raw, t, rows, cols)
                got = []
                for rep in range(25):                  # uploaded handle, host path
                    y = np.zeros(rows, np.float32)
                    m.matvec_host(xs[rep % 4], y)
                    got.append(y)
                for rep in range(8):                   # the keyed drop-in
                    y = np.zeros(rows, np.float32)
                    c.mat_vec_mul(raw, t, xs[rep % 4], y, rows, cols)
                    got.append(y)
                outs[k] = got
                m.free()
            finally:
                c.close()
        except Exception as e:                         # reported by the main thread
            errors.append((k, repr(e)))

    threads = [threading.Thread(target=work, args=(k,)) for k in range(len(jobs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    for k, (t, rows, cols, raw, xs, refs) in enumerate(jobs):
        got = outs[k]
        for i, y in enumerate(got):
            ref = refs[(i if i < 25 else i - 25) % 4]
            assert normwise_err(y, ref) <= GEMV_TOL, (t, rows, cols, i)
        # same x, same kernel: bit-identical across the concurrent repetitions
        for i in range(4, 25):
            assert np.array_equal(got[i], got[i - 4]), (t, i)


def test_models_in_parallel_threads(rinf, oracle, synth):
    """Two decode-step models, each on its own context and host thread,
    generate at the same time (batched prefill, HIP-graph decode, on-device
    sampler): each thread's tokens equal those of the same model run alone."""
    from test_decode_gpu import SMALL, build
    prompt = (np.arange(3, 45, dtype=np.uint32) * 7) % SMALL["vocab_size"]
    seeds = (21, 22)

    def run(seed):
        c = rinf.GpuContext(0)
        try:
            dev, _, _ = build(rinf, synth, oracle, c, dict(SMALL), "q4_k_m", seed, 128)
            try:
                return np.array(dev.generate(prompt, 24)[0])
            finally:
                dev.close()
        finally:
            c.close()

    alone = {s: run(s) for s in seeds}
    got, errors = {}, []

    def work(s):
        try:
            got[s] = run(s)
        except Exception as e:                         # reported by the main thread
            errors.append((s, repr(e)))

    threads = [threading.Thread(target=work, args=(s,)) for s in seeds]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    for s in seeds:
        assert np.array_equal(got[s], alone[s]), (s, got[s][:8], alone[s][:8])
    assert not np.array_equal(alone[seeds[0]], alone[seeds[1]])
