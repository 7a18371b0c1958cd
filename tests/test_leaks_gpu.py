"""Device memory comes back: contexts, uploaded and keyed matrices (sampled
and exact freshness), the f32 path and decode-step models with their
batched prefill, built and torn down several times in one process, leave the
device's free memory where the first round left it (hipMemGetInfo; the
library allocates with hipMalloc, outside torch's caching allocator).
"""
from __future__ import annotations

import numpy as np
import pytest

from test_decode_gpu import SMALL, build

pytestmark = pytest.mark.gpu

Q4_K = 12
MiB = 1 << 20


def one_round(rinf, synth, oracle):
    c = rinf.GpuContext(0)
    try:
        rows, cols = 1024, 3584
        raw = synth.gen_blocks(Q4_K, rows, cols, 11)
        x = synth.gen_x(cols, 11)
        y = np.zeros(rows, np.float32)
        m = c.upload(raw, Q4_K, rows, cols)
        m.matvec_host(x, y)
        m.free()
        c.mat_vec_mul(raw, Q4_K, x, y, rows, cols)             # keyed copy, sampled
        c.set_freshness(rinf.FRESH_EXACT)
        c.mat_vec_mul(raw, Q4_K, x, y, rows, cols)             # keyed copy again, exact
        c.set_precision(rinf.PRECISION_F32)
        c.mat_vec_mul(raw, Q4_K, x, y, rows, cols)
        c.set_precision(rinf.PRECISION_FIXED22)
        dev, _, _ = build(rinf, synth, oracle, c, dict(SMALL), "q4_k_m", 5, 128)
        try:
            dev.generate(np.arange(1, 40, dtype=np.uint32) % SMALL["vocab_size"], 8)
        finally:
            dev.close()
        c.synchronize()
    finally:
        c.close()


def test_device_memory_returns(rinf, synth, oracle):
    import torch
    one_round(rinf, synth, oracle)                               # first-use allocations (runtime, code objects)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(4):
        one_round(rinf, synth, oracle)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    print(f"free device memory: {free0 / MiB:.1f} MiB after the first round, {free1 / MiB:.1f} MiB after "
          f"four more", flush=True)
    assert free0 - free1 < 16 * MiB
