#!/usr/bin/env python3
"""Benchmark of the hot path: Q4_K mat-vec at 4096 x 14336 on one MI355X.

One step = one QuantizedMatrix::mat_vec_mul (src/quant.rs:178) over a
4096 x 14336 Q4_K matrix already resident in HBM, launched through the C ABI
(qg_matvec_dev).  Steps rotate over enough distinct weight copies (>= 512 MB)
that every launch misses the 256 MB Infinity Cache and streams from HBM.

value        whole-job GB/s = algorithmic bytes x K / wall time of K back-to-back
             launches (the better of eager launches and a HIP-graph replay)
roofline     algorithmic bytes / average launch duration of the GEMV kernel:
             HIP events around K back-to-back launches, eager or replayed from
             a HIP graph, whichever is faster (one kernel per launch, so
             rocprofv3 --kernel-trace --stats of the same command gives the
             same average up to the inter-kernel gaps), against 8 TB/s;
             `traffic` is the HBM bytes per launch from rocprofv3 FETCH_SIZE +
             WRITE_SIZE (profiles/traffic.json, written by --pmc-summary), or null
cpu_baseline the oracle's restatement of the reference's --cpu loop
             (src/quant.rs:188-205) on one host core, same matrix
ceiling      the streaming-read ceiling at the same byte count: a sweep of
             plain read designs (libqgprobe.so, include/qgprobe.h: 256/512/1024
             threads, 1-8 loads per thread, full or persistent grids of
             256-4096 workgroups), gemv_wave's own load pattern without its
             compute, and torch.sum, over rotating copies; also at 76 MB and
             447 MB (the 7B [gate;up] and lm_head sizes); roofline.ceiling_us
             is the fastest read at the headline size
sweep        BASELINE.json configs[1]: the per-type GEMVs at the Qwen2-0.5B
             shapes and the Q6_K 151936 x 896 lm_head
decode, decode_configs
             configs[3] (Qwen2-7B Q4_K_M, 64 + 256) and configs[2] / [4]
             (Qwen2-0.5B Q4_K_M 32 + 128; Llama-3-8B Q4_K_M / Q5_K / Q8_0,
             64 + 512): greedy decode tok/s with the HBM roofline fraction
--timeline   instead of all that: the s_memrealtime stamps of the GEMV the
             shape plans (libqgemv_timeline.so: the wave-private kernel for
             Q4_K 4096 x 14336, the LDS-ring kernel for e.g. Q6_K 3584 x 18944)
             -- where a launch spends its time; with --timeline-glu those of
             the stream kernel's [gate; up] form

Algorithmic bytes per GEMV: ceil(rows*cols/256)*144 + 4*cols + 4*rows.
Only rank 0 of one GPU is supported (--gpus > 1 exits with a message).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Q4_K GEMV HBM GB/s (% of 8 TB/s); decode tok/s Qwen2-7B-shape"
PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def alg_bytes(rinf, dtype, rows, cols):
    return rinf.nbytes_for(dtype, rows, cols) + 4 * cols + 4 * rows


def time_gemv(ctx, torch, mats, dx, dy, steps, warmup):
    """Four timings of `steps` launches that rotate over `mats`:
    c_loop -- wall ms of back-to-back qg_matvec_dev calls issued from C
              (qg_matvec_dev_repeat), as a compiled caller issues them,
    eager  -- wall ms of back-to-back launches from Python (host-bound if the
              launch call is slower than the kernel),
    graph  -- wall ms of the same launches captured once in a HIP graph
              (one graph = one pass over the copies) and replayed,
    per    -- per-launch event pairs around eager launches (kernel duration
              plus event overhead)."""
    n = len(mats)
    st = torch.cuda.ExternalStream(ctx.stream)
    for i in range(warmup):
        mats[i % n].matvec_dev(dx, dy, ctx.stream)
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    e0, e1 = ev(), ev()
    e0.record(st)
    for i in range(steps):
        mats[i % n].matvec_dev(dx, dy, ctx.stream)
    e1.record(st)
    torch.cuda.synchronize()
    eager = e0.elapsed_time(e1)

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            s = torch.cuda.current_stream().cuda_stream
            for m in mats:
                m.matvec_dev(dx, dy, s)
    torch.cuda.synchronize()
    reps = max(1, steps // n)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    g0, g1 = ev(), ev()
    g0.record(cur)
    for _ in range(reps):
        g.replay()
    g1.record(cur)
    torch.cuda.synchronize()
    graph = g0.elapsed_time(g1) * steps / (reps * n)

    ctx.matvec_repeat(mats, dx, dy, warmup, ctx.stream)
    torch.cuda.synchronize()
    c0, c1 = ev(), ev()
    c0.record(st)
    h0 = time.perf_counter()
    ctx.matvec_repeat(mats, dx, dy, steps, ctx.stream)
    h1 = time.perf_counter()
    c1.record(st)
    torch.cuda.synchronize()
    c_loop = c0.elapsed_time(c1)
    log(f"C loop: host enqueue {(h1 - h0) * 1e6 / steps:.2f} us per launch")

    evs = [(ev(), ev()) for _ in range(steps)]
    for i, (a, b) in enumerate(evs):
        a.record(st)
        mats[i % n].matvec_dev(dx, dy, ctx.stream)
        b.record(st)
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) for a, b in evs]
    del g
    return c_loop, eager, graph, per


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _time_loop(fn, seconds):
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end and len(times) >= 5:
            return times


def cpu_baseline(oracle, raw, dtype, rows, cols, x, seconds, nbytes):
    """Both reference CPU paths, restated in oracle/qref.c, single-threaded and
    pinned to one core (the reference has no threads): (A) the --cpu loop of
    QuantizedMatrix::mat_vec_mul (src/quant.rs:188-205), reported as `value`,
    and (B) fallback_cpu (src/gpu_backend.rs:543-567: dequantize, then
    mat_vec_mul_transposed), reported beside it.  Bounded sample: about
    `seconds` of CPU work for (A) and a third of that for (B)."""
    pinned = None
    if hasattr(os, "sched_getaffinity"):
        old = os.sched_getaffinity(0)
        core = min(old)
        try:
            os.sched_setaffinity(0, {core})
            pinned = core
        except OSError:
            old = None
    try:
        ta = _time_loop(lambda: oracle.mat_vec_mul(raw, dtype, rows, cols, x), seconds)
        tb = _time_loop(lambda: oracle.fallback_cpu(raw, dtype, rows, cols, x), seconds / 3)
    finally:
        if pinned is not None and old:
            os.sched_setaffinity(0, old)
    ma, mb = statistics.median(ta), statistics.median(tb)
    where = f"core {pinned} of {os.cpu_count()} ({_cpu_model()})" if pinned is not None else \
        f"1 thread, unpinned, of {os.cpu_count()} ({_cpu_model()})"
    return {"value": round(nbytes / ma / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(ta)} full Q4_K {rows}x{cols} GEMVs (median {ma * 1e3:.1f} ms each) through "
                      f"oracle/qref.c's restatement of src/quant.rs:188-205, one thread on {where}",
            "us_per_gemv": round(ma * 1e6, 1),
            "fallback_cpu": {"value": round(nbytes / mb / 1e9, 4), "unit": "GB/s",
                             "us_per_gemv": round(mb * 1e6, 1), "runs": len(tb),
                             "path": "src/gpu_backend.rs:543-567 (dequantize + mat_vec_mul_transposed)"}}


def decode_run(rinf, synth, ctx, args, arch=None, mix=None, n_prompt=None, n_new=None, cfg_index=3):
    """BASELINE.json configs[3] (by default): greedy decode of a random-init
    model of `arch` in the `mix` GGUF mix, all GEMVs on this GPU.  The prompt
    goes through the batched prefill (chunks of up to 64 tokens per layer,
    MFMA GEMMs; qg_model_prefill) where the mix has it, then `n_new` greedy
    steps with the reference's repetition penalty 1.1 over the last 64
    tokens; the prompt is then timed again one token at a time, as the
    reference feeds it (src/model.rs:361-365)."""
    import numpy as np
    arch = arch or args.decode
    mix = mix or args.decode_mix
    n_prompt = args.decode_prompt if n_prompt is None else n_prompt
    n_new = args.decode_tokens if n_new is None else n_new
    cfg = synth.ARCH[arch]
    seed = synth.config_seed(cfg_index)
    t0 = time.perf_counter()
    t = synth.gen_model(cfg, mix, seed)
    max_seq = n_prompt + n_new + 1
    dev = rinf.DeviceModel(ctx, cfg["embed_dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                           cfg["hidden_dim"], cfg["vocab_size"], max_seq, cfg["rope_base"],
                           cfg["norm_eps"])
    slots = {"token_embd": rinf.M_TOKEN_EMBD, "lm_head": rinf.M_LM_HEAD, "wq": rinf.M_WQ,
             "wk": rinf.M_WK, "wv": rinf.M_WV, "wo": rinf.M_WO, "gate": rinf.M_GATE,
             "up": rinf.M_UP, "down": rinf.M_DOWN}
    vslots = {"final_norm": rinf.V_FINAL_NORM, "attn_norm": rinf.V_ATTN_NORM,
              "ffn_norm": rinf.V_FFN_NORM, "bq": rinf.V_BQ, "bk": rinf.V_BK, "bv": rinf.V_BV}
    shared = None
    for (slot, layer), (raw, dtype, rows, cols) in list(t["mats"].items()):
        if slot == "token_embd" and cfg.get("tied"):
            shared = ctx.upload(raw, dtype, rows, cols)
            dev.share_matrix(rinf.M_TOKEN_EMBD, 0, shared)
            dev.share_matrix(rinf.M_LM_HEAD, 0, shared)
        else:
            dev.set_matrix(slots[slot], layer, raw, dtype, rows, cols)
        del t["mats"][(slot, layer)]
    for (name, layer), v in t["vecs"].items():
        dev.set_vector(vslots[name], layer, v)
    setup_s = time.perf_counter() - t0
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab_size"], n_prompt)
    dev.generate(prompt[:4], 4)                           # warm-up (kernels, clocks)
    toks, pre_s, dec_s = dev.generate(prompt, n_new)
    dev.use_batched_prefill(False)
    _, pre_tt_s, _ = dev.generate(prompt, 1)
    rb = dev.resident_bytes()
    dev.close()
    if shared is not None:
        shared.free()
    tok_s = n_new / dec_s
    wbytes = synth.model_bytes(cfg, mix)
    E = cfg["embed_dim"]
    kv_dim = cfg["n_kv_heads"] * (E // cfg["n_heads"])
    mean_pos = n_prompt + (n_new + 1) / 2
    kv_bytes = 2 * cfg["n_layers"] * mean_pos * kv_dim * 4
    per_tok = wbytes + kv_bytes
    log(f"decode {arch} {mix}: {tok_s:.1f} tok/s ({dec_s * 1e3 / n_new:.3f} ms/token), "
        f"{per_tok / 1e9:.3f} GB/token -> {per_tok * tok_s / 1e9:.1f} GB/s; prefill "
        f"{n_prompt / pre_s:.1f} tok/s (token by token {n_prompt / pre_tt_s:.1f}); set-up {setup_s:.1f} s; "
        f"weights resident {rb['weights'] / 1e9:.3f} GB = {rb['weights'] / rb['file_bytes']:.4f} x the file's "
        f"{rb['file_bytes'] / 1e9:.3f} GB, device total {rb['total'] / 1e9:.3f} GB")
    return {"model": f"{arch} ({mix}, random init, synthetic)",
            "prompt_tokens": n_prompt, "decode_tokens": n_new,
            "tok_s": round(tok_s, 2), "ms_per_token": round(dec_s * 1e3 / n_new, 4),
            "prefill_tok_s": round(n_prompt / pre_s, 2),
            "prefill_token_by_token_tok_s": round(n_prompt / pre_tt_s, 2),
            "bytes_per_token": int(per_tok), "weight_bytes_per_token": int(wbytes),
            "achieved_GBs": round(per_tok * tok_s / 1e9, 2),
            "frac_of_8TBs": round(per_tok * tok_s / 8e12, 4),
            "resident_weight_bytes": rb["weights"], "file_weight_bytes": rb["file_bytes"],
            "resident_over_file": round(rb["weights"] / rb["file_bytes"], 4),
            "resident_total_bytes": rb["total"],
            "first_tokens": [int(v) for v in toks[:8]]}


def _event_loop(torch, st, fn, n, warmup):
    """Wall ms of n back-to-back calls fn(i) on stream st, HIP events on st."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(n):
        fn(i)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


CEIL_THREADS = (256, 512, 1024)
CEIL_LOADS = (1, 2, 4, 8)
CEIL_WGS = (0, 256, 512, 1024, 2048, 4096)          # 0: one round over a full grid


def ceiling_run(rinf, ctx, torch, sizes, rotate_min=1 << 30, wave_rows=None):
    """Streaming-read ceiling at each byte count: every read design of
    libqgprobe.so's qgp_read (workgroups of 256/512/1024 threads; 1, 2, 4 or
    8 16-byte loads in flight per thread; a full grid or 256..4096 persistent
    workgroups), for the headline size also gemv_wave's own load pattern
    without its compute (qgp_read_wave_lds: rows G apart, LDS DMA, one step
    of four rows in flight), and torch.sum of a float32 view; each over
    enough rotating copies (>= 1 GiB) that every launch misses the 256 MB
    Infinity Cache, launches issued back to back from C.  ceiling_us is the
    fastest of them all."""
    import ctypes
    probe = rinf.load_probe_library()
    out = {}
    st = torch.cuda.ExternalStream(ctx.stream)
    sp = ctypes.c_void_p(ctx.stream)
    for name, nbytes in sizes:
        nb16 = nbytes // 16 * 16
        ncopy = max(3, -(-rotate_min // nb16))
        bufs = [torch.empty(nb16 // 4, dtype=torch.float32, device="cuda").uniform_() for _ in range(ncopy)]
        arr = (ctypes.c_void_p * ncopy)(*[b.data_ptr() for b in bufs])
        dout = torch.zeros(4, dtype=torch.int32, device="cuda")
        n = 60 if nbytes > 2e8 else 200

        def timed(launch):
            launch(20)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            launch(n)
            e1.record(st)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / n

        designs = []
        for threads in CEIL_THREADS:
            for loads in CEIL_LOADS:
                for wgs in CEIL_WGS:
                    def launch(k, t=threads, w=wgs, l=loads):
                        if probe.qgp_read(arr, ncopy, nb16, dout.data_ptr(), t, w, l, k, sp):
                            raise SystemExit("qgp_read failed")
                    us = timed(launch)
                    designs.append({"threads": threads, "workgroups": wgs or "full grid", "loads": loads,
                                    "us": round(us, 3), "GBs": round(nb16 / us / 1e3, 1)})
        best = min(designs, key=lambda d: d["us"])
        res = {"bytes": nb16, "rotating_copies": ncopy, "launches": n, "designs": designs, "best_read": best}
        cands = [best["us"]]
        if wave_rows and nb16 == wave_rows[0] * wave_rows[1]:
            def launch_w(k):
                if probe.qgp_read_wave_lds(arr, ncopy, wave_rows[0], wave_rows[1], dout.data_ptr(), k, sp):
                    raise SystemExit("qgp_read_wave_lds failed")
            wus = timed(launch_w)
            res["wave_lds_read_us"] = round(wus, 3)
            cands.append(wus)
        cur = torch.cuda.current_stream()
        torch_ms = _event_loop(torch, cur, lambda i: torch.sum(bufs[i % ncopy]), n, 20)
        t_us = torch_ms * 1e3 / n
        res["torch_sum_us"] = round(t_us, 3)
        cands.append(t_us)
        c = min(cands)
        res["ceiling_us"] = round(c, 3)
        res["ceiling_frac_of_8TBs"] = round(nb16 / c / 1e3 / PEAK_GBS, 4)
        del bufs
        torch.cuda.empty_cache()
        out[name] = res
        log(f"ceiling {name}: best plain read {best['us']:.2f} us ({best['GBs']:.0f} GB/s: {best['threads']} "
            f"threads, {best['loads']} loads, {best['workgroups']} workgroups) of {len(designs)} designs"
            + (f"; gemv_wave's load pattern {res['wave_lds_read_us']:.2f} us" if "wave_lds_read_us" in res else "")
            + f"; torch.sum {t_us:.2f} us")
    return out


# per-type GEMVs at Qwen2-0.5B shapes, plus the Q6_K lm_head
SWEEP_TYPES = ("Q8_0", "Q4_0", "Q5_0", "Q5_K", "Q6_K", "F16")
SWEEP_SHAPES = ((896, 896), (128, 896), (896, 4864))


def sweep_run(rinf, synth, ctx, torch, rotate_mb=256, max_copies=256, steps=200):
    """Per-type GEMV time at the configs[1] shapes: back-to-back launches
    issued from C over rotating copies (>= rotate_mb MiB, at most max_copies
    copies: the small shapes stay within the caches), HIP events around the
    loop.  A launch of these small kernels costs about as much as the kernel:
    the µs here are launch-inclusive, rocprofv3's kernel durations are the
    kernels alone (profiles/)."""
    import numpy as np
    entries = []
    st = torch.cuda.ExternalStream(ctx.stream)
    cases = [(t, r, c) for t in SWEEP_TYPES for r, c in SWEEP_SHAPES] + [("Q6_K", 151936, 896)]
    for tname, rows, cols in cases:
        dtype = rinf.TYPE_IDS[tname]
        nb = rinf.nbytes_for(dtype, rows, cols)
        ncopy = int(min(max_copies, max(2, -(-rotate_mb * 2**20 // nb))))
        raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(1))
        x = synth.gen_x(cols, synth.config_seed(1))
        mats = [ctx.upload(raw, dtype, rows, cols) for _ in range(ncopy)]
        dx = torch.from_numpy(x).cuda()
        dy = torch.zeros(rows, dtype=torch.float32, device="cuda")
        n = steps if nb < 1e8 else 60
        # launches issued back to back from C (qg_matvec_dev_repeat): a Python
        # launch costs more than these kernels take
        ctx.matvec_repeat(mats, dx, dy, 20, ctx.stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        ctx.matvec_repeat(mats, dx, dy, n, ctx.stream)
        e1.record(st)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        B = alg_bytes(rinf, dtype, rows, cols)
        kind = {0: "generic", 1: "stream", 2: "ring", 3: "wave"}.get(mats[0].kernel_kind, "?")
        entries.append({"type": tname, "rows": rows, "cols": cols, "us": round(us, 3),
                        "GBs": round(B / us / 1e3, 1), "frac_of_8TBs": round(B / us / 1e3 / PEAK_GBS, 4),
                        "alg_bytes": B, "rotating_bytes": ncopy * nb, "kernel": kind})
        log(f"sweep {tname} {rows}x{cols}: {us:.2f} us, {B / us / 1e3:.0f} GB/s ({kind}, {ncopy} copies)")
        if not np.all(np.isfinite(dy.cpu().numpy())):
            raise SystemExit(f"sweep {tname} {rows}x{cols}: non-finite output")
        for m in mats:
            m.free()
        del dx, dy
    return entries


def shape_run(rinf, synth, ctx, torch, tname, rows, cols, steps, warmup, rotate_mb=512):
    """One more GEMV shape timed like the headline (time_gemv: the better of
    the C loop, eager and graph launches over >= rotate_mb MiB of rotating
    copies), e.g. configs[4]'s Q4_K 14336 x 4096."""
    import numpy as np
    dtype = rinf.TYPE_IDS[tname]
    nb = rinf.nbytes_for(dtype, rows, cols)
    ncopy = max(2, -(-rotate_mb * 2**20 // nb))
    raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(4))
    x = synth.gen_x(cols, synth.config_seed(4))
    mats = [ctx.upload(raw, dtype, rows, cols) for _ in range(ncopy)]
    dx = torch.from_numpy(x).cuda()
    dy = torch.zeros(rows, dtype=torch.float32, device="cuda")
    c_ms, eager_ms, graph_ms, _ = time_gemv(ctx, torch, mats, dx, dy, steps, warmup)
    us = min(c_ms, eager_ms, graph_ms) * 1e3 / steps
    B = alg_bytes(rinf, dtype, rows, cols)
    kind = {1: "gemv_stream", 2: "gemv_ring", 3: "gemv_wave"}.get(mats[0].kernel_kind, "gemv_generic")
    if not np.all(np.isfinite(dy.cpu().numpy())):
        raise SystemExit(f"{tname} {rows}x{cols}: non-finite output")
    for m in mats:
        m.free()
    log(f"{tname} {rows}x{cols}: {us:.2f} us per GEMV, {B / us / 1e3:.0f} GB/s ({kind})")
    return {"type": tname, "rows": rows, "cols": cols, "us": round(us, 3), "GBs": round(B / us / 1e3, 1),
            "frac_of_8TBs": round(B / us / 1e3 / PEAK_GBS, 4), "alg_bytes": B, "kernel": kind,
            "rotating_copies": ncopy, "us_c_loop": round(c_ms * 1e3 / steps, 3),
            "us_eager": round(eager_ms * 1e3 / steps, 3), "us_graph": round(graph_ms * 1e3 / steps, 3)}


def timeline_run(rinf, synth, args):
    """s_memrealtime stamps of one GEMV kernel from libqgemv_timeline.so: the
    wave-private or LDS-ring GEMV the shape plans, or with --timeline-glu the
    stream kernel's [gate; up] form
    (RMSNorm prologue, silu(gate) * up) on a matrix of 2 * hidden rows.  Per
    event, the median over workgroups of (stamp - first entry stamp), for the
    last of 20 back-to-back launches over rotating copies, over `reps`
    repetitions (the median of the per-repetition medians)."""
    import ctypes
    import numpy as np
    import torch
    lib = rinf.use_library(ROOT / "rust-inference_amd" / "libqgemv_timeline.so")
    lib.qg_timeline_read.restype = ctypes.c_int
    lib.qg_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)]
    lib.qg_timeline_clear.restype = ctypes.c_int
    glu = args.timeline_glu
    dtype = rinf.TYPE_IDS[args.type]
    rows, cols = args.rows, args.cols
    nb = rinf.nbytes_for(dtype, rows, cols)
    ncopy = max(2, -(-args.rotate_mb * 2**20 // nb))
    ctx = rinf.GpuContext(0)
    raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(4))
    x = synth.gen_x(cols, synth.config_seed(4))
    mats = [ctx.upload(raw, dtype, rows, cols) for _ in range(ncopy)]
    kind = mats[0].kernel_kind
    mode = "glu" if glu else {2: "ring", 3: "wave"}.get(kind)
    if mode is None or (glu and (kind not in (1, 2, 3) or rows % 2)):
        raise SystemExit(f"{args.type} {rows}x{cols} (kernel kind {kind}) has no "
                         f"{'stream-kernel [gate; up]' if glu else 'LDS-ring or wave-private'} timeline")
    dx = torch.from_numpy(x).cuda()
    dy = torch.zeros(rows, dtype=torch.float32, device="cuda")
    if glu:
        dxb = torch.from_numpy(synth.gen_x(cols, synth.config_seed(5))).cuda()
        dnw = torch.ones(cols, dtype=torch.float32, device="cuda")
        launch = lambda m: m.matvec_norm_glu_dev(dx, dxb, dnw, 1e-6, dy, None, ctx.stream)
        names = {0: "wave 0: entry", 1: "wave 0: x loads issued", 2: "wave 0: first weight batches issued",
                 3: "wave 0: x staged as planes", 4: "wave 0: workgroup barrier passed",
                 5: "wave 0: x slice in registers", 31: "wave 0: end"}
        for i in range(25):
            names[6 + i] = f"wave 0: batch {i} done"
        first = list(range(48, 64))                       # every wave's entry
        end_ev = 31
    elif mode == "wave":
        launch = lambda m: m.matvec_dev(dx, dy, ctx.stream)
        names = {0: "wave 0: entry", 1: "wave 0: x and rows 0-3 requested", 2: "wave 0: x landed",
                 3: "wave 0: x converted (in registers)", 12: "wave 0: workgroup barrier passed",
                 13: "wave 0: y written (end)"}
        for i in range(4):
            names[4 + 2 * i] = f"wave 0: step {i} landed (rows {4 * i}-{4 * i + 3})"
            names[5 + 2 * i] = f"wave 0: step {i} computed"
        first = list(range(48, 56))                       # the 8 waves' entries
        end_ev = 13
    else:
        launch = lambda m: m.matvec_dev(dx, dy, ctx.stream)
        names = {0: "compute: entry", 1: "compute: x arrived", 2: "compute: x converted",
                 3: "compute: planes published", 30: "compute: last stage done", 31: "compute: y written (end)",
                 32: "loader: entry", 33: "loader: first stages issued", 34: "loader: planes published",
                 63: "loader: end"}
        for i in range(13):
            names[4 + 2 * i] = f"compute: stage {i} reached"
            names[5 + 2 * i] = f"compute: stage {i} published"
        for i in range(28):
            names[35 + i] = f"loader: stage {i} landed"
        first = [32]
        end_ev = 31
    n_ev, n_wg = 64, 2048
    buf = np.zeros(n_ev * n_wg, np.uint64)
    khz = ctypes.c_int(0)
    per_rep, wave_end = [], []
    for rep in range(args.timeline_reps):
        for i in range(20):
            launch(mats[(rep * 20 + i) % ncopy])
        ctx.synchronize()
        if lib.qg_timeline_read(buf.ctypes.data, buf.size, ctypes.byref(khz)):
            raise SystemExit("qg_timeline_read failed")
        t = buf.reshape(n_wg, n_ev).astype(np.int64)
        wg = [w for w in range(n_wg) if t[w, 0] and t[w, end_ev]]
        t = t[wg]
        starts = t[:, [0] + first]
        t0 = starts[starts != 0].min()
        us = (t - t0) / (khz.value / 1e3)
        med = {}
        for e in names:
            col = us[:, e][t[:, e] != 0]
            if col.size:
                med[e] = (float(np.median(col)), float(np.percentile(col, 10)), float(np.percentile(col, 90)))
        if mode in ("glu", "wave"):
            ends = np.where(t[:, 32:48] != 0, us[:, 32:48], np.nan)
            nw = int((~np.isnan(ends)).any(axis=0).sum())
            wave_end.append([float(np.nanmedian(ends[:, w])) for w in range(nw)] + [float(np.nanmax(ends))])
            med["end_max"] = (float(np.nanmax(ends)),) * 3
        else:
            med["end_max"] = (float(us[:, 31].max()),) * 3
        per_rep.append(med)
    table = []
    for e in sorted(k for k in per_rep[0] if isinstance(k, int)):
        vals = [r[e] for r in per_rep if e in r]
        table.append({"event": names[e], "median_us": round(float(np.median([v[0] for v in vals])), 3),
                      "p10_us": round(float(np.median([v[1] for v in vals])), 3),
                      "p90_us": round(float(np.median([v[2] for v in vals])), 3)})
    end_max = float(np.median([r["end_max"][0] for r in per_rep]))
    for m in mats:
        m.free()
    ctx.close()
    kernel = {"glu": "qg::gemv_stream, [gate; up] form", "ring": "qg::gemv_ring",
              "wave": "qg::gemv_wave"}[mode] + " (timeline build)"
    res = {"workload": f"{args.type.lower()}_gemv{'_glu' if glu else ''}_{rows}x{cols}", "kernel": kernel,
           "workgroups": len(wg), "clock_khz": khz.value, "reps": args.timeline_reps,
           "last_wave_end_us" if mode != "ring" else "last_workgroup_end_us": round(end_max, 3), "events": table}
    for r in table:
        log(f"{r['event']:44s} {r['median_us']:8.3f} us  (p10 {r['p10_us']:.3f}, p90 {r['p90_us']:.3f})")
    if mode in ("glu", "wave"):
        we = np.median(np.array(wave_end), axis=0)
        res["wave_end_median_us"] = [round(float(v), 3) for v in we[:-1]]
        log("per wave index, median end over workgroups: " + " ".join(f"{v:.2f}" for v in we[:-1]) + " us")
        log(f"last wave ends at {end_max:.3f} us after the first entry")
    else:
        log(f"last workgroup ends at {end_max:.3f} us after the first entry")
    print(json.dumps(res), flush=True)


def _pmc_rows(d):
    """(kernel name, counter value in KiB, grid size) of every dispatch in a rocprofv3 run."""
    import csv
    out = []
    for f in sorted(pathlib.Path(d).rglob("*counter_collection.csv")):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                out.append((r["Kernel_Name"], float(r["Counter_Value"]), int(r["Grid_Size"])))
    return out


def trace_summary(args):
    """Markdown table of a rocprofv3 --kernel-trace run: consecutive dispatches
    of one kernel with one launch shape form a run (e.g. one read design of
    the ceiling sweep at one size, or the GEMV's timed loop); per run the
    dispatch count and the mean / median / min duration.  Runs shorter than
    --trace-min-calls dispatches are left out."""
    import csv
    rows = []
    for f in sorted(pathlib.Path(args.trace_summary).rglob("*kernel_trace.csv")):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                rows.append((int(r["Start_Timestamp"]), r["Kernel_Name"], int(r["Workgroup_Size_X"]),
                             int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])),
                             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    rows.sort()
    runs = []
    for t, name, wg, grid, us in rows:
        if runs and runs[-1][0] == (name, wg, grid):
            runs[-1][1].append(us)
        else:
            runs.append([(name, wg, grid), [us]])
    pat = args.trace_filter
    print("| run | kernel | workgroup | workgroups | dispatches | mean us | median us | min us |")
    print("|---:|---|---:|---:|---:|---:|---:|---:|")
    for i, ((name, wg, grid), d) in enumerate(runs):
        if len(d) < args.trace_min_calls or (pat and pat not in name):
            continue
        short = name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        print(f"| {i} | `{short}` | {wg} | {grid} | {len(d)} | {statistics.mean(d):.3f} | "
              f"{statistics.median(d):.3f} | {min(d):.3f} |")


def pmc_summary(args):
    """profiles/traffic.json from a FETCH_SIZE run and a WRITE_SIZE run of
    `bench.py ... --copy-probe-mb M`.  Both counters report KiB per dispatch;
    the copy kernel moves exactly M MiB each way, so its readings give the
    factor that turns the counters into bytes."""
    res = {}
    for key, d in (("fetch", args.pmc_summary[0]), ("write", args.pmc_summary[1])):
        rows = _pmc_rows(d)
        gemv = [v for k, v, _ in rows if "qg::gemv_" in k]
        copy = [v for k, v, _ in rows if "elementwise" in k.lower() and "mul" in k.lower()]
        if not gemv or not copy:
            raise SystemExit(f"{d}: no gemv or no copy-probe dispatches found")
        res[key] = (statistics.median(gemv), statistics.median(copy), len(gemv), len(copy))
    ideal_kib = args.copy_probe_mb * 1024
    f_scale = ideal_kib / res["fetch"][1]
    w_scale = ideal_kib / res["write"][1]
    fetch_b = res["fetch"][0] * f_scale * 1024
    write_b = res["write"][0] * w_scale * 1024
    import __graft_entry__ as ge
    rinf = ge.load_package()
    dtype = rinf.TYPE_IDS[args.type]
    alg = alg_bytes(rinf, dtype, args.rows, args.cols)
    workload = f"{args.type.lower()}_gemv_{args.rows}x{args.cols}"
    tf = ROOT / "profiles" / "traffic.json"
    data = json.loads(tf.read_text()) if tf.exists() else {}
    data[workload] = {
        "hbm_bytes_per_launch": int(round(fetch_b + write_b)),
        "fetch_bytes": int(round(fetch_b)), "write_bytes": int(round(write_b)),
        "algorithmic_bytes": alg, "traffic_over_algorithmic": round((fetch_b + write_b) / alg, 4),
        "raw_fetch_kib_median": res["fetch"][0], "raw_write_kib_median": res["write"][0],
        "copy_probe_mib": args.copy_probe_mb,
        "copy_fetch_kib_median": res["fetch"][1], "copy_write_kib_median": res["write"][1],
        "fetch_scale": round(f_scale, 5), "write_scale": round(w_scale, 5),
        "dispatches": {"gemv_fetch": res["fetch"][2], "gemv_write": res["write"][2]},
    }
    tf.parent.mkdir(exist_ok=True)
    tf.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    print(json.dumps(data[workload], indent=1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--rows", type=int, default=4096)
    ap.add_argument("--cols", type=int, default=14336)
    ap.add_argument("--type", default="Q4_K")
    ap.add_argument("--rotate-mb", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode", default="qwen2-7b",
                    help="architecture of the synthetic decode run (synth.ARCH key; 'none' skips it)")
    ap.add_argument("--decode-mix", default="q4_k_m")
    ap.add_argument("--decode-prompt", type=int, default=64)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the decode leg (prints its JSON object)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="after timing, run 4 elementwise copies (y = 1.0 * x) of this many MiB: the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc runs of this script (FETCH_SIZE, then "
                         "WRITE_SIZE, each with --copy-probe-mb) into profiles/traffic.json")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print a markdown table of the kernel runs in a rocprofv3 --kernel-trace output dir")
    ap.add_argument("--trace-filter", default="", help="with --trace-summary: kernels whose name contains this")
    ap.add_argument("--trace-min-calls", type=int, default=20)
    ap.add_argument("--no-ceiling", action="store_true", help="skip the streaming-read ceiling leg")
    ap.add_argument("--no-sweep", action="store_true", help="skip the configs[1] per-type sweep")
    ap.add_argument("--no-decode-configs", action="store_true",
                    help="skip the configs[2] / configs[4] decode runs")
    ap.add_argument("--timeline", action="store_true",
                    help="only the s_memrealtime timeline of the planned wave-private or LDS-ring GEMV "
                         "(libqgemv_timeline.so)")
    ap.add_argument("--timeline-reps", type=int, default=9)
    ap.add_argument("--timeline-glu", action="store_true",
                    help="with --timeline: the stream kernel's [gate; up] form instead")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args)
        return
    if args.pmc_summary:
        pmc_summary(args)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the row-sharded multi-GPU GEMV is a design note, not "
              "a measured path", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__ as ge
    rinf = ge.load_package()
    synth = importlib.import_module(ge.PKG_NAME + ".synth")
    if args.timeline:
        timeline_run(rinf, synth, args)
        return
    dtype = rinf.TYPE_IDS[args.type]
    rows, cols = args.rows, args.cols
    nb = rinf.nbytes_for(dtype, rows, cols)
    B = alg_bytes(rinf, dtype, rows, cols)
    ncopy = max(2, -(-args.rotate_mb * 2**20 // nb))

    ctx = rinf.GpuContext(0)
    if args.decode_only:
        print(json.dumps(decode_run(rinf, synth, ctx, args)), flush=True)
        ctx.close()
        return
    log(f"device CUs={ctx.cu_count}; {args.type} {rows}x{cols}: {nb} weight bytes, "
        f"{B} algorithmic bytes/launch, {ncopy} rotating copies ({ncopy * nb / 2**20:.0f} MiB)")
    raw = synth.gen_blocks(dtype, rows, cols, synth.config_seed(4))
    x = synth.gen_x(cols, synth.config_seed(4))
    mats = [ctx.upload(raw, dtype, rows, cols) for _ in range(ncopy)]
    kernel = {1: "qg::gemv_stream", 2: "qg::gemv_ring", 3: "qg::gemv_wave"}.get(mats[0].kernel_kind, "qg::gemv_generic")
    dx = torch.from_numpy(x).cuda()
    dy = torch.zeros(rows, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    c_ms, eager_ms, graph_ms, per = time_gemv(ctx, torch, mats, dx, dy, args.steps, args.warmup)
    wall_ms = min(c_ms, eager_ms, graph_ms)
    ms_step = wall_ms / args.steps
    value = B / (ms_step * 1e-3) / 1e9
    # average launch duration: HIP events on the launch stream around the
    # back-to-back loops, the fastest of the C loop, Python eager and graph
    # replay (a profiler's callbacks inflate the eager ones); it includes the
    # gaps between kernels, so it is an upper bound on rocprofv3's per-kernel
    # average
    kern_ms = wall_ms / args.steps
    achieved = B / (kern_ms * 1e-3) / 1e9
    log(f"C loop {c_ms / args.steps * 1e3:.2f} us/step, Python eager {eager_ms / args.steps * 1e3:.2f} us/step, "
        f"graph {graph_ms / args.steps * 1e3:.2f} us/step")
    log(f"wall {wall_ms:.3f} ms / {args.steps} launches = {ms_step * 1e3:.2f} us/step -> "
        f"{value:.1f} GB/s; kernel {kern_ms * 1e3:.2f} us -> {achieved:.1f} GB/s "
        f"({achieved / PEAK_GBS:.1%} of 8 TB/s); isolated launches with event pairs: median "
        f"{statistics.median(per) * 1e3:.2f} us")
    if args.copy_probe_mb > 0:
        n = args.copy_probe_mb * 2**20 // 4
        a = torch.ones(n, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(4):
            torch.mul(a, 1.0, out=b)                    # elementwise: reads M MiB, writes M MiB
        torch.cuda.synchronize()
        del a, b

    # consistency of the measured launches (parity itself is tests/test_gemv_gpu.py):
    # every copy holds the same bytes, so two launches on different copies
    # must give bit-identical, finite outputs
    y = dy.cpu().numpy().copy()
    mats[1].matvec_dev(dx, dy, ctx.stream)
    ctx.synchronize()
    if not (np.all(np.isfinite(y)) and np.array_equal(y.view(np.uint32), dy.cpu().numpy().view(np.uint32))):
        raise SystemExit("measured launches disagree or are not finite")
    oracle = None
    if not args.no_cpu_baseline:
        try:
            oracle = ge.load_oracle()
        except ImportError as e:
            log(f"oracle not built ({e}); cpu_baseline skipped")

    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    workload = f"{args.type.lower()}_gemv_{rows}x{cols}"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get(workload, {}).get("hbm_bytes_per_launch")

    cpu = None
    if oracle is not None and not args.no_cpu_baseline:
        cpu = cpu_baseline(oracle, raw, dtype, rows, cols, x, args.cpu_seconds, B)
        log(f"cpu_baseline: {cpu['value']} GB/s ({cpu['us_per_gemv']} us/GEMV)")

    ceiling = None
    if not args.no_ceiling:
        wave_rows = (rows, nb // rows) if mats[0].kernel_kind == 3 else None
        ceiling = ceiling_run(rinf, ctx, torch, [(workload, nb), ("qwen2_7b_gate_up_76MB", 76382208),
                                                 ("qwen2_7b_lm_head_447MB", 447166464)], wave_rows=wave_rows)

    # configs[4]'s other standalone shape (the headline is 4096 x 14336)
    other_shape = None
    if (args.type, rows, cols) == ("Q4_K", 4096, 14336):
        other_shape = shape_run(rinf, synth, ctx, torch, "Q4_K", 14336, 4096, args.steps, args.warmup)

    decode = None
    if args.decode != "none":
        decode = decode_run(rinf, synth, ctx, args)

    sweep = None if args.no_sweep else sweep_run(rinf, synth, ctx, torch)
    decode_configs = None
    if not args.no_decode_configs and args.decode != "none":
        decode_configs = {
            "configs[2] qwen2-0.5b q4_k_m 32+128": decode_run(rinf, synth, ctx, args, "qwen2-0.5b", "q4_k_m", 32, 128, 2),
            "configs[4] llama3-8b q4_k_m 64+512": decode_run(rinf, synth, ctx, args, "llama3-8b", "q4_k_m", 64, 512, 4),
            "configs[4] llama3-8b q5_k 64+512": decode_run(rinf, synth, ctx, args, "llama3-8b", "q5_k", 64, 512, 4),
            "configs[4] llama3-8b q8_0 64+512": decode_run(rinf, synth, ctx, args, "llama3-8b", "q8_0", 64, 512, 4),
        }

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "compute": "int8 dot4 of weight codes with x as 22-bit fixed point per 32-element segment "
                   "(three signed-byte digit planes), exact int32 sums, f32 scales and accumulation",
        "data": "synthetic (seeded GGUF blocks: f16 scales U[1e-3,2e-2], uniform code bytes; x ~ N(0,1))",
        "config": {"workload": workload, "type": args.type, "rows": rows, "cols": cols,
                   "bytes_per_launch": B, "rotating_copies": ncopy,
                   "launch": {c_ms: "c_loop", eager_ms: "eager", graph_ms: "hip_graph"}[wall_ms],
                   "us_per_step_c_loop": round(c_ms / args.steps * 1e3, 3),
                   "us_per_step_eager": round(eager_ms / args.steps * 1e3, 3),
                   "us_per_step_graph": round(graph_ms / args.steps * 1e3, 3),
                   "frac_of_8TBs_wall": round(value / PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "event_us_per_launch": round(kern_ms * 1e3, 3),
                     "kernel": kernel + " (rust-inference_amd/csrc/qgemv_kernels.hip)"},
        "cpu_baseline": cpu,
        "decode": decode,
        "ceiling": ceiling,
        "q4_k_gemv_14336x4096": other_shape,
        "sweep": sweep,
        "decode_configs": decode_configs,
    }
    if ceiling:
        c = ceiling[workload]
        out["roofline"]["ceiling_us"] = c["ceiling_us"]
        out["roofline"]["ceiling_frac"] = c["ceiling_frac_of_8TBs"]
        out["roofline"]["frac_of_ceiling"] = round(c["ceiling_us"] / (kern_ms * 1e3), 4)
    for m in mats:
        m.free()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
