"""Seeded synthetic GGUF blocks and activations (numpy).

Inputs for every parity test and for bench.py, generated the same way on the
CPU container and on the GPU box:

* f16 scale fields (Q4_K/Q5_K d and dmin, Q6_K d, Q8_0/Q4_0/Q5_0 d) are
  f16(U[1e-3, 2e-2]);
* every other byte (6-bit scale/min packs, nibbles, high bits, Q6_K int8
  sub-block scales, Q8_0 int8 codes) is uniform over 0..255;
* F16 weights are f16(N(0,1) * 0.02) and F32 weights N(0,1) * 0.02 (finite);
* x is f32 N(0,1).

Field offsets inside a block follow src/quant.rs:106-292.
"""
from __future__ import annotations

import numpy as np

# (block elements, block bytes, byte offsets of f16 scale fields)
LAYOUT = {
    0: (1, 4, ()),           # F32
    1: (1, 2, ()),           # F16
    2: (32, 18, (0,)),       # Q4_0: d
    6: (32, 22, (0,)),       # Q5_0: d
    8: (32, 34, (0,)),       # Q8_0: d
    12: (256, 144, (0, 2)),  # Q4_K: d, dmin
    13: (256, 176, (0, 2)),  # Q5_K: d, dmin
    14: (256, 210, (208,)),  # Q6_K: d
}


def n_blocks(dtype: int, rows: int, cols: int) -> int:
    bs = LAYOUT[dtype][0]
    return -(-(rows * cols) // bs)


def gen_blocks(dtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Raw bytes of a rows x cols matrix of `dtype` (flat uint8 array)."""
    bs, bb, f16_offs = LAYOUT[dtype]
    nb = n_blocks(dtype, rows, cols)
    rng = np.random.default_rng(seed)
    if dtype == 0:
        return (rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).view(np.uint8)
    if dtype == 1:
        w = (rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
        return w.view(np.uint8)
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    for off in f16_offs:
        d = rng.uniform(1e-3, 2e-2, size=nb).astype(np.float16)
        raw[:, off:off + 2] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def gen_x(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed ^ 0x5A5A5A5A).standard_normal(n, dtype=np.float32)


def config_seed(index: int) -> int:
    """Seed of BASELINE.json config `index` (0-based)."""
    return 0x5EED0000 + index


def _f16(v) -> np.ndarray:
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint8)


def _pack_k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """The 12-byte 6-bit scale/min pack of Q4_K/Q5_K (the inverse of
    get_scale_min_k4, quant.rs:606-615) for (nb, 8) arrays of 0..63."""
    q = np.zeros((sc.shape[0], 12), np.uint8)
    q[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    q[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    q[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return q


def gen_weights(dtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Raw bytes of a random-init weight matrix: dequantized values centred on
    zero with standard deviation about 1/sqrt(cols), so that every mat-vec of
    a normalised input stays O(1) through any number of layers (the uniform
    bytes of gen_blocks have a positive mean of about 2 per weight: a model
    built from them grows activations to 1e7..1e10 and one-hot attention, where
    the reference's own f32 path is 4e-3 away from exact).  Codes stay uniform
    over their bit range; the scale fields carry the magnitude and the centring:
      Q4_K/Q5_K: sub-block scales sc in 1..15, mins m = sc, dmin = f16(c * d)
                 with c the codes' mean (7.5 / 15.5), so each sub-block is
                 d * sc * (q - c);
      Q6_K: int8 sub-block scales in -8..7; Q8_0/Q4_0/Q5_0: as in the format;
      every block's d (and dmin with it) gets a random sign;
      F16/F32: N(0, 1/cols)."""
    bs, bb, _ = LAYOUT[dtype]
    nb = n_blocks(dtype, rows, cols)
    rng = np.random.default_rng(seed)
    sigma = 1.0 / np.sqrt(max(cols, 1))
    if dtype in (0, 1):
        w = rng.standard_normal(nb, dtype=np.float32) * np.float32(sigma)
        return (w if dtype == 0 else w.astype(np.float16)).view(np.uint8)
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    # a random sign per block cancels the -d/2 mean of the unsigned codes
    jitter = rng.uniform(0.75, 1.25, size=nb) * rng.choice([-1.0, 1.0], size=nb)
    if dtype in (12, 13):                       # Q4_K, Q5_K
        c, code_sd = (7.5, 4.61) if dtype == 12 else (15.5, 9.23)
        sc = rng.integers(1, 16, size=(nb, 8), dtype=np.uint8)
        d = sigma / (8.8 * code_sd) * jitter
        raw[:, 0:2] = _f16(d).reshape(nb, 2)
        raw[:, 2:4] = _f16(c * np.asarray(d, np.float16).astype(np.float64)).reshape(nb, 2)
        raw[:, 4:16] = _pack_k_scales(sc, sc)
    elif dtype == 14:                           # Q6_K: w = d * sc * (q - 32)
        raw[:, 192:208] = rng.integers(-8, 8, size=(nb, 16)).astype(np.int8).view(np.uint8)
        raw[:, 208:210] = _f16(sigma / (4.6 * 18.5) * jitter).reshape(nb, 2)
    else:                                       # Q8_0 d*q, Q4_0 d*(q-8), Q5_0 d*(q-16)
        code_sd = {8: 73.9, 2: 4.61, 6: 9.23}[dtype]
        raw[:, 0:2] = _f16(sigma / code_sd * jitter).reshape(nb, 2)
    return raw.reshape(-1)


# ------------------------------------------------------------ whole models
#
# random-init models of a named architecture in a
# GGUF quantization mix.  Q4_K_M: attn_v and ffn_down Q6_K, every other
# matrix Q4_K; the lm_head is Q6_K unless it is tied to token_embd.  Weight
# matrices come from gen_weights (centred, ~1/sqrt(cols)); RMSNorm weights
# are f32 1 + N(0, 0.02); q/k/v biases f32 N(0, 0.02).

ARCH = {
    # embed, layers, heads, kv heads, ffn, vocab, rope base, tied lm_head
    "qwen2-0.5b": dict(embed_dim=896, n_layers=24, n_heads=14, n_kv_heads=2, hidden_dim=4864,
                       vocab_size=151936, rope_base=1e6, norm_eps=1e-6, tied=True, bias=True),
    "qwen2-7b": dict(embed_dim=3584, n_layers=28, n_heads=28, n_kv_heads=4, hidden_dim=18944,
                     vocab_size=152064, rope_base=1e6, norm_eps=1e-6, tied=False, bias=True),
    "llama3-8b": dict(embed_dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, hidden_dim=14336,
                      vocab_size=128256, rope_base=5e5, norm_eps=1e-5, tied=False, bias=False),
}

MIXES = {
    # slot -> GGML type; "base" covers every matrix not listed
    "q4_k_m": dict(base=12, wv=14, down=14, lm_head=14),
    "q5_k": dict(base=13, lm_head=14),
    "q5_k_m": dict(base=13, wv=14, down=14, lm_head=14),
    "q8_0": dict(base=8, lm_head=8),
    "f16": dict(base=1, lm_head=1),          # no fused-norm kernel: separate RMSNorm path
}

SLOTS = ("token_embd", "lm_head", "wq", "wk", "wv", "wo", "gate", "up", "down")


def slot_shape(cfg: dict, slot: str):
    """(rows, cols) of a matrix slot (src/model.rs:197-298: rows = ne1 = out)."""
    E, H, V = cfg["embed_dim"], cfg["hidden_dim"], cfg["vocab_size"]
    hd = E // cfg["n_heads"]
    q_dim, kv_dim = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    return {"token_embd": (V, E), "lm_head": (V, E), "wq": (q_dim, E), "wk": (kv_dim, E),
            "wv": (kv_dim, E), "wo": (E, q_dim), "gate": (H, E), "up": (H, E), "down": (E, H)}[slot]


def gen_model(cfg: dict, mix: str = "q4_k_m", seed: int = 0):
    """{"mats": {(slot, layer): (raw, dtype, rows, cols)}, "vecs": {(name, layer): f32}}.
    Layer is 0 for token_embd / lm_head / final_norm.  A tied lm_head is absent
    from "mats" (the caller shares token_embd)."""
    m = MIXES[mix]
    rng = np.random.default_rng(seed)
    mats, vecs = {}, {}
    for slot in SLOTS:
        if slot == "lm_head" and cfg.get("tied"):
            continue
        layers = [0] if slot in ("token_embd", "lm_head") else range(cfg["n_layers"])
        rows, cols = slot_shape(cfg, slot)
        dtype = m.get(slot, m["base"])
        for layer in layers:
            s = int(rng.integers(0, 2**31))
            mats[(slot, layer)] = (gen_weights(dtype, rows, cols, s), dtype, rows, cols)
    E = cfg["embed_dim"]
    hd = E // cfg["n_heads"]
    kv_dim = cfg["n_kv_heads"] * hd
    vecs[("final_norm", 0)] = (1.0 + 0.02 * rng.standard_normal(E)).astype(np.float32)
    for layer in range(cfg["n_layers"]):
        vecs[("attn_norm", layer)] = (1.0 + 0.02 * rng.standard_normal(E)).astype(np.float32)
        vecs[("ffn_norm", layer)] = (1.0 + 0.02 * rng.standard_normal(E)).astype(np.float32)
        if cfg.get("bias", True):
            vecs[("bq", layer)] = (0.02 * rng.standard_normal(E)).astype(np.float32)
            vecs[("bk", layer)] = (0.02 * rng.standard_normal(kv_dim)).astype(np.float32)
            vecs[("bv", layer)] = (0.02 * rng.standard_normal(kv_dim)).astype(np.float32)
    return {"mats": mats, "vecs": vecs}


def model_bytes(cfg: dict, mix: str = "q4_k_m") -> int:
    """Quantized weight bytes one decode step reads (tied lm_head read twice)."""
    m = MIXES[mix]
    total = 0
    for slot in SLOTS:
        rows, cols = slot_shape(cfg, slot)
        src = "token_embd" if (slot == "lm_head" and cfg.get("tied")) else slot
        dtype = m.get(src, m["base"])
        bs, bb, _ = LAYOUT[dtype]
        nb = -(-(rows * cols) // bs) * bb
        if slot == "token_embd":
            total += -(-cols // bs) * bb            # one row per token
        elif slot == "lm_head":
            total += nb
        else:
            total += nb * cfg["n_layers"]
    return total
