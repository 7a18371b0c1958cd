"""Writes tests/golden/kat_blocks.json: known-answer blocks for every type.

Each block is built by a hand encoder that places chosen integer codes and
scales at the byte/bit positions the GGUF layouts define (GGML block
layouts; Q4_0 in the reference's interleaved order, src/quant.rs:114-121).
Scales are chosen so that every dequantized value is a small dyadic rational
computed exactly in Python, so the expected values are closed forms that do
not depend on the decoder's rounding or evaluation order.  A decoder that
reads a nibble, a bit or a scale from the wrong place fails these.

Run: python tests/golden/make_kat.py   (deterministic; no reference code used)
"""
from __future__ import annotations

import json
import pathlib
import struct

import numpy as np

OUT = pathlib.Path(__file__).resolve().parent / "kat_blocks.json"


def f16_bits(v: float) -> int:
    return int(np.array([v], np.float16).view(np.uint16)[0])


def pack_k_scales(sc, m):
    """12-byte K-quant scale pack: inverse of get_scale_min_k4."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def q4k_block(d, dmin, sc, m, q):
    qs = [0] * 128
    for p in range(4):
        for l in range(32):
            qs[32 * p + l] = (q[64 * p + l] & 15) | ((q[64 * p + 32 + l] & 15) << 4)
    b = struct.pack("<HH", f16_bits(d), f16_bits(dmin)) + bytes(pack_k_scales(sc, m)) + bytes(qs)
    exp = [d * sc[e // 32] * q[e] - dmin * m[e // 32] for e in range(256)]
    return b, exp


def q5k_block(d, dmin, sc, m, q):
    qs = [0] * 128
    qh = [0] * 32
    for p in range(4):
        for l in range(32):
            qs[32 * p + l] = (q[64 * p + l] & 15) | ((q[64 * p + 32 + l] & 15) << 4)
    for e in range(256):
        j, l = e // 32, e % 32
        qh[l] |= ((q[e] >> 4) & 1) << j
    b = (struct.pack("<HH", f16_bits(d), f16_bits(dmin)) + bytes(pack_k_scales(sc, m))
         + bytes(qh) + bytes(qs))
    exp = [d * sc[e // 32] * q[e] - dmin * m[e // 32] for e in range(256)]
    return b, exp


def q6k_block(d, sc16, q):
    ql = [0] * 128
    qh = [0] * 64
    for e in range(256):
        n, r = e // 128, e % 128
        k, l = r // 32, r % 32
        idx = 64 * n + l + 32 * (k & 1)
        ql[idx] |= (q[e] & 15) << (4 if k >= 2 else 0)
        qh[32 * n + l] |= ((q[e] >> 4) & 3) << (2 * k)
    b = bytes(ql) + bytes(qh) + bytes([s & 0xFF for s in sc16]) + struct.pack("<H", f16_bits(d))
    exp = []
    for e in range(256):
        n, r = e // 128, e % 128
        k, l = r // 32, r % 32
        exp.append(d * sc16[8 * n + l // 16 + 2 * k] * (q[e] - 32))
    return b, exp


def q8_0_block(d, q):
    b = struct.pack("<H", f16_bits(d)) + bytes([v & 0xFF for v in q])
    return b, [d * v for v in q]


def q4_0_block(d, q):
    qs = [0] * 16
    for i in range(32):
        qs[i // 2] |= (q[i] & 15) << (4 * (i % 2))          # interleaved order
    return struct.pack("<H", f16_bits(d)) + bytes(qs), [d * (v - 8) for v in q]


def q5_0_block(d, q):
    qs = [0] * 16
    qh = 0
    for i in range(32):
        if i < 16:
            qs[i] |= q[i] & 15
        else:
            qs[i - 16] |= (q[i] & 15) << 4
        qh |= ((q[i] >> 4) & 1) << i
    return struct.pack("<HI", f16_bits(d), qh) + bytes(qs), [d * (v - 16) for v in q]


def f16_specials():
    bits = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF,
            0x7C00, 0xFC00, 0x3555, 0x1234, 0xC000, 0x0200]
    exp = []
    for h in bits:
        v = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        exp.append(None if np.isnan(v) else (float(v) if np.isfinite(v) else ("inf" if v > 0 else "-inf")))
    return b"".join(struct.pack("<H", h) for h in bits), exp


def main():
    kats = []
    # Q4_K: d = 0.5, dmin = 0.25, distinct scales/mins per sub-block (all 6 bits used)
    sc = [1, 63, 17, 32, 5, 48, 33, 62]
    m = [60, 2, 47, 16, 31, 1, 58, 40]
    q = [(7 * e + e // 32) % 16 for e in range(256)]
    b, e = q4k_block(0.5, 0.25, sc, m, q)
    kats.append({"type": 12, "name": "Q4_K", "raw": b.hex(), "expected": e})
    q5 = [(11 * e + e // 16) % 32 for e in range(256)]
    b, e = q5k_block(0.25, 0.5, sc, m, q5)
    kats.append({"type": 13, "name": "Q5_K", "raw": b.hex(), "expected": e})
    sc16 = [-128, 127, -3, 4, 9, -17, 1, -1, 2, -2, 64, -64, 31, -31, 100, -100]
    q6 = [(13 * e + e // 64) % 64 for e in range(256)]
    b, e = q6k_block(0.125, sc16, q6)
    kats.append({"type": 14, "name": "Q6_K", "raw": b.hex(), "expected": e})
    q8 = [(-128 + 9 * i) if i < 29 else (127 - i) for i in range(32)]
    q8[31] = -128
    b, e = q8_0_block(0.5, q8)
    kats.append({"type": 8, "name": "Q8_0", "raw": b.hex(), "expected": e})
    q4 = [(5 * i + 3) % 16 for i in range(32)]
    b, e = q4_0_block(2.0, q4)
    kats.append({"type": 2, "name": "Q4_0", "raw": b.hex(), "expected": e})
    # the source-only quirk pinned explicitly: byte 0x21 -> elements [1-8, 2-8]
    b, e = q4_0_block(1.0, [1, 2] + [8] * 30)
    assert b[2] == 0x21
    kats.append({"type": 2, "name": "Q4_0_interleave_0x21", "raw": b.hex(), "expected": e})
    q5b = [(7 * i + 1) % 32 for i in range(32)]
    b, e = q5_0_block(0.5, q5b)
    kats.append({"type": 6, "name": "Q5_0", "raw": b.hex(), "expected": e})
    b, e = f16_specials()
    kats.append({"type": 1, "name": "F16_specials", "raw": b.hex(), "expected": e})
    OUT.write_text(json.dumps(kats, indent=1))
    print(f"wrote {OUT} ({len(kats)} blocks)")


if __name__ == "__main__":
    main()
