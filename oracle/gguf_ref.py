"""CPU restatement of yudono/rust-inference's GGUF reader and model config.

TEST INFRASTRUCTURE ONLY: the checker for libqgemv's GGUF reader
(include/qggguf.h).  Only tests/ import it.

* parse()          GgufFile::parse (src/gguf.rs:261-341) with read_string
                   (gguf.rs:422-428), read_metadata_value (431-462) and
                   read_metadata_value_by_type (465-485): magic, version 3,
                   counts, key/value pairs (the last of a repeated key wins,
                   HashMap::insert), tensor descriptors (unknown type ids are
                   an error, gguf.rs:310-318), data offset = align_to(pos, 32)
                   (gguf.rs:330, 364-367).
* to_u64 / to_f32  MetadataValue::to_u64 / to_f32 (gguf.rs:171-186).
* model_config()   ModelConfig::from_metadata (src/model.rs:50-117).
* load_bytes()     the byte size Model::load reads per type (model.rs:166-180).
"""
from __future__ import annotations

import struct

MAGIC = 0x46554747
KNOWN_TYPES = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14}       # GgufDataType::from_u32
LOAD_BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 12: (256, 144), 13: (256, 176), 6: (32, 22),
               14: (256, 210), 8: (32, 34)}                       # model.rs:168-175


class GgufError(Exception):
    pass


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.pos = data, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.d):
            raise GgufError("unexpected end of file")
        b = self.d[self.pos:self.pos + n]
        self.pos += n
        return b

    def u(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.u("<Q")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GgufError(f"Invalid UTF-8: {e}")


_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}


def _value_by_type(r: _Reader, t: int):
    if t in _FMT:
        return (t, r.u(_FMT[t]))
    if t == 7:
        return (t, r.u("<B") != 0)
    if t == 8:
        return (t, r.string())
    raise GgufError(f"Unknown metadata array element type: {t}")


def _value(r: _Reader):
    t = r.u("<I")
    if t == 9:
        et, n = r.u("<I"), r.u("<Q")
        return (9, (et, [_value_by_type(r, et) for _ in range(n)]))
    if t in _FMT or t in (7, 8):
        return _value_by_type(r, t)
    raise GgufError(f"Unknown metadata value type: {t}")


def parse(data: bytes) -> dict:
    r = _Reader(data)
    if r.u("<I") != MAGIC:
        raise GgufError("Invalid GGUF magic")
    version = r.u("<I")
    if version != 3:
        raise GgufError(f"Unsupported GGUF version: {version}")
    n_tensors, n_kv = r.u("<Q"), r.u("<Q")
    meta = {}
    for _ in range(n_kv):
        key = r.string()
        meta[key] = _value(r)
    tensors = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.u("<I")
        dims = [r.u("<Q") for _ in range(nd)]
        t = r.u("<I")
        if t not in KNOWN_TYPES:
            raise GgufError(f"Unknown tensor data type: {t}")
        tensors.append({"name": name, "dims": dims, "type": t, "offset": r.u("<Q")})
    data_offset = (r.pos + 31) // 32 * 32
    return {"version": version, "metadata": meta, "tensors": tensors, "data_offset": data_offset}


def to_u64(v):
    if v is None or v[0] not in (10, 11, 4):
        return None
    return v[1] % (1 << 64)


def to_f32(v):
    if v is None or v[0] not in (6, 12):
        return None
    return struct.unpack("<f", struct.pack("<f", v[1]))[0]


def model_config(meta: dict, max_seq_len: int = 0) -> dict:
    arch_v = meta.get("general.architecture")
    arch = arch_v[1] if arch_v is not None and arch_v[0] == 8 else "llama"
    p = arch + "."
    u = lambda k: to_u64(meta.get(p + k)) or 0
    f = lambda k: to_f32(meta.get(p + k)) or 0.0
    e = meta.get(p + "attention.layer_norm_rms_epsilon")
    if e is None:
        e = meta.get(p + "attention.layer_norm_epsilon")
    eps = to_f32(e)
    eps = 1e-5 if eps is None else eps
    defaults = {"qwen2": (3584, 28, 28, 18944, 151936, 1000000.0),
                "llama": (4096, 32, 32, 11008, 32000, 10000.0),
                "mistral": (4096, 32, 32, 14336, 32000, 10000.0)}
    d = defaults.get(arch, (4096, 32, 32, 11008, 32000, 10000.0))
    embed, layers, heads = u("embedding_length") or d[0], u("block_count") or d[1], u("attention.head_count") or d[2]
    kv = u("attention.head_count_kv") or heads
    hidden, vocab = u("feed_forward_length") or d[3], u("vocab_size") or d[4]
    ctx = u("context_length") or 32768
    rope = f("rope.freq_base") or d[5]
    if max_seq_len:
        ctx = max_seq_len
    return {"embed_dim": embed, "n_layers": layers, "n_heads": heads, "n_kv_heads": kv, "hidden_dim": hidden,
            "vocab_size": vocab, "max_seq_len": ctx, "rope_base": struct.unpack("<f", struct.pack("<f", rope))[0],
            "norm_eps": struct.unpack("<f", struct.pack("<f", eps))[0]}


def n_elements(t: dict) -> int:
    n = 1
    for d in t["dims"]:
        n *= d
    return n


def load_bytes(t: dict) -> int:
    if t["type"] not in LOAD_BLOCKS:
        return 0
    bs, bb = LOAD_BLOCKS[t["type"]]
    return (n_elements(t) + bs - 1) // bs * bb
