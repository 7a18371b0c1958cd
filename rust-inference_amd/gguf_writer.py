"""GGUF v3 writer and synthetic model files.

The layout is the one GgufFile::parse reads (src/gguf.rs:261-341): magic
"GGUF", version 3, u64 tensor and metadata counts, the metadata key/value
pairs (length-prefixed UTF-8 keys, u32 type tag, value; arrays as element
type + u64 count + elements), the tensor descriptors (name, u32 n_dims, u64
dims with ne0 first, u32 GGML type, u64 offset relative to the data section),
then the data section at the next multiple of 32 bytes.  Tensor offsets are
multiples of 32 as well.

`write_model` produces files that Model::load accepts (src/model.rs:136-329
and the rules of its tokenizer, tokenizer.rs:110-120): the architecture's
hyper-parameters under "<arch>.", "<arch>.vocab_size", a
"tokenizer.ggml.tokens" string array, F32 norms and biases, the GGUF tensor
names Model::load looks up, and the quantized weights of `synth.gen_model`.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
ALIGN = 32

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, v) for v in items)
    if vtype == BOOL:
        return struct.pack("<B", 1 if value else 0)
    return struct.pack(_SCALAR[vtype], value)


def _pad(n: int) -> int:
    return (ALIGN - n % ALIGN) % ALIGN


def write_gguf(path, metadata, tensors):
    """metadata: [(key, type, value)] (arrays: value = (element type, items));
    tensors: [(name, dims ne0-first, ggml type, raw bytes as a numpy array)]."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for key, vtype, value in metadata:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offset, sizes = 0, []
    for name, dims, ggml_type, raw in tensors:
        nbytes = raw.nbytes
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ggml_type, offset)
        sizes.append(nbytes)
        offset += nbytes + _pad(nbytes)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * _pad(len(head)))
        for (name, dims, ggml_type, raw), nbytes in zip(tensors, sizes):
            b = np.ascontiguousarray(raw).view(np.uint8)
            assert b.nbytes == nbytes, name
            f.write(b.tobytes())
            f.write(b"\0" * _pad(nbytes))


def model_tensors(synth, cfg: dict, mix: str, seed: int):
    """[(GGUF name, dims ne0-first, type, raw)] of synth.gen_model's model,
    named as Model::load looks them up (model.rs:197-298)."""
    t = synth.gen_model(cfg, mix, seed)
    E = cfg["embed_dim"]
    names = {"token_embd": "token_embd.weight", "lm_head": "output.weight"}
    per = {"wq": "attn_q.weight", "wk": "attn_k.weight", "wv": "attn_v.weight", "wo": "attn_output.weight",
           "gate": "ffn_gate.weight", "up": "ffn_up.weight", "down": "ffn_down.weight"}
    vnames = {"attn_norm": "attn_norm.weight", "ffn_norm": "ffn_norm.weight", "bq": "attn_q.bias",
              "bk": "attn_k.bias", "bv": "attn_v.bias"}
    out = []
    for (slot, layer), (raw, dtype, rows, cols) in t["mats"].items():
        name = names.get(slot) or f"blk.{layer}.{per[slot]}"
        out.append((name, [cols, rows], dtype, raw))
    out.append(("output_norm.weight", [E], 0, t["vecs"][("final_norm", 0)]))
    for (vname, layer), v in t["vecs"].items():
        if vname == "final_norm":
            continue
        out.append((f"blk.{layer}.{vnames[vname]}", [v.size], 0, v))
    return out, t


def model_metadata(cfg: dict, arch: str = "qwen2", context_length: int = 4096, n_tokens=None):
    """The keys ModelConfig::from_metadata reads (model.rs:50-117) as UINT32 /
    FLOAT32, plus the tokenizer's vocabulary."""
    V = cfg["vocab_size"]
    p = arch + "."
    return [
        ("general.architecture", STRING, arch),
        ("general.alignment", U32, ALIGN),
        (p + "context_length", U32, context_length),
        (p + "embedding_length", U32, cfg["embed_dim"]),
        (p + "block_count", U32, cfg["n_layers"]),
        (p + "feed_forward_length", U32, cfg["hidden_dim"]),
        (p + "attention.head_count", U32, cfg["n_heads"]),
        (p + "attention.head_count_kv", U32, cfg["n_kv_heads"]),
        (p + "rope.freq_base", F32, cfg["rope_base"]),
        (p + "attention.layer_norm_rms_epsilon", F32, cfg["norm_eps"]),
        (p + "vocab_size", U32, V),
        ("tokenizer.ggml.model", STRING, "gpt2"),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"<t{i}>" for i in range(n_tokens or V)])),
    ]


def write_model(path, synth, cfg: dict, mix: str = "q4_k_m", seed: int = 0, arch: str = "qwen2",
                context_length: int = 4096):
    """A synthetic model file; returns synth.gen_model's tensors (for checks)."""
    tensors, t = model_tensors(synth, cfg, mix, seed)
    write_gguf(path, model_metadata(cfg, arch, context_length), tensors)
    return t
