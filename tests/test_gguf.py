"""GGUF reader (include/qggguf.h) against the oracle's restatement of
GgufFile::parse / ModelConfig::from_metadata (oracle/gguf_ref.py, src/gguf.rs:
261-341, src/model.rs:50-117), on a hand-assembled known-answer file, on files
of the synthetic writer (rust-inference_amd/gguf_writer.py), and on the
reference's quirks and error cases.  Host code only (no GPU)."""
from __future__ import annotations

import importlib
import pathlib
import struct
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def gref():
    sys.path.insert(0, str(ROOT / "oracle"))
    try:
        return importlib.import_module("gguf_ref")
    finally:
        sys.path.pop(0)


@pytest.fixture(scope="module")
def gw(rinf):
    return importlib.import_module(rinf.__name__ + ".gguf_writer")


def s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def kat_bytes() -> bytes:
    """A file assembled field by field from the format definition."""
    h = b"GGUF" + struct.pack("<IQQ", 3, 2, 4)
    h += s("general.architecture") + struct.pack("<I", 8) + s("qwen2")
    h += s("qwen2.embedding_length") + struct.pack("<II", 4, 64)
    h += s("qwen2.rope.freq_base") + struct.pack("<If", 6, 5000.0)
    h += s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + s("a") + s("bc")
    h += s("token_embd.weight") + struct.pack("<IQQIQ", 2, 64, 3, 0, 0)       # F32 64 x 3
    h += s("blk.0.attn_q.weight") + struct.pack("<IQQIQ", 2, 256, 2, 12, 800)  # Q4_K 256 x 2
    pad = (-len(h)) % 32
    data = bytearray(800 + 2 * 144)
    data[0:4] = struct.pack("<f", 1.5)
    data[800:802] = b"\x34\x12"
    return bytes(h) + b"\0" * pad + bytes(data), len(h) + pad


def test_known_answer_file(rinf, gref, tmp_path):
    raw, data_off = kat_bytes()
    p = tmp_path / "kat.gguf"
    p.write_bytes(raw)
    ref = gref.parse(raw)
    assert ref["data_offset"] == data_off and data_off % 32 == 0
    g = rinf.GgufFile(p)
    assert g.version == 3 and g.data_offset == data_off
    assert g.metadata_count() == 4
    assert g.get_string("general.architecture") == "qwen2"
    assert g.get_u64("qwen2.embedding_length") == 64
    assert g.get_f32("qwen2.rope.freq_base") == 5000.0
    assert g.get_array_info("tokenizer.ggml.tokens") == (8, 2)
    assert g.get_u64("qwen2.rope.freq_base") is None                  # to_u64 rejects f32
    t = g.tensors()
    assert t == [("token_embd.weight", 0, (64, 3), 0, 64 * 3 * 4),
                 ("blk.0.attn_q.weight", 12, (256, 2), 800, 2 * 144)]
    assert [(x["name"], x["type"], tuple(x["dims"]), x["offset"], gref.load_bytes(x)) for x in ref["tensors"]] == t
    e = g.tensor_bytes("token_embd.weight")
    assert struct.unpack("<f", e[:4].tobytes())[0] == 1.5 and e.size == 768
    q = g.tensor_bytes("blk.0.attn_q.weight")
    assert q[:2].tobytes() == b"\x34\x12" and q.size == 288
    cfg = g.model_config()
    assert cfg == pytest.approx(gref.model_config(ref["metadata"]))
    # defaults of the qwen2 architecture for everything but embed and rope
    assert (cfg["embed_dim"], cfg["n_layers"], cfg["hidden_dim"], cfg["vocab_size"]) == (64, 28, 18944, 151936)
    assert cfg["rope_base"] == 5000.0 and cfg["max_seq_len"] == 32768 and cfg["norm_eps"] == pytest.approx(1e-5)
    assert g.model_config(77)["max_seq_len"] == 77
    g.close()


SMALL = dict(embed_dim=256, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=512, vocab_size=600,
             rope_base=1e6, norm_eps=1e-6, tied=False, bias=True)


@pytest.mark.parametrize("mix,tied", [("q4_k_m", False), ("q8_0", True), ("q5_k", False)])
def test_writer_round_trip(rinf, synth, gref, gw, tmp_path, mix, tied):
    cfg = dict(SMALL, tied=tied)
    p = tmp_path / "m.gguf"
    t = gw.write_model(p, synth, cfg, mix, 5, context_length=128)
    raw = p.read_bytes()
    ref = gref.parse(raw)
    g = rinf.GgufFile(p)
    assert g.data_offset == ref["data_offset"]
    assert g.metadata_count() == len(ref["metadata"])
    for key, (vt, val) in ref["metadata"].items():
        assert g.metadata_type(key) == vt
        if vt == 8:
            assert g.get_string(key) == val
        elif vt == 9:
            assert g.get_array_info(key) == (val[0], len(val[1]))
        else:
            assert g.get_u64(key) == gref.to_u64((vt, val))
            assert g.get_f32(key) == gref.to_f32((vt, val))
    mine = g.tensors()
    assert [(x["name"], x["type"], tuple(x["dims"][:4]), x["offset"], gref.load_bytes(x))
            for x in ref["tensors"]] == mine
    # the bytes of every matrix are the generator's
    names = {"token_embd": "token_embd.weight", "lm_head": "output.weight"}
    per = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "gate": "ffn_gate",
           "up": "ffn_up", "down": "ffn_down"}
    for (slot, layer), (mraw, dtype, rows, cols) in t["mats"].items():
        name = names[slot] if slot in names else f"blk.{layer}.{per[slot]}.weight"
        assert np.array_equal(g.tensor_bytes(name), mraw)
        x = next(x for x in ref["tensors"] if x["name"] == name)
        off = ref["data_offset"] + x["offset"]
        assert raw[off:off + mraw.nbytes] == mraw.tobytes()
    assert (g.tensor_bytes("output.weight") is None) == tied
    cfgr = g.model_config()
    assert cfgr == pytest.approx(gref.model_config(ref["metadata"]))
    for k in ("embed_dim", "n_layers", "n_heads", "n_kv_heads", "hidden_dim", "vocab_size"):
        assert cfgr[k] == cfg[k]
    assert cfgr["max_seq_len"] == 128
    assert cfgr["rope_base"] == np.float32(cfg["rope_base"]) and cfgr["norm_eps"] == np.float32(cfg["norm_eps"])
    g.close()


def meta_file(path, gw, meta, tensors=()):
    gw.write_gguf(path, meta, list(tensors))
    return path


def test_metadata_quirks(rinf, gref, gw, tmp_path):
    """to_u64 takes UINT64 / INT64 / UINT32 only (an INT32 value counts as
    missing: the architecture default applies); the rms epsilon key shadows
    layer_norm_epsilon even when it is not a float; a repeated key: the last
    one wins; architecture 'llama' when general.architecture is absent."""
    meta = [("qwen2.embedding_length", gw.I32, 128), ("general.architecture", gw.STRING, "qwen2"),
            ("qwen2.block_count", gw.U64, 3), ("qwen2.feed_forward_length", gw.I64, 640),
            ("qwen2.attention.layer_norm_rms_epsilon", gw.U32, 7),
            ("qwen2.attention.layer_norm_epsilon", gw.F32, 1e-3),
            ("qwen2.vocab_size", gw.U32, 100), ("qwen2.vocab_size", gw.U32, 200),
            ("qwen2.rope.freq_base", gw.F64, 2.5e5), ("qwen2.attention.head_count", gw.U16, 4)]
    p = meta_file(tmp_path / "q.gguf", gw, meta)
    ref = gref.parse(p.read_bytes())
    g = rinf.GgufFile(p)
    c = g.model_config()
    assert c == pytest.approx(gref.model_config(ref["metadata"]))
    assert c["embed_dim"] == 3584 and c["n_layers"] == 3 and c["hidden_dim"] == 640
    assert c["vocab_size"] == 200 and c["n_heads"] == 28 and c["n_kv_heads"] == 28
    assert c["rope_base"] == 2.5e5 and c["norm_eps"] == pytest.approx(1e-5)
    g.close()
    p2 = meta_file(tmp_path / "l.gguf", gw, [("llama.embedding_length", gw.U32, 512)])
    c2 = rinf.GgufFile(p2).model_config()
    assert (c2["embed_dim"], c2["n_layers"], c2["vocab_size"], c2["rope_base"]) == (512, 32, 32000, 1e4)


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "tensor_type", "nested_array",
                                  "value_type", "utf8"])
def test_rejected_files(rinf, gref, gw, tmp_path, case):
    good = b"GGUF" + struct.pack("<IQQ", 3, 1, 1) + s("k") + struct.pack("<II", 4, 1) + \
        s("t") + struct.pack("<IQIQ", 1, 32, 0, 0)
    bad = {
        "magic": b"GGUG" + good[4:],
        "version": b"GGUF" + struct.pack("<I", 2) + good[8:],
        "truncated": good[:-3],
        "tensor_type": good[:-12] + struct.pack("<IQ", 4, 0),
        "nested_array": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + s("k") + struct.pack("<IIQ", 9, 9, 1),
        "value_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + s("k") + struct.pack("<II", 13, 0),
        "utf8": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28" + struct.pack("<II", 4, 1),
    }[case]
    gref.parse(good + b"\0" * 200)
    with pytest.raises(gref.GgufError):
        gref.parse(bad)
    p = tmp_path / "bad.gguf"
    p.write_bytes(bad)
    with pytest.raises(rinf.GgufError):
        rinf.GgufFile(p)


def test_tensor_past_end_of_file(rinf, gw, tmp_path):
    """Parsing succeeds (gguf.rs never reads the data); reading the tensor fails
    (Model::load's read_exact, model.rs:184-187)."""
    p = tmp_path / "short.gguf"
    gw.write_gguf(p, [], [("w", [64], 0, np.zeros(64, np.float32))])
    b = p.read_bytes()
    p.write_bytes(b[:-100])
    g = rinf.GgufFile(p)
    assert g.tensors()[0][0] == "w"
    with pytest.raises(rinf.GgufError) as e:
        g.tensor_bytes("w")
    assert e.value.status == 3                                            # QG_ERR_SHORT_DATA


def test_overflowing_dims_are_an_error(rinf, tmp_path):
    """Tensor dims whose element or byte count does not fit in 64 bits (a
    crafted header) give QG_ERR_SHAPE, never a wrapped small byte count that
    would pass the bounds check."""
    h = b"GGUF" + struct.pack("<IQQ", 3, 3, 0)
    h += s("a") + struct.pack("<IQQIQ", 2, 1 << 32, 1 << 32, 0, 0)      # 2^64 elements: wraps to 0
    h += s("b") + struct.pack("<IQIQ", 1, 1 << 62, 0, 0)                 # 2^62 f32: 2^64 bytes
    h += s("c") + struct.pack("<IQQIQ", 2, (1 << 40) + 1, 1 << 24, 1, 0)  # wraps to 2^24 f16
    pad = (-len(h)) % 32
    p = tmp_path / "overflow.gguf"
    p.write_bytes(h + b"\0" * pad + b"\0" * 4096)
    g = rinf.GgufFile(p)
    for name in ("a", "b", "c"):
        with pytest.raises(rinf.GgufError) as e:
            g.tensor_bytes(name)
        assert e.value.status == 7                                        # QG_ERR_SHAPE
    with pytest.raises(rinf.GgufError) as e:
        g.tensors()                                                       # tensor_info reports it too
    assert e.value.status == 7
    g.close()
