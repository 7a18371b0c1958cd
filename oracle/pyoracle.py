"""ctypes binding of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of yudono/rust-inference's quantized mat-vec path
(oracle/qref.c, oracle/qref_model.c).  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this module, and only as the
checker (or, for cpu_baseline, as the timed CPU port), never as the product.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32
_F = ctypes.c_float

_SIGS = {
    "qref_block_size": (_SZ, [_U32]),
    "qref_block_bytes": (_SZ, [_U32]),
    "qref_fp16_to_fp32": (_F, [ctypes.c_uint16]),
    "qref_get_scale_min_k4": (None, [_SZ, _P, _P, _P]),
    "qref_dequantize_block": (None, [_P, _SZ, _U32, _SZ, _P]),
    "qref_dequantize": (ctypes.c_longlong, [_P, _SZ, _U32, _SZ, _P]),
    "qref_dequantize_len": (_SZ, [_U32, _SZ]),
    "qref_mat_vec_mul": (None, [_P, _SZ, _U32, _SZ, _SZ, _P, _P]),
    "qref_mat_vec_mul_rows": (None, [_P, _SZ, _U32, _SZ, _SZ, _P, _P]),
    "qref_mat_vec_mul_transposed": (None, [_P, _P, _P, _SZ, _SZ]),
    "qref_fallback_cpu": (ctypes.c_int, [_P, _SZ, _U32, _SZ, _SZ, _P, _P]),
    "qref_dequantize_row": (None, [_P, _SZ, _U32, _SZ, _SZ, _SZ, _P]),
    "qref_rmsnorm": (None, [_P, _P, _P, _SZ, _F]),
    "qref_silu": (_F, [_F]),
    "qref_softmax_inplace": (None, [_P, _SZ]),
    "qref_argmax": (_SZ, [_P, _SZ]),
    "qref_rope_tables": (None, [_SZ, _F, _SZ, _P, _P]),
    "qref_rope_apply": (None, [_P, _SZ, _SZ, _P, _P, _SZ]),
    "qref_repetition_penalty": (None, [_P, _SZ, _P, _SZ, _F, _SZ]),
    "qref_model_create": (_P, [_SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _F, _F]),
    "qref_model_destroy": (None, [_P]),
    "qref_model_set_mat": (ctypes.c_int, [_P, ctypes.c_int, _SZ, _P, _SZ, _U32, _SZ, _SZ]),
    "qref_model_set_vec": (ctypes.c_int, [_P, ctypes.c_int, _SZ, _P]),
    "qref_model_reset": (None, [_P]),
    "qref_model_forward": (ctypes.c_int, [_P, _SZ, _SZ, _P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} not built; run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def fp16_to_fp32(bits: int) -> float:
    return lib().qref_fp16_to_fp32(bits)


def get_scale_min_k4(j: int, scales: np.ndarray):
    sc, m = np.zeros(1, np.float32), np.zeros(1, np.float32)
    lib().qref_get_scale_min_k4(j, _p(np.ascontiguousarray(scales, np.uint8)), _p(sc), _p(m))
    return float(sc[0]), float(m[0])


def dequantize_block(raw: np.ndarray, dtype: int, block_idx: int, buf=None) -> np.ndarray:
    if buf is None:
        buf = np.zeros(256, np.float32)
    lib().qref_dequantize_block(_p(raw), raw.nbytes, dtype, block_idx, _p(buf))
    return buf


def dequantize(raw: np.ndarray, dtype: int, n: int):
    """Vec<f32> of quant::dequantize, or None for the reference's Err."""
    L = lib()
    out = np.zeros(max(L.qref_dequantize_len(dtype, n), 1), np.float32)
    got = L.qref_dequantize(_p(raw), raw.nbytes, dtype, n, _p(out))
    return None if got < 0 else out[:got]


def mat_vec_mul(raw: np.ndarray, dtype: int, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """quant.rs:188-205 (the --cpu path), faithful flat-index loop."""
    out = np.zeros(rows, np.float32)
    lib().qref_mat_vec_mul(_p(raw), raw.nbytes, dtype, rows, cols, _p(x), _p(out))
    return out


def mat_vec_mul_rows(raw: np.ndarray, dtype: int, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """Row-ordered, multi-threaded loop bit-identical to mat_vec_mul."""
    out = np.zeros(rows, np.float32)
    lib().qref_mat_vec_mul_rows(_p(raw), raw.nbytes, dtype, rows, cols, _p(x), _p(out))
    return out


def fallback_cpu(raw: np.ndarray, dtype: int, rows: int, cols: int, x: np.ndarray):
    """gpu_backend.rs:556-567; None where the reference panics."""
    out = np.zeros(rows, np.float32)
    rc = lib().qref_fallback_cpu(_p(raw), raw.nbytes, dtype, rows, cols, _p(x), _p(out))
    return None if rc != 0 else out


def mat_vec_mul_transposed(w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    out = np.zeros(out_dim, np.float32)
    lib().qref_mat_vec_mul_transposed(_p(w), _p(x), _p(out), out_dim, in_dim)
    return out


def dequantize_row(raw: np.ndarray, dtype: int, rows: int, cols: int, row: int, buf=None):
    if buf is None:
        buf = np.zeros(cols, np.float32)
    lib().qref_dequantize_row(_p(raw), raw.nbytes, dtype, rows, cols, row, _p(buf))
    return buf


def rmsnorm(x, w, eps):
    out = np.zeros_like(x)
    lib().qref_rmsnorm(_p(x), _p(w), _p(out), x.size, eps)
    return out


def silu(v: float) -> float:
    return lib().qref_silu(v)


def softmax_inplace(a: np.ndarray):
    lib().qref_softmax_inplace(_p(a), a.size)


def argmax(a: np.ndarray) -> int:
    return int(lib().qref_argmax(_p(a), a.size))


def rope_tables(dim: int, base: float, max_seq_len: int):
    c = np.zeros(max_seq_len * (dim // 2), np.float32)
    s = np.zeros_like(c)
    lib().qref_rope_tables(dim, base, max_seq_len, _p(c), _p(s))
    return c, s


def rope_apply(x: np.ndarray, position: int, cos_t, sin_t, max_pos: int):
    lib().qref_rope_apply(_p(x), x.size, position, _p(cos_t), _p(sin_t), max_pos)


def repetition_penalty(logits: np.ndarray, recent, penalty=1.1, window=64):
    r = np.ascontiguousarray(recent, dtype=np.uint64)
    lib().qref_repetition_penalty(_p(logits), logits.size, _p(r) if r.size else None, r.size,
                                  penalty, window)


# matrix / vector slots of qref_model_set_mat / qref_model_set_vec
QM = dict(token_embd=0, lm_head=1, wq=2, wk=3, wv=4, wo=5, gate=6, up=7, down=8)
QV = dict(final_norm=0, attn_norm=1, ffn_norm=2, bq=3, bk=4, bv=5)


class Model:
    """transformer.rs:63-98 restated (qref_model.c); borrows numpy buffers."""

    def __init__(self, cfg: dict):
        self.cfg = cfg
        L = lib()
        self.h = L.qref_model_create(cfg["embed_dim"], cfg["n_layers"], cfg["n_heads"],
                                     cfg["n_kv_heads"], cfg["hidden_dim"], cfg["vocab_size"],
                                     cfg["max_seq_len"], cfg["rope_base"], cfg["norm_eps"])
        self._keep = []

    def set_mat(self, name: str, layer: int, raw: np.ndarray, dtype: int, rows: int, cols: int):
        self._keep.append(raw)
        rc = lib().qref_model_set_mat(self.h, QM[name], layer, _p(raw), raw.nbytes, dtype, rows, cols)
        assert rc == 0

    def set_vec(self, name: str, layer: int, v: np.ndarray):
        v = np.ascontiguousarray(v, np.float32)
        self._keep.append(v)
        assert lib().qref_model_set_vec(self.h, QV[name], layer, _p(v)) == 0

    def reset(self):
        lib().qref_model_reset(self.h)

    def forward(self, token_id: int, pos: int) -> np.ndarray:
        logits = np.zeros(self.cfg["vocab_size"], np.float32)
        rc = lib().qref_model_forward(self.h, token_id, pos, _p(logits))
        if rc != 0:
            raise RuntimeError("KV cache overflow (kv_cache.rs:54-59)")
        return logits

    def __del__(self):
        try:
            lib().qref_model_destroy(self.h)
        except Exception:
            pass
