"""rust-inference_amd -- MI355X (gfx950) quantized mat-vec for yudono/rust-inference.

Python plumbing over the C ABI of ``include/qgemv.h`` (``libqgemv.so``, built
in-tree by ``__graft_entry__.build()``).  The product is the HIP library; this
module only binds it with ctypes for tests and ``bench.py``, and mirrors the
reference's host API names so that tests read like calls of the reference:

* ``GpuContext.try_init()``            -- src/gpu_backend.rs:317-348
* ``GpuContext.mat_vec_mul(...)``      -- src/gpu_backend.rs:429-450
* ``QuantizedMatrix(data, dtype, rows, cols)`` and ``.mat_vec_mul(x, out, gpu)``
                                        -- src/quant.rs:44-55, 178-206

There is no CPU fallback in this package: if the library is missing or no
HIP device is present the calls raise.

The directory name contains a hyphen, so load it with importlib under the
module name ``rust_inference_amd`` (``__graft_entry__.load_package()`` does).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libqgemv.so"
HEADER_PATH = HERE.parent / "include" / "qgemv.h"
HEADERS = (HEADER_PATH, HERE.parent / "include" / "qgmodel.h", HERE.parent / "include" / "qggguf.h")

# GGML type ids, src/gguf.rs:43-59
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = (
    0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14)
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0",
              Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}
SUPPORTED = tuple(TYPE_NAMES)
# (block elements, block bytes), src/quant.rs:57-79
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_0: (32, 18), Q5_0: (32, 22),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

QG_OK = 0
# include/qgemv.h qg_gpu_set_freshness and qg_set_precision modes
FRESH_SAMPLED, FRESH_EXACT = 0, 1
PRECISION_FIXED22, PRECISION_F32 = 0, 1
STATUS = {0: "QG_OK", 1: "QG_ERR_INVALID_ARG", 2: "QG_ERR_UNSUPPORTED_TYPE",
          3: "QG_ERR_SHORT_DATA", 4: "QG_ERR_NO_DEVICE", 5: "QG_ERR_HIP",
          6: "QG_ERR_OUT_OF_MEMORY", 7: "QG_ERR_SHAPE"}


def nbytes_for(dtype: int, rows: int, cols: int) -> int:
    """ceil(rows*cols/bs)*bb -- the byte count src/model.rs:167-175 reads."""
    bs, bb = BLOCK[dtype]
    return -(-(rows * cols) // bs) * bb


class QgemvError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS.get(status, status)}")
        self.status = status


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32
_FP = ctypes.POINTER(ctypes.c_float)

_SIGS = {
    "qg_init": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_P)]),
    "qg_destroy": (ctypes.c_int, [_P]),
    "qg_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "qg_last_error": (ctypes.c_char_p, [_P]),
    "qg_upload": (ctypes.c_int, [_P, _P, _SZ, _U32, _SZ, _SZ, ctypes.POINTER(_P)]),
    "qg_wrap_device": (ctypes.c_int, [_P, _P, _SZ, _U32, _SZ, _SZ, ctypes.POINTER(_P)]),
    "qg_mat_free": (ctypes.c_int, [_P, _P]),
    "qg_mat_info": (ctypes.c_int, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_SZ),
                                   ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "qg_mat_kernel_kind": (ctypes.c_int, [_P]),
    "qg_matvec_dev": (ctypes.c_int, [_P, _P, _P, _P, _P]),
    "qg_matvec_norm_dev": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P]),
    "qg_matvec_silu_dev": (ctypes.c_int, [_P, _P, _P, _P, _P, _P]),
    "qg_matvec_norm_glu_dev": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P]),
    "qg_matvec_norm_glu_dev_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P]),
    "qg_mat_stack": (ctypes.c_int, [_P, ctypes.POINTER(_P), ctypes.c_int, ctypes.POINTER(_P)]),
    "qg_gpu_invalidate": (ctypes.c_int, [_P, _P]),
    "qg_gpu_set_freshness": (ctypes.c_int, [_P, ctypes.c_int]),
    "qg_set_precision": (ctypes.c_int, [_P, ctypes.c_int]),
    "qg_matvec_dev_repeat": (ctypes.c_int, [_P, _P, _SZ, _P, _P, _SZ, _P]),
    "qg_test_fail_allocations": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int]),
    "qg_matvec_host": (ctypes.c_int, [_P, _P, _P, _P]),
    "qg_gpu_mat_vec_mul": (ctypes.c_int, [_P, _P, _SZ, _U32, _P, _P, _SZ, _SZ]),
    "qg_dequant_dev": (ctypes.c_int, [_P, _P, _P, _P]),
    "qg_dequant_host": (ctypes.c_int, [_P, _P, _P]),
    "qg_dequantize_row_dev": (ctypes.c_int, [_P, _P, _SZ, _P, _P]),
    "qg_synchronize": (ctypes.c_int, [_P]),
    "qg_stream": (_P, [_P]),
    "qg_device_cu_count": (ctypes.c_int, [_P]),
    # include/qggguf.h
    "qg_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "qg_gguf_close": (ctypes.c_int, [_P]),
    "qg_gguf_last_error": (ctypes.c_char_p, [_P]),
    "qg_gguf_open_error": (ctypes.c_char_p, []),
    "qg_gguf_version": (ctypes.c_int, [_P, ctypes.POINTER(_U32)]),
    "qg_gguf_data_offset": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "qg_gguf_metadata_count": (ctypes.c_int, [_P, ctypes.POINTER(_SZ)]),
    "qg_gguf_metadata_type": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_U32)]),
    "qg_gguf_get_u64": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "qg_gguf_get_f32": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
    "qg_gguf_get_string": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_char_p, _SZ, ctypes.POINTER(_SZ)]),
    "qg_gguf_get_array_info": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_U32),
                                              ctypes.POINTER(ctypes.c_uint64)]),
    "qg_gguf_tensor_count": (ctypes.c_int, [_P, ctypes.POINTER(_SZ)]),
    "qg_gguf_find_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_SZ)]),
    "qg_gguf_tensor_info": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32),
                                           ctypes.POINTER(_U32), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_SZ)]),
    "qg_gguf_tensor_data": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
    "qg_gguf_model_config": (ctypes.c_int, [_P, _U32, _P]),
    "qg_model_load_gguf": (ctypes.c_int, [_P, ctypes.c_char_p, _U32, ctypes.POINTER(_P)]),
    # include/qgmodel.h
    "qg_model_create": (ctypes.c_int, [_P, _P, ctypes.POINTER(_P)]),
    "qg_model_destroy": (ctypes.c_int, [_P]),
    "qg_model_set_matrix": (ctypes.c_int, [_P, _U32, _U32, _P, _SZ, _U32, _SZ, _SZ]),
    "qg_model_share_matrix": (ctypes.c_int, [_P, _U32, _U32, _P]),
    "qg_model_set_vector": (ctypes.c_int, [_P, _U32, _U32, _P, _SZ]),
    "qg_model_use_graphs": (ctypes.c_int, [_P, ctypes.c_int]),
    "qg_model_reset": (ctypes.c_int, [_P]),
    "qg_model_seq_len": (ctypes.c_int, [_P, ctypes.POINTER(_SZ)]),
    "qg_model_forward": (ctypes.c_int, [_P, _U32, _U32, _P]),
    "qg_model_prefill": (ctypes.c_int, [_P, _P, _SZ, _P]),
    "qg_model_use_batched_prefill": (ctypes.c_int, [_P, ctypes.c_int]),
    "qg_model_set_attention_path": (ctypes.c_int, [_P, ctypes.c_int]),
    "qg_model_resident_bytes": (ctypes.c_int, [_P, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "qg_model_sample_greedy": (ctypes.c_int, [_P, _P, _SZ, ctypes.c_float, _SZ, ctypes.POINTER(_U32)]),
    "qg_model_generate": (ctypes.c_int, [_P, _P, _SZ, _SZ, ctypes.c_float, _SZ, _P,
                                         ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
}

# include/qgmodel.h slots (names of the GGUF tensors, src/model.rs:197-298)
M_TOKEN_EMBD, M_LM_HEAD, M_WQ, M_WK, M_WV, M_WO, M_GATE, M_UP, M_DOWN = range(9)
V_FINAL_NORM, V_ATTN_NORM, V_FFN_NORM, V_BQ, V_BK, V_BV = range(6)


class ModelConfig(ctypes.Structure):
    """qg_model_config: ModelConfig (src/model.rs:34-46)."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("embed_dim", "n_layers", "n_heads", "n_kv_heads",
                                                 "hidden_dim", "vocab_size", "max_seq_len")] + \
               [("rope_base", ctypes.c_float), ("norm_eps", ctypes.c_float)]

_lib = None


def header_symbols(paths=HEADERS) -> list[str]:
    """Every function the C ABI headers declare."""
    if isinstance(paths, (str, pathlib.Path)):
        paths = (paths,)
    out = set()
    for path in paths:
        text = re.sub(r"/\*.*?\*/", "", pathlib.Path(path).read_text(), flags=re.S)
        out.update(re.findall(r"\b(qg_[a-z0-9_]+)\s*\(", text))
    return sorted(out)


def use_library(path: pathlib.Path | str):
    """Make `path` (a build of the same library, e.g. libqgemv_timeline.so)
    the library every context of this process binds; call before the first
    GpuContext."""
    global _lib
    _lib = load_library(path)
    return _lib


def load_library(path: pathlib.Path | str = LIB_PATH):
    """Load libqgemv.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    p = pathlib.Path(path)
    # torch ships its own libamdhip64.so with the same SONAME as /opt/rocm's.
    # Importing torch first makes this library bind to that already-loaded
    # runtime, so a process that also uses torch tensors has one HIP runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not p.exists():
        raise ImportError(f"{p} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


PROBE_LIB_PATH = HERE / "libqgprobe.so"
_PROBE_SIGS = {
    "qgp_read": (ctypes.c_int, [_P, _SZ, _SZ, _P, _U32, _U32, _U32, _SZ, _P]),
    "qgp_read_wave_lds": (ctypes.c_int, [_P, _SZ, _SZ, _SZ, _P, _SZ, _P]),
}


def load_probe_library(path: pathlib.Path | str = PROBE_LIB_PATH):
    """libqgprobe.so (include/qgprobe.h): the measurement-only read kernels
    bench.py times for the streaming ceiling; not part of the mat-vec
    library.  Loaded after libqgemv.so, so both bind one HIP runtime."""
    load_library()
    p = pathlib.Path(path)
    if not p.exists():
        raise ImportError(f"{p} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _PROBE_SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _ptr(a):
    """Address of a numpy array's data or a torch tensor's storage."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return ctypes.c_void_p(a.data_ptr())
    return ctypes.c_void_p(a.ctypes.data)


class GpuContext:
    """One HIP device and stream (mirror of the reference's GpuContext)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _P()
        rc = self.lib.qg_init(device, ctypes.byref(h))
        if rc != QG_OK:
            raise QgemvError(rc, f"qg_init(device={device})")
        self.h = h
        self._mats = []

    @classmethod
    def try_init(cls, device: int = 0):
        """None when no device can be opened (src/gpu_backend.rs:317-348)."""
        try:
            return cls(device)
        except (QgemvError, OSError, ImportError):
            return None

    def check(self, rc: int, what: str):
        if rc != QG_OK:
            err = self.lib.qg_last_error(self.h)
            raise QgemvError(rc, f"{what} ({err.decode() if err else ''})")

    def close(self):
        if self.h:
            self.lib.qg_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return self.lib.qg_stream(self.h) or 0

    @property
    def cu_count(self) -> int:
        return self.lib.qg_device_cu_count(self.h)

    def synchronize(self):
        self.check(self.lib.qg_synchronize(self.h), "qg_synchronize")

    def upload(self, raw, dtype: int, rows: int, cols: int) -> "DeviceMatrix":
        m = _P()
        rc = self.lib.qg_upload(self.h, _ptr(raw), raw.nbytes, dtype, rows, cols, ctypes.byref(m))
        self.check(rc, "qg_upload")
        return DeviceMatrix(self, m, dtype, rows, cols)

    def wrap_device(self, d_raw, dtype: int, rows: int, cols: int) -> "DeviceMatrix":
        """A matrix over GGUF-layout bytes already in device memory (a torch
        uint8 tensor, 16-byte aligned, with >= 512 readable bytes after the
        data); not copied, so the tensor must outlive the handle (qg_wrap_device)."""
        m = _P()
        rc = self.lib.qg_wrap_device(self.h, _ptr(d_raw), nbytes_for(dtype, rows, cols), dtype, rows, cols,
                                     ctypes.byref(m))
        self.check(rc, "qg_wrap_device")
        return DeviceMatrix(self, m, dtype, rows, cols)

    def stack(self, parts) -> "DeviceMatrix":
        """One matrix with the rows of `parts` (DeviceMatrix, same type and
        cols) in order (qg_mat_stack)."""
        arr = (_P * len(parts))(*[p.h for p in parts])
        m = _P()
        rc = self.lib.qg_mat_stack(self.h, arr, len(parts), ctypes.byref(m))
        self.check(rc, "qg_mat_stack")
        return DeviceMatrix(self, m, parts[0].dtype, sum(p.rows for p in parts), parts[0].cols)

    def mat_vec_mul(self, weight_data, dtype: int, x, out, rows: int, cols: int):
        """src/gpu_backend.rs:429-437 signature; host numpy arrays in and out."""
        rc = self.lib.qg_gpu_mat_vec_mul(self.h, _ptr(weight_data), weight_data.nbytes, dtype,
                                         _ptr(x), _ptr(out), rows, cols)
        self.check(rc, "qg_gpu_mat_vec_mul")

    def matvec_repeat(self, mats, d_x, d_y, n_launches: int, stream=None):
        """n_launches qg_matvec_dev calls cycling over mats, issued from C
        (qg_matvec_dev_repeat)."""
        arr = (ctypes.c_void_p * len(mats))(*[m.h for m in mats])
        rc = self.lib.qg_matvec_dev_repeat(self.h, arr, len(mats), _ptr(d_x), _ptr(d_y), int(n_launches),
                                           ctypes.c_void_p(stream) if stream else None)
        self.check(rc, "qg_matvec_dev_repeat")

    def invalidate(self, weight_data):
        """Drop the device copies mat_vec_mul keeps for this host buffer (qg_gpu_invalidate)."""
        self.check(self.lib.qg_gpu_invalidate(self.h, _ptr(weight_data)), "qg_gpu_invalidate")

    def set_freshness(self, mode: int):
        """How mat_vec_mul checks its device copies against the host bytes
        (qg_gpu_set_freshness): FRESH_SAMPLED (16 windows, the default) or
        FRESH_EXACT (every byte on every call)."""
        self.check(self.lib.qg_gpu_set_freshness(self.h, int(mode)), "qg_gpu_set_freshness")

    def set_precision(self, mode: int):
        """Arithmetic of this context's plain mat-vecs (qg_set_precision):
        PRECISION_FIXED22 (the default) or PRECISION_F32."""
        self.check(self.lib.qg_set_precision(self.h, int(mode)), "qg_set_precision")

    def fail_allocations(self, n: int, skip: int = 0):
        """Test hook: after `skip` more allocations, the next n allocations of
        this context report out-of-memory (qg_test_fail_allocations)."""
        self.check(self.lib.qg_test_fail_allocations(self.h, int(skip), int(n)), "qg_test_fail_allocations")


class DeviceMatrix:
    """A matrix resident in HBM (qg_mat)."""

    def __init__(self, ctx: GpuContext, h, dtype: int, rows: int, cols: int):
        self.ctx, self.h, self.dtype, self.rows, self.cols = ctx, h, dtype, rows, cols

    def free(self):
        # a closed context has already freed its matrices (qg_destroy)
        if self.h and self.ctx.h:
            self.ctx.check(self.ctx.lib.qg_mat_free(self.ctx.h, self.h), "qg_mat_free")
        self.h = None

    @property
    def kernel_kind(self) -> int:
        return self.ctx.lib.qg_mat_kernel_kind(self.h)

    def matvec_dev(self, d_x, d_y, stream=None):
        """d_x, d_y: torch device tensors (float32)."""
        rc = self.ctx.lib.qg_matvec_dev(self.ctx.h, self.h, _ptr(d_x), _ptr(d_y),
                                        ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_matvec_dev")

    def matvec_norm_dev(self, d_xa, d_xb, d_nw, eps, d_y, d_sum_out=None, stream=None):
        """y = W · (rmsnorm(xa + xb) * nw); torch device tensors (float32),
        d_xb / d_sum_out may be None."""
        rc = self.ctx.lib.qg_matvec_norm_dev(self.ctx.h, self.h, _ptr(d_xa),
                                             _ptr(d_xb) if d_xb is not None else None, _ptr(d_nw),
                                             float(eps),
                                             _ptr(d_sum_out) if d_sum_out is not None else None,
                                             _ptr(d_y), ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_matvec_norm_dev")

    def matvec_norm_glu_dev(self, d_xa, d_xb, d_nw, eps, d_h, d_sum_out=None, stream=None):
        """h = silu(gate · x) * (up · x), x = rmsnorm(xa + xb) * nw, for this
        [gate; up] matrix; torch device tensors (float32)."""
        rc = self.ctx.lib.qg_matvec_norm_glu_dev(self.ctx.h, self.h, _ptr(d_xa),
                                                 _ptr(d_xb) if d_xb is not None else None, _ptr(d_nw),
                                                 float(eps),
                                                 _ptr(d_sum_out) if d_sum_out is not None else None,
                                                 _ptr(d_h), ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_matvec_norm_glu_dev")

    def matvec_norm_glu_dev_noalloc(self, d_xa, d_xb, d_nw, eps, d_h, d_sum_out=None, stream=None):
        """matvec_norm_glu_dev through qg_matvec_norm_glu_dev_noalloc (no device
        allocation; the per-GPU static scratch array)."""
        rc = self.ctx.lib.qg_matvec_norm_glu_dev_noalloc(self.ctx.h, self.h, _ptr(d_xa),
                                                         _ptr(d_xb) if d_xb is not None else None, _ptr(d_nw),
                                                         float(eps),
                                                         _ptr(d_sum_out) if d_sum_out is not None else None,
                                                         _ptr(d_h), ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_matvec_norm_glu_dev_noalloc")

    def matvec_silu_dev(self, d_g, d_u, d_y, stream=None):
        """y = W · (silu(g) * u); torch device tensors (float32)."""
        rc = self.ctx.lib.qg_matvec_silu_dev(self.ctx.h, self.h, _ptr(d_g), _ptr(d_u), _ptr(d_y),
                                             ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_matvec_silu_dev")

    def matvec_host(self, x, y):
        self.ctx.check(self.ctx.lib.qg_matvec_host(self.ctx.h, self.h, _ptr(x), _ptr(y)),
                       "qg_matvec_host")

    def dequant_host(self, out):
        self.ctx.check(self.ctx.lib.qg_dequant_host(self.ctx.h, self.h, _ptr(out)),
                       "qg_dequant_host")

    def dequant_dev(self, d_out, stream=None):
        rc = self.ctx.lib.qg_dequant_dev(self.ctx.h, self.h, _ptr(d_out),
                                         ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_dequant_dev")

    def dequantize_row_dev(self, row: int, d_out, stream=None):
        rc = self.ctx.lib.qg_dequantize_row_dev(self.ctx.h, self.h, row, _ptr(d_out),
                                                ctypes.c_void_p(stream) if stream else None)
        self.ctx.check(rc, "qg_dequantize_row_dev")


class QuantizedMatrix:
    """Mirror of src/quant.rs:44-55: raw GGUF bytes plus dtype/rows/cols."""

    def __init__(self, data, dtype: int, rows: int, cols: int):
        self.data, self.dtype, self.rows, self.cols = data, dtype, rows, cols

    def mat_vec_mul(self, x, out, gpu: GpuContext):
        """src/quant.rs:178-186 with Some(gpu); this package has no CPU branch."""
        if len(x) != self.cols or len(out) != self.rows:     # quant.rs:179-180
            raise QgemvError(7, "mat_vec_mul length mismatch")
        gpu.mat_vec_mul(self.data, self.dtype, x, out, self.rows, self.cols)


class GgufError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS.get(status, status)}")
        self.status = status


class GgufFile:
    """GGUF v3 file (include/qggguf.h; GgufFile, src/gguf.rs:244-357), mapped
    read-only.  Needs only the host part of libqgemv.so (no GPU)."""

    def __init__(self, path):
        self.lib = load_library()
        h = _P()
        rc = self.lib.qg_gguf_open(str(path).encode(), ctypes.byref(h))
        if rc:
            raise GgufError(rc, f"qg_gguf_open: {self.lib.qg_gguf_open_error().decode()}")
        self.h = h

    def close(self):
        if self.h:
            self.lib.qg_gguf_close(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _q(self, rc, what):
        if rc:
            raise GgufError(rc, what)

    @property
    def version(self) -> int:
        v = _U32()
        self._q(self.lib.qg_gguf_version(self.h, ctypes.byref(v)), "version")
        return v.value

    @property
    def data_offset(self) -> int:
        v = ctypes.c_uint64()
        self._q(self.lib.qg_gguf_data_offset(self.h, ctypes.byref(v)), "data_offset")
        return v.value

    def metadata_count(self) -> int:
        n = _SZ()
        self._q(self.lib.qg_gguf_metadata_count(self.h, ctypes.byref(n)), "metadata_count")
        return n.value

    def metadata_type(self, key: str):
        t = _U32()
        rc = self.lib.qg_gguf_metadata_type(self.h, key.encode(), ctypes.byref(t))
        return None if rc else t.value

    def get_u64(self, key: str):
        """MetadataValue::to_u64 (None when absent or of another type)."""
        v = ctypes.c_uint64()
        return None if self.lib.qg_gguf_get_u64(self.h, key.encode(), ctypes.byref(v)) else v.value

    def get_f32(self, key: str):
        v = ctypes.c_float()
        return None if self.lib.qg_gguf_get_f32(self.h, key.encode(), ctypes.byref(v)) else v.value

    def get_string(self, key: str):
        n = _SZ()
        if self.lib.qg_gguf_get_string(self.h, key.encode(), None, 0, ctypes.byref(n)):
            return None
        buf = ctypes.create_string_buffer(n.value + 1)
        self._q(self.lib.qg_gguf_get_string(self.h, key.encode(), buf, n.value + 1, ctypes.byref(n)), key)
        return buf.raw[: n.value].decode()

    def get_array_info(self, key: str):
        t, c = _U32(), ctypes.c_uint64()
        if self.lib.qg_gguf_get_array_info(self.h, key.encode(), ctypes.byref(t), ctypes.byref(c)):
            return None
        return t.value, c.value

    def tensors(self):
        """[(name, ggml type, dims (ne0 first), offset, bytes the loader reads)]."""
        n = _SZ()
        self._q(self.lib.qg_gguf_tensor_count(self.h, ctypes.byref(n)), "tensor_count")
        out = []
        for i in range(n.value):
            name, t, nd = ctypes.c_char_p(), _U32(), _U32()
            dims, off, nb = (ctypes.c_uint64 * 4)(), ctypes.c_uint64(), _SZ()
            self._q(self.lib.qg_gguf_tensor_info(self.h, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd),
                                                 dims, ctypes.byref(off), ctypes.byref(nb)), "tensor_info")
            out.append((name.value.decode(), t.value, tuple(dims[: min(nd.value, 4)]), off.value, nb.value))
        return out

    def tensor_bytes(self, name: str):
        """A copy of the tensor's bytes (numpy uint8), or None if absent."""
        import numpy as np
        i = _SZ()
        if self.lib.qg_gguf_find_tensor(self.h, name.encode(), ctypes.byref(i)):
            return None
        p, nb = _P(), _SZ()
        self._q(self.lib.qg_gguf_tensor_data(self.h, i.value, ctypes.byref(p), ctypes.byref(nb)), name)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), (nb.value,)).copy()

    def model_config(self, max_seq_len: int = 0) -> dict:
        cfg = ModelConfig()
        self._q(self.lib.qg_gguf_model_config(self.h, max_seq_len, ctypes.byref(cfg)), "model_config")
        return {k: getattr(cfg, k) for k, _ in ModelConfig._fields_}


class DeviceModel:
    """The decode step on device (include/qgmodel.h): Transformer::forward
    (src/transformer.rs:63-98), greedy Sampler::sample (src/sampler.rs:72-83,
    109-127) and Model::generate's loop (src/model.rs:357-440)."""

    def __init__(self, ctx: GpuContext, embed_dim: int, n_layers: int, n_heads: int,
                 n_kv_heads: int, hidden_dim: int, vocab_size: int, max_seq_len: int,
                 rope_base: float, norm_eps: float):
        self.ctx = ctx
        self.cfg = ModelConfig(embed_dim, n_layers, n_heads, n_kv_heads, hidden_dim, vocab_size,
                               max_seq_len, rope_base, norm_eps)
        h = _P()
        ctx.check(ctx.lib.qg_model_create(ctx.h, ctypes.byref(self.cfg), ctypes.byref(h)),
                  "qg_model_create")
        self.h = h

    @classmethod
    def load_gguf(cls, ctx: GpuContext, path, max_seq_len: int = 0):
        """Model::load's weights from a GGUF file (qg_model_load_gguf)."""
        self = cls.__new__(cls)
        self.ctx = ctx
        h = _P()
        ctx.check(ctx.lib.qg_model_load_gguf(ctx.h, str(path).encode(), max_seq_len, ctypes.byref(h)),
                  "qg_model_load_gguf")
        self.h = h
        g = GgufFile(path)
        c = g.model_config(max_seq_len)
        g.close()
        self.cfg = ModelConfig(*[c[k] for k, _ in ModelConfig._fields_])
        return self

    def close(self):
        # a closed context has already freed its models (qg_destroy)
        if self.h and self.ctx.h:
            self.ctx.lib.qg_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_matrix(self, which: int, layer: int, raw, dtype: int, rows: int, cols: int):
        self.ctx.check(self.ctx.lib.qg_model_set_matrix(self.h, which, layer, _ptr(raw), raw.nbytes,
                                                        dtype, rows, cols), "qg_model_set_matrix")

    def share_matrix(self, which: int, layer: int, mat: DeviceMatrix):
        self.ctx.check(self.ctx.lib.qg_model_share_matrix(self.h, which, layer, mat.h),
                       "qg_model_share_matrix")

    def set_vector(self, which: int, layer: int, v):
        self.ctx.check(self.ctx.lib.qg_model_set_vector(self.h, which, layer, _ptr(v), len(v)),
                       "qg_model_set_vector")

    def use_graphs(self, enable: bool):
        """HIP graph replay of the forward pass (default) or one launch per kernel."""
        self.ctx.check(self.ctx.lib.qg_model_use_graphs(self.h, int(bool(enable))), "qg_model_use_graphs")

    def reset(self):
        self.ctx.check(self.ctx.lib.qg_model_reset(self.h), "qg_model_reset")

    @property
    def seq_len(self) -> int:
        n = _SZ()
        self.ctx.check(self.ctx.lib.qg_model_seq_len(self.h, ctypes.byref(n)), "qg_model_seq_len")
        return n.value

    def prefill(self, tokens, logits=None):
        """qg_model_prefill: the prompt loop at the cached positions; logits
        (numpy f32 [vocab], optional) receives the last token's."""
        import numpy as np
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self.ctx.check(self.ctx.lib.qg_model_prefill(self.h, _ptr(t) if len(t) else None, len(t), _ptr(logits)),
                       "qg_model_prefill")

    def use_batched_prefill(self, enable: bool):
        self.ctx.check(self.ctx.lib.qg_model_use_batched_prefill(self.h, int(bool(enable))),
                       "qg_model_use_batched_prefill")

    def resident_bytes(self) -> dict:
        """Device bytes: {"weights", "file_bytes", "total"} (qg_model_resident_bytes)."""
        w, f, t = _SZ(), _SZ(), _SZ()
        self.ctx.check(self.ctx.lib.qg_model_resident_bytes(self.h, ctypes.byref(w), ctypes.byref(f), ctypes.byref(t)),
                       "qg_model_resident_bytes")
        return {"weights": w.value, "file_bytes": f.value, "total": t.value}

    def set_attention_path(self, path: int):
        """0: by length (up to 512 cached positions two workgroups per head
        merged in the wo GEMV where every wo allows it, else one; beyond,
        split), 1: always one workgroup per head, 2: always split over
        position ranges, 3: always two workgroups per head where allowed."""
        self.ctx.check(self.ctx.lib.qg_model_set_attention_path(self.h, int(path)), "qg_model_set_attention_path")

    def forward(self, token: int, pos: int, logits=None):
        """logits: numpy float32[vocab] receiving the step's logits, or None."""
        self.ctx.check(self.ctx.lib.qg_model_forward(self.h, token, pos, _ptr(logits)),
                       "qg_model_forward")

    def sample_greedy(self, recent, penalty: float = 1.1, window: int = 64) -> int:
        import numpy as np
        r = np.ascontiguousarray(recent, dtype=np.uint32)
        t = _U32()
        self.ctx.check(self.ctx.lib.qg_model_sample_greedy(self.h, _ptr(r) if len(r) else None, len(r),
                                                           penalty, window, ctypes.byref(t)),
                       "qg_model_sample_greedy")
        return t.value

    def generate(self, prompt, n_new: int, penalty: float = 1.1, window: int = 64):
        """(new tokens, prefill seconds, decode seconds)."""
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(n_new, 1), np.uint32)
        a, b = ctypes.c_double(), ctypes.c_double()
        self.ctx.check(self.ctx.lib.qg_model_generate(self.h, _ptr(p), len(p), n_new, penalty, window,
                                                      _ptr(out), ctypes.byref(a), ctypes.byref(b)),
                       "qg_model_generate")
        return out[:n_new], a.value, b.value


def env_flag(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0")
