"""C-ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and reports errors without touching a device."""
from __future__ import annotations

import ctypes
import pathlib

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _declared(header: pathlib.Path, prefix: str):
    import re
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(rf"\b({prefix}[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(rinf):
    lib = rinf.load_library()
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        names += _declared(h, "qg_")
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header(rinf):
    names = rinf.header_symbols()
    assert set(names) <= set(rinf._SIGS), set(names) - set(rinf._SIGS)


def test_status_strings(rinf):
    lib = rinf.load_library()
    for s in range(8):
        assert lib.qg_status_string(s)
    assert lib.qg_status_string(99) == b"unknown status"


def test_null_arguments_rejected_without_device(rinf):
    lib = rinf.load_library()
    assert lib.qg_init(0, None) == 1
    assert lib.qg_destroy(None) == 1
    assert lib.qg_upload(None, None, 0, 12, 1, 1, None) == 1
    assert lib.qg_matvec_dev(None, None, None, None, None) == 1
    assert lib.qg_mat_info(None, None, None, None, None) == 1
    assert lib.qg_mat_kernel_kind(None) == -1
    assert lib.qg_last_error(None) == b""
    assert lib.qg_gpu_set_freshness(None, 0) == 1
    assert lib.qg_set_precision(None, 0) == 1


def test_init_without_gpu_reports_no_device(rinf):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = rinf.load_library()
    h = ctypes.c_void_p()
    assert lib.qg_init(0, ctypes.byref(h)) == 4          # QG_ERR_NO_DEVICE
    assert rinf.GpuContext.try_init() is None            # try_init -> None


def test_nbytes_for_matches_model_loader(rinf):
    # src/model.rs:167-175 byte sizes
    assert rinf.nbytes_for(rinf.Q4_K, 4864, 896) == 17024 * 144
    assert rinf.nbytes_for(rinf.Q6_K, 151936, 896) == 111672960
    assert rinf.nbytes_for(rinf.Q8_0, 896, 896) == 896 * 28 * 34
    assert rinf.nbytes_for(rinf.F16, 3, 5) == 30


def test_probe_library_exports(rinf):
    """libqgprobe.so (the measurement-only reads bench.py times) exports what
    include/qgprobe.h declares, and rejects bad arguments before any launch."""
    lib = rinf.load_probe_library()
    names = _declared(ROOT / "include" / "qgprobe.h", "qgp_")
    assert names == sorted(rinf._PROBE_SIGS)
    assert all(hasattr(lib, n) for n in names)
    assert lib.qgp_read(None, 0, 16, None, 256, 0, 1, 1, None) == -1
    assert lib.qgp_read_wave_lds(None, 0, 16, 8064, None, 1, None) == -1
