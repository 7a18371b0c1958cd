"""The C ABI's contract at its edges, on a device: the drop-in
qg_gpu_mat_vec_mul (GpuContext::mat_vec_mul, src/gpu_backend.rs:429-450)
must compute with the bytes the caller holds now, as the reference uploads
them on every call (gpu_backend.rs:478-482); failures are status codes that
leave `out` untouched, which is what a caller maps to its CPU fallback
(gpu_backend.rs:438-447); handles that are freed or still in use are refused
instead of read.  Allocation failures are forced from the host
(qg_test_fail_allocations), never by exhausting the device.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import GEMV_TOL, normwise_err

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 12, 14, 8
OOM, INVALID = 6, 1


def test_drop_in_sees_bytes_changed_in_place(ctx, oracle, synth):
    rows, cols = 256, 1024
    raw = synth.gen_blocks(Q4_K, rows, cols, 1)
    x = synth.gen_x(cols, 1)
    out = np.zeros(rows, np.float32)
    ctx.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
    assert normwise_err(out, oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) <= GEMV_TOL
    first = out.copy()
    # whole buffer rewritten in place (same address, same size)
    raw[:] = synth.gen_blocks(Q4_K, rows, cols, 2)
    ctx.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
    assert normwise_err(out, oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) <= GEMV_TOL
    assert not np.array_equal(out, first)
    # one block's scale changed in place (block 0: a sampled window)
    raw[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    ctx.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
    assert normwise_err(out, oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) <= GEMV_TOL


def test_invalidate_drops_the_copy(ctx, oracle, synth):
    """A change between the fingerprint windows is seen after qg_gpu_invalidate."""
    rows, cols = 256, 1024
    raw = synth.gen_blocks(Q4_K, rows, cols, 3)
    x = synth.gen_x(cols, 3)
    out = np.zeros(rows, np.float32)
    ctx.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
    n = raw.nbytes
    step = (n - 64) // 15
    off = step // 2 + 200                          # between windows 0 and 1
    assert 64 <= off < step and off % 144 >= 16     # a code byte of block off // 144
    raw[off] ^= 0xFF
    ctx.invalidate(raw)
    ctx.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
    assert np.array_equal(out, oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) or \
        normwise_err(out, oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) <= GEMV_TOL


def test_exact_freshness_sees_any_byte(rinf, oracle, synth):
    """QG_FRESH_EXACT: a change between the fingerprint windows is seen on the
    next call with no qg_gpu_invalidate (the reference's upload-every-call
    result); the default sampled mode keeps its copy, which is what makes
    the byte below a between-windows one."""
    rows, cols = 256, 1024
    raw = synth.gen_blocks(Q4_K, rows, cols, 5)
    x = synth.gen_x(cols, 5)
    n = raw.nbytes
    step = (n - 64) // 15
    off = step // 2 + 200                          # between windows 0 and 1
    assert 64 <= off < step and off % 144 >= 16     # a code byte of block off // 144
    exact, sampled = rinf.GpuContext(0), rinf.GpuContext(0)
    try:
        exact.set_freshness(rinf.FRESH_EXACT)
        with pytest.raises(rinf.QgemvError) as e:
            exact.set_freshness(2)
        assert e.value.status == INVALID
        outs = {c: np.zeros(rows, np.float32) for c in ("e", "s")}
        exact.mat_vec_mul(raw, Q4_K, x, outs["e"], rows, cols)
        sampled.mat_vec_mul(raw, Q4_K, x, outs["s"], rows, cols)
        first = outs["e"].copy()
        assert np.array_equal(outs["s"], first)
        for k in range(3):                          # three edits, each seen at once
            raw[off + 9 * k] ^= 0x5A
            ref = oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)
            exact.mat_vec_mul(raw, Q4_K, x, outs["e"], rows, cols)
            assert normwise_err(outs["e"], ref) <= GEMV_TOL
            assert not np.array_equal(outs["e"], first)
        sampled.mat_vec_mul(raw, Q4_K, x, outs["s"], rows, cols)
        assert np.array_equal(outs["s"], first)     # stale: the edits lie between its windows
        # back to sampled: the exact-mode copy is uploaded again, then kept
        exact.set_freshness(rinf.FRESH_SAMPLED)
        exact.mat_vec_mul(raw, Q4_K, x, outs["e"], rows, cols)
        assert normwise_err(outs["e"], oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)) <= GEMV_TOL
        # an unchanged buffer under the exact mode keeps its copy (same result bit for bit)
        exact.set_freshness(rinf.FRESH_EXACT)
        a, b = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
        exact.mat_vec_mul(raw, Q4_K, x, a, rows, cols)
        exact.mat_vec_mul(raw, Q4_K, x, b, rows, cols)
        assert np.array_equal(a, b)
    finally:
        exact.close()
        sampled.close()


def test_injected_allocation_failures(rinf, oracle, synth):
    """Every allocation a context attempts can be made to fail from the host:
    the call returns QG_ERR_OUT_OF_MEMORY, hands out no matrix and leaves
    `out` as it was, and the context keeps working afterwards."""
    rows, cols = 128, 512
    raw = synth.gen_blocks(Q4_K, rows, cols, 4)
    x = synth.gen_x(cols, 4)
    ref = oracle.mat_vec_mul(raw, Q4_K, rows, cols, x)
    c = rinf.GpuContext(0)
    try:
        # qg_upload: the device copy (skip 0) and the repacked copy (skip 1)
        for skip in (0, 1):
            c.fail_allocations(1, skip)
            with pytest.raises(rinf.QgemvError) as e:
                c.upload(raw, Q4_K, rows, cols)
            assert e.value.status == OOM
        c.fail_allocations(0)
        m = c.upload(raw, Q4_K, rows, cols)
        # qg_mat_stack: the stacked copy
        c.fail_allocations(1)
        with pytest.raises(rinf.QgemvError) as e:
            c.stack([m, m])
        assert e.value.status == OOM
        c.fail_allocations(0)
        m.free()
    finally:
        c.close()
    # qg_matvec_host on a fresh context: pinned x, pinned y, device x, device y
    for skip in range(4):
        c = rinf.GpuContext(0)
        try:
            m = c.upload(raw, Q4_K, rows, cols)
            c.fail_allocations(1, skip)
            y = np.full(rows, 7.0, np.float32)
            with pytest.raises(rinf.QgemvError) as e:
                m.matvec_host(x, y)
            assert e.value.status == OOM and np.all(y == 7.0)
            m.matvec_host(x, y)                                    # recovers
            assert normwise_err(y, ref) <= GEMV_TOL
            m.free()
        finally:
            c.close()
    # the drop-in: its upload or its staging fails, out untouched; then it works
    for skip in (0, 2):
        c = rinf.GpuContext(0)
        try:
            c.fail_allocations(1, skip)
            out = np.full(rows, 3.0, np.float32)
            with pytest.raises(rinf.QgemvError) as e:
                c.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
            assert e.value.status == OOM and np.all(out == 3.0)
            c.mat_vec_mul(raw, Q4_K, x, out, rows, cols)
            assert normwise_err(out, ref) <= GEMV_TOL
        finally:
            c.close()


def test_freed_handle_is_refused(rinf, synth):
    c = rinf.GpuContext(0)
    try:
        raw = synth.gen_blocks(Q8_0, 64, 256, 5)
        m = c.upload(raw, Q8_0, 64, 256)
        stale = ctypes.c_void_p(m.h.value)
        m.free()
        x = np.zeros(256, np.float32)
        y = np.full(64, 5.0, np.float32)
        rc = c.lib.qg_matvec_host(c.h, stale, x.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p))
        assert rc == INVALID and np.all(y == 5.0)
        assert c.lib.qg_mat_free(c.h, stale) == INVALID
        other = rinf.GpuContext(0)
        m2 = other.upload(raw, Q8_0, 64, 256)
        rc = c.lib.qg_matvec_host(c.h, m2.h, x.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p))
        assert rc == INVALID                                      # another context's matrix
        m2.free()
        other.close()
    finally:
        c.close()


def test_shared_matrix_cannot_be_freed_while_in_use(rinf, synth):
    c = rinf.GpuContext(0)
    try:
        V, E = 300, 256
        raw = synth.gen_blocks(Q6_K, V, E, 6)
        tok = c.upload(raw, Q6_K, V, E)
        dev = rinf.DeviceModel(c, E, 1, 4, 2, 512, V, 8, 1e6, 1e-6)
        dev.share_matrix(rinf.M_TOKEN_EMBD, 0, tok)
        dev.share_matrix(rinf.M_LM_HEAD, 0, tok)
        with pytest.raises(rinf.QgemvError) as e:
            tok.free()
        assert e.value.status == INVALID
        # the slot gets its own matrix: one use left (lm_head)
        dev.set_matrix(rinf.M_TOKEN_EMBD, 0, raw, Q6_K, V, E)
        with pytest.raises(rinf.QgemvError):
            tok.free()
        dev.close()
        tok.free()                                                # no model uses it now
    finally:
        c.close()


def test_probe_reads(rinf, ctx):
    """libqgprobe.so's measurement reads (include/qgprobe.h) run every design
    bench.py sweeps and the gemv_wave-shaped LDS read: zeros never match
    the constant, so d_out stays 0; bad arguments are refused."""
    import ctypes
    import torch
    probe = rinf.load_probe_library()
    rows, row_bytes = 64, 8064                      # the wave read's row shape (Q4_K 14336 columns)
    bufs = [torch.zeros(rows * row_bytes // 4, dtype=torch.float32, device="cuda") for _ in range(2)]
    arr = (ctypes.c_void_p * 2)(*[b.data_ptr() for b in bufs])
    out = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nb = rows * row_bytes
    for threads in (256, 512, 1024):
        for loads in (1, 2, 4, 8):
            for wgs in (0, 4, 256):
                assert probe.qgp_read(arr, 2, nb, out.data_ptr(), threads, wgs, loads, 3, st) == 0
    assert probe.qgp_read_wave_lds(arr, 2, rows, row_bytes, out.data_ptr(), 3, st) == 0
    torch.cuda.synchronize()
    assert int(out[0]) == 0
    assert probe.qgp_read(arr, 2, 100, out.data_ptr(), 256, 0, 1, 1, st) == -1       # not whole 16-byte pieces
    assert probe.qgp_read(arr, 2, nb, out.data_ptr(), 256, 0, 3, 1, st) == -1        # 3 loads per thread
    assert probe.qgp_read_wave_lds(arr, 2, rows, 100, out.data_ptr(), 1, st) == -1   # row not 128-byte pieces


def test_wrap_device_needs_the_tail_pad(ctx):
    """qg_wrap_device's kernels read whole 16-byte pieces up to 512 bytes past
    the matrix data: a matrix that ends less than 512 bytes before the end of
    its device allocation is refused (QG_ERR_INVALID_ARG), one that leaves
    exactly 512 is accepted, and a host pointer is refused."""
    import torch
    rows, cols = 64, 256
    need = rows * (cols // 256) * 144                      # Q4_K: 144 bytes per 256 columns
    buf = torch.zeros(8 << 20, dtype=torch.uint8, device="cuda")
    seg = next(s for s in torch.cuda.memory_snapshot()
               if s["address"] <= buf.data_ptr() < s["address"] + s["total_size"])
    end = seg["address"] + seg["total_size"]
    lib, out = ctx.lib, ctypes.c_void_p()

    def wrap(addr):
        return lib.qg_wrap_device(ctx.h, ctypes.c_void_p(addr), need, Q4_K, rows, cols, ctypes.byref(out))

    for slack, want in ((0, INVALID), (256, INVALID), (496, INVALID), (512, 0), (4096, 0)):
        addr = end - need - slack
        assert addr % 16 == 0 and addr >= seg["address"]
        rc = wrap(addr)
        assert rc == want, (slack, rc)
        if rc == 0:
            assert lib.qg_mat_free(ctx.h, out) == 0
    host = np.zeros(need + 1024, np.uint8)
    assert wrap(host.ctypes.data) == INVALID
    # no sticky HIP error is left behind for the next launch
    torch.ones(16, device="cuda").sum().item()
    del buf
