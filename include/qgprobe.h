/* qgprobe.h -- C ABI of libqgprobe.so: measurement-only kernels that read a
 * device buffer and compute nothing.  They have no counterpart in
 * yudono/rust-inference and are not part of the mat-vec library
 * (libqgemv.so); bench.py times them to find the fastest plain read of the
 * GEMV's byte count on the device -- the streaming ceiling its HBM rate is
 * compared with.
 *
 * Every entry point is asynchronous on `stream` (a hipStream_t; NULL = the
 * null stream), reads `nbytes` (a multiple of 16, 16-byte aligned) once per
 * launch, and writes at most d_out[0] (only if the XOR of everything read
 * equals a constant, so no load can be dropped).  Returns 0, or -1 for bad
 * arguments, -2 when a launch fails. */
#ifndef QGPROBE_H
#define QGPROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Grid-wide coalesced read: workgroups of `threads` threads (64..1024, a
 * multiple of 64), each thread `loads` 16-byte loads in flight per round
 * (1, 2, 4 or 8), consecutive threads on consecutive 16-byte pieces.
 * workgroups = 0: one round, ceil(nbytes / (16 threads loads)) workgroups;
 * otherwise that many workgroups stride over the buffer (persistent).
 * n_launches launches, launch i reading bufs[i % n_bufs] (every buffer
 * nbytes long), issued back to back from C. */
int qgp_read(const void *const *bufs, size_t n_bufs, size_t nbytes, uint32_t *d_out, uint32_t threads,
             uint32_t workgroups, uint32_t loads, size_t n_launches, void *stream);

/* The load pattern of the wave-private Q4_K GEMV (qg::gemv_wave) without its
 * compute: the buffer is `rows` rows of row_bytes (a multiple of 128, at
 * most 8 KiB), ceil(rows / 16) workgroups of 8 waves; workgroup b owns rows
 * b + G i (i < 16, G workgroups), wave w copies its eighth of each row
 * straight into LDS (global_load_lds_dwordx4, one instruction per row), four
 * rows per step with one step in flight.  n_launches launches over bufs as
 * for qgp_read. */
int qgp_read_wave_lds(const void *const *bufs, size_t n_bufs, size_t rows, size_t row_bytes, uint32_t *d_out,
                      size_t n_launches, void *stream);

#ifdef __cplusplus
}
#endif

#endif
