// qg_common.h -- shared definitions for the gfx950 quantized GEMV library.
//
// Layout facts restated from yudono/rust-inference:
//   GGML type ids                 src/gguf.rs:43-59
//   (block elements, block bytes) src/quant.rs:57-79
//   element (r, c) = flat index r*cols + c; block b starts at byte b*bb
//                                 src/quant.rs:82-86, 195-203
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace qg {

enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8,
    T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14
};

constexpr uint32_t block_elems(uint32_t t)
{
    return t == T_F32 || t == T_F16 ? 1u
         : t == T_Q4_0 || t == T_Q5_0 || t == T_Q8_0 ? 32u
         : t == T_Q4_K || t == T_Q5_K || t == T_Q6_K ? 256u : 0u;
}

constexpr uint32_t block_bytes(uint32_t t)
{
    return t == T_F32 ? 4u : t == T_F16 ? 2u : t == T_Q8_0 ? 34u : t == T_Q4_0 ? 18u
         : t == T_Q5_0 ? 22u : t == T_Q4_K ? 144u : t == T_Q5_K ? 176u
         : t == T_Q6_K ? 210u : 0u;
}

constexpr bool type_supported(uint32_t t) { return block_bytes(t) != 0; }

// Bytes of zero padding after every uploaded matrix: the GEMV kernels read
// whole aligned windows and two-block items, which may run up to this far past
// the last block of the matrix.
constexpr size_t kTailPad = 512;

// How a matrix is mat-vec'd; fixed at upload time.
struct Plan {
    int kind;              // 0 = generic per-element kernel, 1 = stream kernel family
    uint32_t g;            // rows per row group
    uint32_t n_groups;     // ceil(rows / g)
    uint32_t ni;           // items (64- or 32-element units) per row group
    uint32_t tsub;         // team lanes if <= 64, else 0 (a team spans wpt waves)
    uint32_t ts;           // team lanes
    uint64_t group_bytes;  // bytes per row group
    uint32_t n_teams;      // teams in the grid
    uint32_t grid, block;  // launch shape
    uint32_t R;            // row groups per batch
    uint32_t n_batches;    // ceil(n_groups / R)
    uint32_t per_team;     // batches each team runs
    uint32_t wpt;          // waves per team when a team spans several waves
    uint32_t chunk;        // batches per partial-sum flush (several-wave teams)
    uint32_t red_off;      // LDS offset of the partial-sum slots
    uint32_t lds;          // dynamic LDS bytes
    const void *fn;        // kernel chosen for this matrix
    const void *fn_norm;   // the same kernel with the fused RMSNorm input
    const void *fn_silu;   // the same kernel with the silu(g) * u input
    const void *fn_norm_glu;  // RMSNorm input, [gate; up] rows paired into silu(g) * u
    bool rp;               // the kernels read the repacked layout (launch_repack)
    // plain mat-vec through the LDS ring kernel (gemv_ring) where it applies:
    const void *fn_ring;   // nullptr otherwise
    uint32_t ring_grid, ring_block, ring_per, ring_lds, ring_slot2;
    // plain mat-vec through the wave-private column kernel (gemv_wave, repacked
    // Q4_K rows of 96 or 112 items) where it applies; it takes precedence
    const void *fn_wave;   // nullptr otherwise
    uint32_t wave_grid;
};

}  // namespace qg

// Launchers implemented in qgemv_kernels.hip (C++ linkage, library-internal).
struct ihipStream_t;
namespace qg {
// rp: plan the kernels of the repacked layout where the type has one (Q8_0,
// Q4_K, Q5_K, Q6_K with whole row groups; Plan::rp tells whether it applied).
int make_plan(uint32_t type, size_t rows, size_t cols, int n_cu, Plan *p, bool rp = false);
// Whether make_plan(..., rp = true) would give a repacked-layout plan.
bool repack_eligible(uint32_t type, const Plan &p, size_t rows);
// dst = the repacked layout of src's n_groups row groups (same size); both
// device pointers; asynchronous.
int launch_repack(uint32_t type, const Plan &p, const uint8_t *src, uint8_t *dst, ihipStream_t *stream);
int launch_gemv(uint32_t type, const Plan &p, const uint8_t *w, size_t nbytes, size_t rows,
                size_t cols, const float *x, float *y, ihipStream_t *stream);
// y = W · (rmsnorm(xa + xb) * nw) with the stream kernel (kind 1 plans only;
// -1 otherwise); sum_out (may be NULL) receives xa + xb.  xa, xb, nw,
// sum_out: cols floats, 16-byte aligned.
int launch_gemv_norm(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *xa, const float *xb, const float *nw, float eps, float *sum_out,
                     float *y, ihipStream_t *stream);
// W = [gate; up] (each half a whole number of row groups, teams of one wave
// or less; -1 otherwise): y[r] = silu(gate_r · x) * (up_r · x) for
// r < rows / 2, x = rmsnorm(xa + xb) * nw as in launch_gemv_norm.
int launch_gemv_norm_glu(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                         const float *xa, const float *xb, const float *nw, float eps, float *sum_out,
                         float *y, ihipStream_t *stream);
// y1 = W1 · x and y2 = W2 · x, x = rmsnorm(xa + xb) * nw, in one launch (two
// matrices with the same cols, teams of one wave or less, both with one row
// per group or both with several, supported type pairs Q4_K/Q5_K with Q6_K;
// -1 otherwise).  sum_out (may be
// NULL) receives xa + xb.  n_cu: the device's compute units (both parts are
// sized to be resident together).
int launch_gemv_norm_pair(uint32_t t1, const Plan &p1, const uint8_t *w1, size_t nbytes1, size_t rows1, float *y1,
                          uint32_t t2, const Plan &p2, const uint8_t *w2, size_t nbytes2, size_t rows2, float *y2,
                          size_t cols, const float *xa, const float *xb, const float *nw, float eps,
                          float *sum_out, int n_cu, ihipStream_t *stream);
// y = W · (silu(g) * u) with the stream kernel (kind 1 plans only; -1
// otherwise).  g, u: cols floats, 16-byte aligned.
int launch_gemv_silu(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *g, const float *u, float *y, ihipStream_t *stream);
int launch_gemv_generic(uint32_t type, const uint8_t *w, size_t rows, size_t cols,
                        const float *x, float *y, ihipStream_t *stream);
int launch_dequant(uint32_t type, const uint8_t *w, size_t n_elements, float *out,
                   ihipStream_t *stream);
int launch_dequantize_row(uint32_t type, const uint8_t *w, size_t rows, size_t cols,
                          size_t row, float *out, ihipStream_t *stream);
// the same with the row index read from device memory when the kernel runs
int launch_dequantize_row_dev(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const uint32_t *d_row,
                              float *out, ihipStream_t *stream);
int launch_fill(float *out, size_t n, float v, ihipStream_t *stream);
// Floats of the per-GPU static scratch array (1 MiB) of the no-allocation
// entry point, and its device address on `device` (made current); -2 if
// the runtime cannot resolve it.
constexpr size_t kNoAllocScratchFloats = 262144;
int scratch_address(int device, float **ptr);
int launch_stream_read(const void *buf, size_t nbytes, uint32_t *out, ihipStream_t *stream);
// out = silu(g) * u elementwise
int launch_silu_mul(const float *g, const float *u, float *out, size_t n, ihipStream_t *stream);
// out = rmsnorm(a (+ b)) * w in one workgroup; sum_out (may be NULL) = a + b.
int launch_rmsnorm(const float *a, const float *b, float *sum_out, const float *w, float *out, size_t n,
                   float eps, ihipStream_t *stream);
}  // namespace qg
