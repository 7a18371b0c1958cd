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
    const void *fn_attn;   // the same kernel with the two-range attention merge input
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
// dst = the GGUF layout of the repacked src (the inverse of launch_repack;
// p: the repacked plan, p.rp)
int launch_unrepack(uint32_t type, const Plan &p, const uint8_t *src, uint8_t *dst, ihipStream_t *stream);
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
// y = W · x with x the attention output of n_heads heads of hd elements,
// merged from two position ranges: part[r * cols + i] is range r's
// unnormalised output sum_j exp(s_j - m) v_j[i], ml[2 (r n_heads + h)] and
// ml[2 (r n_heads + h) + 1] its (m, sum_j exp(s_j - m)) for head h, and
// x[i] = sum_r w_r part_r[i] with w_r = exp(m_r - M) / sum_r' exp(m_r' - M) l_r'.
// Stream kernel plans of the fixed-point types only (-1 otherwise); part
// 16-byte aligned, cols = n_heads * hd, hd a multiple of 16.
int launch_gemv_attn(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *part, const float *ml, uint32_t n_heads, uint32_t hd, float *y,
                     ihipStream_t *stream);
int launch_gemv_generic(uint32_t type, const uint8_t *w, size_t rows, size_t cols,
                        const float *x, float *y, ihipStream_t *stream);
// The plain mat-vec in f32 (each product rounded to f32, summed in f32), one
// wave per row, from the matrix's stream-kernel bytes: the repacked layout
// when p.rp, the GGUF one otherwise.  x, y: 4-byte aligned.
int launch_gemv_f32(uint32_t type, const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                    const float *x, float *y, ihipStream_t *stream);
int launch_dequant(uint32_t type, const uint8_t *w, size_t n_elements, float *out,
                   ihipStream_t *stream);
int launch_dequantize_row(uint32_t type, const uint8_t *w, size_t rows, size_t cols,
                          size_t row, float *out, ihipStream_t *stream);
// the same with the row index read from device memory when the kernel runs
int launch_dequantize_row_dev(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const uint32_t *d_row,
                              float *out, ihipStream_t *stream);
int launch_fill(float *out, size_t n, float v, ihipStream_t *stream);
// Batched prefill (qg_prefill.hip): tokens per chunk, supported matrix types,
// and the launchers of its kernels (0 = launched, -1 = shape not supported,
// -2 = launch failure).  x of every token t scaled per 256-element group g by
// a power of two 2^e_tg, xs = x 2^e_tg, as two f16 pieces in xp (4 n
// kPfMaxTokens bytes: per 128-element chunk the 32 KB image of the GEMM's
// LDS buffer, qgp::pf_xoff), the sums of xs per 32-element segment k at
// rec[64 k + t] (two f16 pieces, hi | lo << 16) and 2^-e_tg at
// rec[64 (n / 32) + 64 g + t] (rec holds 64 (n / 32 + ceil(n / 256))
// floats).  GEMM matrices have cols % 128 == 0; outputs are K-split: slice s
// of a result lives sstride floats after slice 0, and its consumer sums the
// slices.
constexpr uint32_t kPfMaxTokens = 64;
bool prefill_type_supported(uint32_t type);
// one matrix of a grouped prefill GEMM: y[t * ldy + r] (+ s * sstride); w in
// the GGUF layout, or (rp) in the repacked layout of launch_repack with g
// rows, ni items and gb bytes per row group
struct PfMat {
    uint32_t type;
    const uint8_t *w;
    size_t rows;
    float *y;
    bool rp;
    uint32_t g, ni;
    size_t gb;
};
uint32_t pf_tiles(size_t rows);
// slices of the K split of a GEMM over `tiles` row tiles and nseg sub-blocks
uint32_t pf_split(uint32_t tiles, uint32_t nseg);
// 1..3 matrices (16-byte aligned) of `cols` columns over the same x, K split
// into `slices` slices (1 .. cols / 32; pf_split of the group's row tiles)
// that every matrix writes, empty or not; one launch per run of one type
int launch_pf_gemm(const PfMat *mats, int n_mats, size_t cols, const uint16_t *xp, const float *rec, uint32_t ntok,
                   uint32_t ldy, uint32_t slices, size_t sstride, ihipStream_t *stream);
// x = sum of the na slices of a (nb of b); mode 0: x = a; 1: x = (a + b) *
// nw, the numerator of rmsnorm(a + b) * nw (b may be NULL; sum_out, if not
// NULL, receives a + b and must not alias a or b; ss_out[t * ceil(n / 256) +
// g] receives the sum of (a + b)^2 over group g: the consumer of the GEMM
// over x multiplies its output by 1 / rms); 2: x = silu(a r) * (b r) with
// r = 1 / rms of the mode-1 call (over pre_n elements) that left its sums at
// pre, or r = 1 if pre is NULL.  Rows of lda floats.
int launch_pf_planes(const float *a, uint32_t na, const float *b, uint32_t nb, size_t sstride, float *sum_out,
                     const float *nw, size_t n, size_t lda, int mode, const float *pre, size_t pre_n, float eps,
                     float *ss_out, uint16_t *xp, float *rec, uint32_t ntok, ihipStream_t *stream);
// out[i] = sum of the ns slices of x[i], i < n
int launch_pf_sum(const float *x, uint32_t ns, size_t sstride, size_t n, float *out, ihipStream_t *stream);
// q, k, v of the QKV GEMM over a mode-1 x (norm sums at ss, over ss_n
// elements) times 1 / rms, plus the biases, RoPE of q and k, the KV append;
// q and k summed over ns slices, v over ns_v
int launch_pf_qkv_post(float *qkv, uint32_t ldq, uint32_t ns, uint32_t ns_v, size_t sstride, const float *ss,
                       size_t ss_n, float eps,
                       const float *bq, const float *bk, const float *bv, float *kc, float *vc, const float *cos_t,
                       const float *sin_t, uint32_t q_dim, uint32_t kv_dim, uint32_t hd, uint32_t pos0, uint32_t slot0,
                       uint32_t ntok, ihipStream_t *stream);
// causal attention of the chunk's tokens (head_dim 64, 128 or 256)
int launch_pf_attention(const float *qkv, uint32_t ldq, const float *kc, const float *vc, float *out, uint32_t n_heads,
                        uint32_t hd, uint32_t kv_dim, uint32_t n_rep, float scale, uint32_t slot0, uint32_t ntok,
                        ihipStream_t *stream);
// rows d_rows[0..n) of a matrix, dequantized into out + i * ldo
int launch_dequantize_rows_dev(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const uint32_t *d_rows,
                               uint32_t n, float *out, size_t ldo, ihipStream_t *stream);
// Floats of the per-GPU static scratch array (1 MiB) of the no-allocation
// entry point, and its device address on `device` (made current); -2 if
// the runtime cannot resolve it.
constexpr size_t kNoAllocScratchFloats = 262144;
int scratch_address(int device, float **ptr);
// out = silu(g) * u elementwise
int launch_silu_mul(const float *g, const float *u, float *out, size_t n, ihipStream_t *stream);
// out = rmsnorm(a (+ b)) * w in one workgroup; sum_out (may be NULL) = a + b.
int launch_rmsnorm(const float *a, const float *b, float *sum_out, const float *w, float *out, size_t n,
                   float eps, ihipStream_t *stream);
}  // namespace qg
