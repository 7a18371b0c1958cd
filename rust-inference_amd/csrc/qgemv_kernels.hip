// qgemv_kernels.hip -- gfx950 kernels for the dequantize-per-block mat-vec
// (QuantizedMatrix::mat_vec_mul, yudono/rust-inference src/quant.rs:178-206).
//
// Compiled with -ffp-contract=off: the bit-exact element decoders below must
// round every product separately, exactly like src/quant.rs.  The GEMV paths
// ask for fused multiply-adds explicitly with __builtin_fmaf.
//
// Kernels:
//   dequant_k<T>      whole-matrix decode to f32, bit-exact (quant.rs:356-840)
//   deq_row_k<T>      one row with the reference's straddle placement
//                     (quant.rs:152-174)
//   gemv_generic<T>   one wave per row, per-element decode; any shape
//   gemv_stream<T,..> the fast path: a persistent workgroup stages x once in
//                     LDS (as fixed-point planes for quant types); a "team"
//                     of lanes owns whole row groups, each lane one 64-weight
//                     item (32 for F32) whose x slice stays in VGPRs while the
//                     team streams its row groups
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include <type_traits>

#include "qg_common.h"

namespace qg {

// ---------------------------------------------------------------- helpers

// Opaque AND: hides the mask from the instruction combiner, which would
// otherwise turn "(w & 0x0F0F0F0F) >> 8k & 0xFF" into one v_bfe per byte
// instead of one v_and per four bytes feeding v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t andm(uint32_t a, uint32_t m)
{
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(a));
    return r;
}

// byte b of v as f32 (v_cvt_f32_ubyte<b>)
__device__ __forceinline__ float ub(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

__device__ __forceinline__ float h2f(uint32_t h16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xFFFFu));
}

// quant.rs:302-342.  v_cvt_f32_f16 is exact for every non-NaN half; the
// reference returns the canonical quiet NaN 0x7FC00000 for every NaN input.
__device__ __forceinline__ float h2f_exact(uint32_t h)
{
    h &= 0xFFFFu;
    if ((h & 0x7C00u) == 0x7C00u && (h & 0x3FFu) != 0u) return __uint_as_float(0x7FC00000u);
    return h2f(h);
}

__device__ __forceinline__ uint32_t rd16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// 16 bytes from a 4-byte-aligned address (global_load_dwordx4)
struct __attribute__((packed, aligned(4))) U4a { uint32_t a, b, c, d; };

// quant.rs:606-615 on the three scale dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11)
__device__ __forceinline__ void k4sm(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                     uint32_t &sc, uint32_t &m)
{
    const uint32_t sh = (j & 3u) * 8u;
    if (j < 4u) {
        sc = (s0 >> sh) & 63u;
        m = (s1 >> sh) & 63u;
    } else {
        sc = ((s2 >> sh) & 15u) | (((s0 >> (sh + 6u)) & 3u) << 4);
        m = ((s2 >> (sh + 4u)) & 15u) | (((s1 >> (sh + 6u)) & 3u) << 4);
    }
}

// The scales and mins of sub-blocks j = 2p and 2p+1 (quant.rs:606-615) as
// bytes 0 and 1 of SC and MN, branch-free for a per-lane pair index p.
__device__ __forceinline__ void k4pair(uint32_t p, uint32_t s0, uint32_t s1, uint32_t s2,
                                       uint32_t &SC, uint32_t &MN)
{
    const bool hs = p >= 2u;                     // j >= 4: 4+2 bit splice
    const uint32_t sh = (p & 1u) * 16u;          // 8 * (j mod 4)
    const uint32_t A = hs ? s2 : s0, C = hs ? (s2 >> 4) : s1;
    const uint32_t mA = hs ? 0x0F0Fu : 0x3F3Fu, mB = hs ? 0x3030u : 0u;
    SC = ((A >> sh) & mA) | ((s0 >> (sh + 2u)) & mB);
    MN = ((C >> sh) & mA) | ((s1 >> (sh + 2u)) & mB);
}

// ------------------------------------------- bit-exact element decoders
// elem_t<T>(b, i) = value i of a block, as src/quant.rs:82-149 computes it,
// where b[o] is byte o of the block in the GGUF layout: a pointer to the
// block, or a view that gathers the block's bytes from the repacked layout
// (RpBlock below).  elem<T>(block, i) is the pointer form.

template <class B> __device__ __forceinline__ uint32_t bytes16(const B &b, uint32_t o)
{
    return (uint32_t)b[o] | ((uint32_t)b[o + 1u] << 8);
}
template <class B> __device__ __forceinline__ uint32_t bytes32(const B &b, uint32_t o)
{
    return bytes16(b, o) | (bytes16(b, o + 2u) << 16);
}

template <uint32_t T, class B> __device__ __forceinline__ float elem_t(const B &b, uint32_t i)
{
    if constexpr (T == T_F32) {
        if constexpr (std::is_pointer<B>::value) return __uint_as_float(*(const uint32_t *)b);
        else return __uint_as_float(bytes32(b, 0u));
    } else if constexpr (T == T_F16) {
        return h2f_exact(bytes16(b, 0u));
    } else if constexpr (T == T_Q8_0) {
        const float d = h2f_exact(bytes16(b, 0u));                 // quant.rs:107
        return d * (float)(int8_t)b[2u + i];                       // quant.rs:110
    } else if constexpr (T == T_Q4_0) {
        const float d = h2f_exact(bytes16(b, 0u));
        const uint32_t v = b[2u + i / 2u];                         // quant.rs:117-118 (interleaved)
        const int nib = (i & 1u) ? (int)(v >> 4) : (int)(v & 15u);
        return d * (float)(nib - 8);
    } else if constexpr (T == T_Q5_0) {
        const float d = h2f_exact(bytes16(b, 0u));
        const uint32_t qh = bytes16(b, 2u) | (bytes16(b, 4u) << 16);
        const uint32_t xl = i < 16u ? ((uint32_t)b[6u + i] & 15u) : ((uint32_t)b[6u + i - 16u] >> 4);
        const uint32_t xh = ((qh >> i) & 1u) << 4;                 // quant.rs:126-135
        return d * (float)((int)(xl | xh) - 16);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const float d = h2f_exact(bytes16(b, 0u)), dmin = h2f_exact(bytes16(b, 2u));
        const uint32_t j = i >> 5, l = i & 31u;
        uint32_t sc, m;
        k4sm(j, bytes32(b, 4u), bytes32(b, 8u), bytes32(b, 12u), sc, m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;      // quant.rs:218-219, 249-250
        if constexpr (T == T_Q4_K) {
            const uint32_t q = b[16u + (j >> 1) * 32u + l];
            const uint32_t nib = (j & 1u) ? (q >> 4) : (q & 15u);
            return d1 * (float)nib - m1;                           // quant.rs:224-225
        } else {
            const uint32_t q = b[48u + (j >> 1) * 32u + l];
            const uint32_t lo = (j & 1u) ? (q >> 4) : (q & 15u);
            const uint32_t hi = (((uint32_t)b[16u + l] >> j) & 1u) ? 16u : 0u;   // quant.rs:238-260
            return d1 * (float)(lo + hi) - m1;
        }
    } else {
        static_assert(T == T_Q6_K, "type");
        const uint32_t n = i >> 7, rr = i & 127u, k = rr >> 5, l = rr & 31u, is = l >> 4;
        const uint32_t qlb = b[64u * n + l + 32u * (k & 1u)];
        const uint32_t nib = k >= 2u ? (qlb >> 4) : (qlb & 15u);
        const uint32_t hb = ((uint32_t)b[128u + 32u * n + l] >> (2u * k)) & 3u;
        const int q = (int)(nib | (hb << 4));
        const float sc = (float)(int8_t)b[192u + 8u * n + is + 2u * k];
        const float d = h2f_exact(bytes16(b, 208u));
        return d * sc * (float)(q - 32);                           // quant.rs:286-289
    }
}

template <uint32_t T> __device__ __forceinline__ float elem(const uint8_t *b, uint32_t i)
{
    return elem_t<T>(b, i);
}

// ------------------------------------------------------------- dequant

template <uint32_t T>
__global__ void __launch_bounds__(256) dequant_k(const uint8_t *__restrict__ w, uint64_t n,
                                                 float *__restrict__ out)
{
    constexpr uint32_t BS = block_elems(T), BB = block_bytes(T);
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; f < n; f += stride)
        out[f] = elem<T>(w + (f / BS) * BB, (uint32_t)(f % BS));
}

// quant.rs:152-174: writes only the positions the reference writes.  The
// row is `row`, or d_row[blockIdx.y] when d_row is not NULL (row indices
// that live in device memory, e.g. the token ids of a decode step or a
// prefill chunk), written to out + blockIdx.y * ldo; rows past the end write
// nothing.
template <uint32_t T>
__global__ void __launch_bounds__(256) deq_row_k(const uint8_t *__restrict__ w, uint64_t rows,
                                                 uint64_t cols, uint64_t row_arg,
                                                 const uint32_t *__restrict__ d_row,
                                                 float *__restrict__ out, uint64_t ldo)
{
    constexpr uint64_t BS = block_elems(T), BB = block_bytes(T);
    const uint64_t row = d_row ? (uint64_t)d_row[blockIdx.y] : row_arg;
    out += blockIdx.y * ldo;
    if (row >= rows) return;
    const uint64_t nbpr = (cols + BS - 1) / BS;
    const uint64_t start_block = row * cols / BS, col_off = row * cols % BS;
    const uint64_t total = rows * cols;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < nbpr * BS;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t bi = idx / BS, k = idx % BS, bidx = start_block + bi;
        if (bidx * BS >= total) continue;                       // quant.rs:163 (break)
        const uint64_t src_start = bi == 0 ? col_off : 0;
        const uint64_t lim = cols + col_off - bi * BS;
        const uint64_t src_end = BS < lim ? BS : lim;
        if (k < src_start || k >= src_end) continue;
        const uint64_t dst = bi == 0 ? k - col_off : bi * BS + k;  // quant.rs:168
        if (dst < cols) out[dst] = elem<T>(w + bidx * BB, (uint32_t)k);
    }
}

constexpr int kProPlain = 0, kProNorm = 1, kProSilu = 2, kProAttn = 3;

// silu(x) = x / (1 + exp(-x)), in the two branches of math.rs:137-146
__device__ __forceinline__ float silu1(float x)
{
    if (x >= 0.0f) {
        const float e = expf(-x);
        return x / (1.0f + e);
    }
    const float e = expf(x);
    return x * e / (1.0f + e);
}

__global__ void fill_k(float *out, uint64_t n, float v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = v;
}

// out = rmsnorm(a (+ b)) * w (math.rs:237-257); with b, sum_out (may be
// NULL) receives a + b.  One workgroup of kNormBlock threads.
constexpr int kNormBlock = 1024;
__global__ void __launch_bounds__(kNormBlock) rmsnorm_k(const float *__restrict__ a,
                                                        const float *__restrict__ b,
                                                        float *__restrict__ sum_out,
                                                        const float *__restrict__ w,
                                                        float *__restrict__ out, uint32_t n, float eps)
{
    __shared__ float red[kNormBlock / 64];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float x = b ? a[i] + b[i] : a[i];
        if (sum_out) sum_out[i] = x;
        ss += x * x;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (uint32_t i = 0; i < blockDim.x / 64u; i++) tot += red[i];
    const float rms = sqrtf(tot / (float)n + eps);
    const float scale = 1.0f / rms;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float x = b ? a[i] + b[i] : a[i];
        out[i] = x * scale * w[i];
    }
}

// out = silu(g) * u elementwise (mlp.rs:36-43)
__global__ void __launch_bounds__(256) silu_mul_k(const float *__restrict__ g, const float *__restrict__ u,
                                                  float *__restrict__ out, uint64_t n)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = silu1(g[i]) * u[i];
}

// ------------------------------------------------------- generic GEMV

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <uint32_t T>
__global__ void __launch_bounds__(256) gemv_generic(const uint8_t *__restrict__ w,
                                                    const float *__restrict__ x,
                                                    float *__restrict__ y, uint32_t rows,
                                                    uint32_t cols)
{
    constexpr uint64_t BS = block_elems(T), BB = block_bytes(T);
    const uint32_t row = blockIdx.x * 4u + threadIdx.x / 64u, lane = threadIdx.x & 63u;
    if (row >= rows) return;                                    // wave-uniform
    const uint64_t f0 = (uint64_t)row * cols;
    float acc = 0.0f;
    for (uint32_t c = lane; c < cols; c += 64u) {
        const uint64_t f = f0 + c;
        acc = __builtin_fmaf(elem<T>(w + (f / BS) * BB, (uint32_t)(f % BS)), x[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// ------------------------------------------------- repacked-layout view
//
// RpBlock<T>{grp, ni, blk}[o] = byte o of block blk of a row group, in the
// GGUF layout, read from the group's repacked bytes (the layout repack_k
// writes; see there): the map from a GGUF offset to the repacked one.  Q5_K's
// qh bytes are reassembled from the bits its four items keep.
template <uint32_t T> struct RpBlock {
    const uint8_t *grp;
    uint32_t ni, blk;
    __device__ uint32_t operator[](uint32_t o) const
    {
        if constexpr (T == T_Q8_0) {
            const uint32_t it = blk >> 1, h = blk & 1u;
            if (o < 2u) return grp[64u * ni + 4u * it + 2u * h + o];
            const uint32_t k = 32u * h + o - 2u;
            return grp[((k >> 4) * ni + it) * 16u + (k & 15u)];
        } else if constexpr (T == T_Q4_K) {
            if (o < 16u) return grp[16u * blk + o];
            const uint32_t q = o - 16u, it = 2u * blk + (q >> 6);
            return grp[(ni >> 1) * 16u + (((q & 63u) >> 4) * ni + it) * 16u + (q & 15u)];
        } else if constexpr (T == T_Q5_K) {
            const uint32_t H = (ni >> 2) * 16u;
            if (o < 16u) return grp[16u * blk + o];
            if (o >= 48u) {
                const uint32_t q = o - 48u, it = 4u * blk + (q >> 5), k = q & 31u;
                return grp[H + ((k >> 4) * ni + it) * 16u + (k & 15u)];
            }
            // qh byte m: bits 2q, 2q + 1 live in item q's word w at 8 bb + 2 t'
            const uint32_t m = o - 16u, w = m >> 4, tp = (m >> 2) & 3u, bb = m & 3u;
            uint32_t v = 0;
            for (uint32_t q = 0; q < 4u; q++) {
                const uint8_t *pw = grp + H + 32u * ni + 8u * (4u * blk + q) + 4u * w + bb;
                v |= (((uint32_t)*pw >> (2u * tp)) & 3u) << (2u * q);
            }
            return v;
        } else {
            static_assert(T == T_Q6_K, "repacked types");
            if (o < 128u) {
                const uint32_t n = o >> 6, r = o & 63u, it = 4u * blk + 2u * n + ((r & 31u) >> 4);
                return grp[((r >> 5) * ni + it) * 16u + (r & 15u)];
            }
            if (o < 192u) {
                const uint32_t q = o - 128u, it = 4u * blk + 2u * (q >> 5) + ((q & 31u) >> 4);
                return grp[(2u * ni + it) * 16u + (q & 15u)];
            }
            if (o < 208u) {
                const uint32_t q = o - 192u, it = 4u * blk + 2u * (q >> 3) + (q & 1u);
                return grp[48u * ni + 4u * it + ((q & 7u) >> 1)];
            }
            return grp[52u * ni + 2u * blk + (o - 208u)];
        }
    }
};

// ------------------------------------------------------ x in fixed point
//
// Quant types multiply integer codes by x with integer dot products.  Every
// 32-element segment of x, with m = max |x| over the segment and
// k = kFix / m, becomes the integers Y = rint(x * k), |Y| < 2^22, written in
// balanced base 256: Y = e0 + 256 e1 + 65536 e2 with every digit a signed
// byte in [-128, 127].  For any byte-sized weight code q (signed or not)
//     sum q*Y = sdot4(q, e0) + 256 * sdot4(q, e1) + 65536 * sdot4(q, e2)
// exactly, and sum q*x = (sum q*Y) / k, within about 2^-22 of m per element.
// Signed digits let a high nibble be used in place, unshifted, as the signed
// byte 16*h - 128 (one AND-XOR): sum h*Y = (sum (16h - 128)*Y + 128 sum Y) / 16.
// Every segment also keeps the record {1/k, sum x[0..16), sum x[16..32), sY},
// sY = sum of Y over the elements that high nibbles meet (all 32, or the odd
// half for Q4_0's even-then-odd order).  A segment whose sum is not finite
// (any inf or NaN in it) gets 1/k = NaN, so every dot product that uses it
// is NaN; the plain mat-vec kernels then recompute their rows in f32
// (row_dot_f32), which gives the reference's infinities and NaNs.  F16 and
// F32 weights keep x in f32.
//
// LDS layout (planes): segment g at byte 96g + 16(g/2) holds 32 bytes of e0,
// 32 of e1, 32 of e2 (16 bytes of padding per segment pair keep the per-lane
// reads below conflict-free); the segment records follow at `meta`.  Q4_0
// stores each segment's planes in even-then-odd element order, matching its
// interleaved nibbles.  f32 layout: float4 i of x at xl4[i + i/16].

constexpr float kFix = 4194000.0f;
// Largest k: 2^122, so that 1/k and the high-nibble factor (1/k) / 16 stay
// normal floats.  Segments with m >= kFix / 2^122 (about 7.9e-31) keep the
// full 22 bits; below that |Y| < m 2^122 (e.g. 12 bits at m = 1e-33).
constexpr float kMaxK = 5.316912e36f;
// A segment with max |x| above 2^64 is left to the f32 path (row_dot_f32):
// its fixed-point sums could overflow where the reference's f32 products do not.
constexpr float kDivertMax = 1.8446744e19f;
// fma(x, k, kMagic) holds rint(x * k) in its low mantissa bits for |x k| < 2^22
constexpr float kMagic = 12582912.0f;            // 1.5 * 2^23
constexpr int kMagicBits = 0x4B400000;

__device__ __forceinline__ uint32_t plane_off(uint32_t g) { return 96u * g + 16u * (g >> 1); }
__host__ __device__ constexpr uint32_t planes_bytes(uint32_t cols)
{
    return (cols / 64) * 208u + ((cols / 32) & 1u) * 96u;
}

// DPP move (gfx9 encodings): quad_perm 0x00-0xFF, row_mirror 0x140,
// row_half_mirror 0x141, row_bcast15 0x142, row_bcast31 0x143.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 ROW_MASK, 0xF, false));
}

// Sum over aligned groups of N lanes (N = 8, 16, 32, 64); the group's last
// lane ends up holding the group sum.
template <int N> __device__ __forceinline__ float group_sum(float v)
{
    v += dpp<0xB1>(v);                       // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);                       // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);                      // row_half_mirror
    if (N >= 16) v += dpp<0x140>(v);         // row_mirror
    if (N >= 32) v += dpp<0x142, 0xA>(v);    // row_bcast15 -> rows 1, 3
    if (N >= 64) v += dpp<0x143, 0xC>(v);    // row_bcast31 -> rows 2, 3
    return v;
}

template <int CTRL> __device__ __forceinline__ uint32_t dppu(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// max(|a|, |b|, |c|, |d|) (v_max3 with abs modifiers; no NaN canonicalisation)
__device__ __forceinline__ float absmax4(float4 v)
{
    float r;
    asm("v_max3_f32 %0, |%1|, |%2|, |%3|\n\tv_max_f32_e64 %0, |%4|, %0"
        : "=&v"(r) : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
    return r;
}

// Stage 16 consecutive elements of x, half h = c & 1 of segment g = c >> 1
// (q: its four float4), as fixed-point planes and the segment record; the two
// halves of a segment sit in adjacent lanes (c even in the even lane) that
// are active together, and each reduction over the segment is one DPP swap
// between them.  The sums use fixed trees: a half's sum of x is
// (t0 + t1) + (t2 + t3) with t_i = (x0 + x1) + (x2 + x3) over float4 i, and
// sY adds the float4s' exact integer sums the same way, then the two halves.
// Returns whether the segment diverts its rows to row_dot_f32 (a non-finite
// sum or max |x| > 2^64).
template <bool EVEN_ODD>
__device__ __forceinline__ bool stage_planes16(const uint4 (&q)[4], uint32_t c, uint8_t *lds, uint32_t meta)
{
    float4 v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = __builtin_bit_cast(float4, q[i]);
    const uint32_t h = c & 1u, g = c >> 1;
    uint32_t mb = max(max(__float_as_uint(absmax4(v[0])), __float_as_uint(absmax4(v[1]))),
                      max(__float_as_uint(absmax4(v[2])), __float_as_uint(absmax4(v[3]))));
    mb = max(mb, dppu<0xB1>(mb));
    const float m = __uint_as_float(mb);
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; i++) t[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float s = (t[0] + t[1]) + (t[2] + t[3]);   // this half's sum
    const float o = dpp<0xB1>(s);                    // the other half's
    const bool bad = !__builtin_isfinite(s + o);
    const float k = (m > 0.f && !bad) ? fminf(kFix * __builtin_amdgcn_rcpf(m), kMaxK) : 0.f;
    const float ik = bad ? __builtin_nanf("") : (k > 0.f ? __builtin_amdgcn_rcpf(k) : 0.f);
    const int off = 0x8080 - kMagicBits;
    uint32_t Y[4][4];
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        Y[i][0] = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].x, k, kMagic)) + off);
        Y[i][1] = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].y, k, kMagic)) + off);
        Y[i][2] = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].z, k, kMagic)) + off);
        Y[i][3] = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].w, k, kMagic)) + off);
        f[i] = (float)(EVEN_ODD ? (int)(Y[i][1] + Y[i][3]) - 2 * 0x8080
                                : (int)((Y[i][0] + Y[i][1]) + (Y[i][2] + Y[i][3])) - 4 * 0x8080);
    }
    float sy = (f[0] + f[1]) + (f[2] + f[3]);
    sy += dpp<0xB1>(sy);
    uint8_t *seg = lds + plane_off(g);
    if (!EVEN_ODD) {
        uint32_t w0[4], w1[4], w2[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t P01 = __builtin_amdgcn_perm(Y[i][1], Y[i][0], 0x05010400u);
            const uint32_t P23 = __builtin_amdgcn_perm(Y[i][3], Y[i][2], 0x05010400u);
            const uint32_t Q01 = __builtin_amdgcn_perm(Y[i][1], Y[i][0], 0x0C0C0602u);
            const uint32_t Q23 = __builtin_amdgcn_perm(Y[i][3], Y[i][2], 0x0C0C0602u);
            w0[i] = __builtin_amdgcn_perm(P23, P01, 0x05040100u) ^ 0x80808080u;
            w1[i] = __builtin_amdgcn_perm(P23, P01, 0x07060302u) ^ 0x80808080u;
            w2[i] = __builtin_amdgcn_perm(Q23, Q01, 0x05040100u);
        }
        *(uint4 *)(seg + 16u * h) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        *(uint4 *)(seg + 32u + 16u * h) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        *(uint4 *)(seg + 64u + 16u * h) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    } else {
        // float4 i holds elements 4i..4i+3 of the half: its even ones go to
        // even positions 8h + 2i, +1, its odd ones to 16 + 8h + 2i, +1
        uint32_t E[4], O[4], E2[4], O2[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            E[i] = __builtin_amdgcn_perm(Y[i][2], Y[i][0], 0x05010400u);
            O[i] = __builtin_amdgcn_perm(Y[i][3], Y[i][1], 0x05010400u);
            E2[i] = __builtin_amdgcn_perm(Y[i][2], Y[i][0], 0x0C0C0602u);
            O2[i] = __builtin_amdgcn_perm(Y[i][3], Y[i][1], 0x0C0C0602u);
        }
        auto lo2 = [](uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); };
        auto hi2 = [](uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); };
        *(uint2 *)(seg + 8u * h) = make_uint2(lo2(E[0], E[1]) ^ 0x80808080u, lo2(E[2], E[3]) ^ 0x80808080u);
        *(uint2 *)(seg + 16u + 8u * h) = make_uint2(lo2(O[0], O[1]) ^ 0x80808080u, lo2(O[2], O[3]) ^ 0x80808080u);
        *(uint2 *)(seg + 32u + 8u * h) = make_uint2(hi2(E[0], E[1]) ^ 0x80808080u, hi2(E[2], E[3]) ^ 0x80808080u);
        *(uint2 *)(seg + 48u + 8u * h) = make_uint2(hi2(O[0], O[1]) ^ 0x80808080u, hi2(O[2], O[3]) ^ 0x80808080u);
        *(uint2 *)(seg + 64u + 8u * h) = make_uint2(lo2(E2[0], E2[1]), lo2(E2[2], E2[3]));
        *(uint2 *)(seg + 80u + 8u * h) = make_uint2(lo2(O2[0], O2[1]), lo2(O2[2], O2[3]));
    }
    if (h == 0) *(float4 *)(lds + meta + 16u * g) = make_float4(ik, s, o, sy);
    return bad || m > kDivertMax;
}

// sum q*Y from the three plane dot products (see above)
__device__ __forceinline__ float fix3(int d0, int d1, int d2)
{
    return __builtin_fmaf((float)(d2 * 256 + d1), 256.0f, (float)d0);
}

// A lane's x for its item: S slots of SEG elements (planes or f32).
template <int S, int SEG> struct XP {
    uint32_t p[S][3][SEG / 4];
    float ik[S], sx[S], sy[S];
};
template <int S, int SEG> struct XF {
    float v[S * SEG];
    float sx[S];
};

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// first dot of a chain (VOP3P form with a zero accumulator: no v_mov 0)
__device__ __forceinline__ int sdot4z(uint32_t a, uint32_t b)
{
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// high nibbles as the signed bytes 16*h - 128
__device__ __forceinline__ uint32_t hi_s(uint32_t w) { return (w & 0xF0F0F0F0u) ^ 0x80808080u; }

// ------------------------------------------------------ team GEMV items
//
// An item is the unit one lane decodes per row group: 64 weights (32 for
// F32) in S slots of SEG weights that each lie in one row.  load() fetches
// the raw bytes of one item; compute() returns each slot's contribution to
// its row's dot product.

template <uint32_t T> struct Item;

// Q4_K (quant.rs:210-228): item = (block, half h): qs[64h .. 64h+64), pairs
// p = 2h, 2h+1, i.e. sub-blocks 4h .. 4h+3 as slots 0..3 (low nibbles of pair
// p -> sub-block 2p, high nibbles -> 2p+1).  128 weights per lane per row
// group halve the per-weight cost of the header, the reduction and the
// addressing against 64-weight items.
template <> struct Item<T_Q4_K> {
    static constexpr uint32_t IE = 128, S = 4, SEG = 32, NRAW = 20, UNIT = 256;
    static constexpr bool PLANES = true, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 1) * 256u + (it & 1u) * 128u + s * 32u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 1) * 144u; }
    __device__ static void load(const uint8_t *ip, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint4 h = *(const uint4 *)ip;
        const uint4 *q = (const uint4 *)(ip + 16u + (it & 1u) * 64u);
        const uint4 q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = q0.x; r[5] = q0.y; r[6] = q0.z; r[7] = q0.w;
        r[8] = q1.x; r[9] = q1.y; r[10] = q1.z; r[11] = q1.w;
        r[12] = q2.x; r[13] = q2.y; r[14] = q2.z; r[15] = q2.w;
        r[16] = q3.x; r[17] = q3.y; r[18] = q3.z; r[19] = q3.w;
    }
    // The same registers from the repacked row group (repack_k): the nb = ni/2
    // block headers, then piece k (16 bytes) of item it at nb*16 + (k*ni + it)*16,
    // so every load instruction of a wave reads one contiguous range.
    __device__ static void load_rp(const uint8_t *grp, uint32_t it, uint32_t ni, uint32_t (&r)[NRAW])
    {
        const uint4 h = *(const uint4 *)(grp + (it >> 1) * 16u);
        const uint8_t *q = grp + (ni >> 1) * 16u + it * 16u;
        const uint4 q0 = *(const uint4 *)q, q1 = *(const uint4 *)(q + ni * 16u);
        const uint4 q2 = *(const uint4 *)(q + 2u * ni * 16u), q3 = *(const uint4 *)(q + 3u * ni * 16u);
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = q0.x; r[5] = q0.y; r[6] = q0.z; r[7] = q0.w;
        r[8] = q1.x; r[9] = q1.y; r[10] = q1.z; r[11] = q1.w;
        r[12] = q2.x; r[13] = q2.y; r[14] = q2.z; r[15] = q2.w;
        r[16] = q3.x; r[17] = q3.y; r[18] = q3.z; r[19] = q3.w;
    }
    // sum q*x of the four sub-blocks, each in units of 1/k of its segment
    __device__ static void dots(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, float (&D)[4])
    {
        int acc[4][3];
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const uint32_t lo = andm(r[4 + 8 * pp], 0x0F0F0F0Fu), hi = hi_s(r[4 + 8 * pp]);
#pragma unroll
            for (int c = 0; c < 3; c++) {
                acc[2 * pp][c] = sdot4z(lo, x.p[2 * pp][c][0]);
                acc[2 * pp + 1][c] = sdot4z(hi, x.p[2 * pp + 1][c][0]);
            }
        }
#pragma unroll
        for (int t = 1; t < 8; t++)
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const uint32_t lo = andm(r[4 + 8 * pp + t], 0x0F0F0F0Fu), hi = hi_s(r[4 + 8 * pp + t]);
#pragma unroll
                for (int c = 0; c < 3; c++) {
                    acc[2 * pp][c] = sdot4(lo, x.p[2 * pp][c][t], acc[2 * pp][c]);
                    acc[2 * pp + 1][c] = sdot4(hi, x.p[2 * pp + 1][c][t], acc[2 * pp + 1][c]);
                }
            }
#pragma unroll
        for (int s = 0; s < 4; s += 2) {
            D[s] = fix3(acc[s][0], acc[s][1], acc[s][2]) * x.ik[s];
            // high nibbles: (sum (16h - 128) Y + 128 sY) / 16
            D[s + 1] = __builtin_fmaf(128.0f, x.sy[s + 1], fix3(acc[s + 1][0], acc[s + 1][1], acc[s + 1][2])) *
                       (x.ik[s + 1] * 0.0625f);
        }
    }
    __device__ static void scales(const uint32_t (&r)[NRAW], uint32_t it, uint32_t (&SC)[2], uint32_t (&MN)[2])
    {
        const uint32_t p0 = (it & 1u) * 2u;
        k4pair(p0, r[1], r[2], r[3], SC[0], MN[0]);
        k4pair(p0 + 1u, r[1], r[2], r[3], SC[1], MN[1]);
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                   float (&out)[S])
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        uint32_t SC[2], MN[2];
        scales(r, it, SC, MN);
        float D[4];
        dots(r, x, D);
#pragma unroll
        for (int s = 0; s < 4; s++)
            out[s] = __builtin_fmaf(d * ub(SC[s >> 1], s & 1), D[s], -(dmin * ub(MN[s >> 1], s & 1)) * x.sx[s]);
    }
    // sum of the four slots (one row per item)
    __device__ static float compute_sum(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it)
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        uint32_t SC[2], MN[2];
        scales(r, it, SC, MN);
        float D[4];
        dots(r, x, D);
        float u = ub(SC[0], 0) * D[0], mm = ub(MN[0], 0) * x.sx[0];
#pragma unroll
        for (int s = 1; s < 4; s++) {
            u = __builtin_fmaf(ub(SC[s >> 1], s & 1), D[s], u);
            mm = __builtin_fmaf(ub(MN[s >> 1], s & 1), x.sx[s], mm);
        }
        return __builtin_fmaf(d, u, -dmin * mm);
    }
};

// Q5_K (quant.rs:231-262): as Q4_K plus the fifth bit, bit j of qh[l].
template <> struct Item<T_Q5_K> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 20, UNIT = 256;
    static constexpr bool PLANES = true, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 2) * 256u + (it & 3u) * 64u + s * 32u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 2) * 176u; }
    __device__ static void load(const uint8_t *ip, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint4 h = *(const uint4 *)ip;
        const uint4 *qh = (const uint4 *)(ip + 16u);
        const uint4 *q = (const uint4 *)(ip + 48u + (it & 3u) * 32u);
        const uint4 h0 = qh[0], h1 = qh[1], q0 = q[0], q1 = q[1];
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = h0.x; r[5] = h0.y; r[6] = h0.z; r[7] = h0.w;
        r[8] = h1.x; r[9] = h1.y; r[10] = h1.z; r[11] = h1.w;
        r[12] = q0.x; r[13] = q0.y; r[14] = q0.z; r[15] = q0.w;
        r[16] = q1.x; r[17] = q1.y; r[18] = q1.z; r[19] = q1.w;
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                   float (&out)[S])
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        const uint32_t j = (it & 3u) * 2u;
        uint32_t SC, MN;
        k4pair(it & 3u, r[1], r[2], r[3], SC, MN);
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t w = r[12 + t], hb = r[4 + t];
            const uint32_t qa = andm(w, 0x0F0F0F0Fu) | (((hb >> j) & 0x01010101u) << 4);
            const uint32_t qb = andm(w >> 4, 0x0F0F0F0Fu) | (((hb >> (j + 1u)) & 0x01010101u) << 4);
            a0 = sdot4(qa, x.p[0][0][t], a0); a1 = sdot4(qa, x.p[0][1][t], a1); a2 = sdot4(qa, x.p[0][2][t], a2);
            b0 = sdot4(qb, x.p[1][0][t], b0); b1 = sdot4(qb, x.p[1][1][t], b1); b2 = sdot4(qb, x.p[1][2][t], b2);
        }
        out[0] = __builtin_fmaf(d * ub(SC, 0), fix3(a0, a1, a2) * x.ik[0], -(dmin * ub(MN, 0)) * x.sx[0]);
        out[1] = __builtin_fmaf(d * ub(SC, 1), fix3(b0, b1, b2) * x.ik[1], -(dmin * ub(MN, 1)) * x.sx[1]);
    }
    // The repacked row group (repack_k): the nb = ni/4 block headers, piece k
    // (16 bytes) of item it's 32 quant bytes at nb*16 + (k*ni + it)*16, and the
    // item's two qh bits per element as 8 bytes at nb*16 + 32ni + 8it -- word
    // w, byte b, bits 2t'+0/1 = bits j, j+1 of qh[16w + 4t' + b] -- so that
    // quant word t = 4w + t' takes its fifth bits with constant shifts.
    // r[4..5] hold those 8 bytes; r[6..11] are unused.
    __device__ static void load_rp(const uint8_t *grp, uint32_t it, uint32_t ni, uint32_t (&r)[NRAW])
    {
        const uint4 h = *(const uint4 *)(grp + (it >> 2) * 16u);
        const uint8_t *q = grp + (ni >> 2) * 16u + it * 16u;
        const uint4 q0 = *(const uint4 *)q, q1 = *(const uint4 *)(q + ni * 16u);
        const uint2 hb = *(const uint2 *)(grp + (ni >> 2) * 16u + 32u * ni + 8u * it);
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = hb.x; r[5] = hb.y;
#pragma unroll
        for (int k = 6; k < 12; k++) r[k] = 0u;
        r[12] = q0.x; r[13] = q0.y; r[14] = q0.z; r[15] = q0.w;
        r[16] = q1.x; r[17] = q1.y; r[18] = q1.z; r[19] = q1.w;
    }
    __device__ static void compute_rp(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                      float (&out)[S])
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        uint32_t SC, MN;
        k4pair(it & 3u, r[1], r[2], r[3], SC, MN);
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t w = r[12 + t], hb = r[4 + (t >> 2)] >> (2 * (t & 3));
            const uint32_t qa = andm(w, 0x0F0F0F0Fu) | ((hb & 0x01010101u) << 4);
            const uint32_t qb = andm(w >> 4, 0x0F0F0F0Fu) | (((hb >> 1) & 0x01010101u) << 4);
            a0 = sdot4(qa, x.p[0][0][t], a0); a1 = sdot4(qa, x.p[0][1][t], a1); a2 = sdot4(qa, x.p[0][2][t], a2);
            b0 = sdot4(qb, x.p[1][0][t], b0); b1 = sdot4(qb, x.p[1][1][t], b1); b2 = sdot4(qb, x.p[1][2][t], b2);
        }
        out[0] = __builtin_fmaf(d * ub(SC, 0), fix3(a0, a1, a2) * x.ik[0], -(dmin * ub(MN, 0)) * x.sx[0]);
        out[1] = __builtin_fmaf(d * ub(SC, 1), fix3(b0, b1, b2) * x.ik[1], -(dmin * ub(MN, 1)) * x.sx[1]);
    }
};

// Q6_K (quant.rs:265-292): item = (block, half n, i = l/16): 4 slots of 16,
// elements 128n + 32k + 16i + (0..15), k = 0..3.  Blocks are 210 bytes, so
// fields sit at 2-byte alignment: load aligned dword windows and realign
// with v_alignbyte.
template <> struct Item<T_Q6_K> {
    static constexpr uint32_t IE = 64, S = 4, SEG = 16, NRAW = 15, UNIT = 256;
    static constexpr bool PLANES = true, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 2) * 256u + ((it >> 1) & 1u) * 128u + s * 32u + (it & 1u) * 16u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 2) * 210u; }
    __device__ static void load(const uint8_t *ip, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint8_t *b = ip;
        const uint32_t n = (it >> 1) & 1u, i = it & 1u;
        const uint32_t mis = (uint32_t)((uintptr_t)b & 3u);
        const uint32_t *base = (const uint32_t *)(b - mis);
        const uint32_t oA = (64u * n + 16u * i) / 4u, oB = oA + 8u, oH = (128u + 32u * n + 16u * i) / 4u;
        const uint32_t oS = (192u + 8u * n) / 4u;
        const U4a A = *(const U4a *)(base + oA), B = *(const U4a *)(base + oB);
        const U4a H = *(const U4a *)(base + oH);
        const uint32_t A4 = base[oA + 4], B4 = base[oB + 4], H4 = base[oH + 4];
        const uint32_t S0 = base[oS], S1 = base[oS + 1], S2 = base[oS + 2], D = base[52];
        const uint32_t sh = mis;
        r[0] = __builtin_amdgcn_alignbyte(A.b, A.a, sh);
        r[1] = __builtin_amdgcn_alignbyte(A.c, A.b, sh);
        r[2] = __builtin_amdgcn_alignbyte(A.d, A.c, sh);
        r[3] = __builtin_amdgcn_alignbyte(A4, A.d, sh);
        r[4] = __builtin_amdgcn_alignbyte(B.b, B.a, sh);
        r[5] = __builtin_amdgcn_alignbyte(B.c, B.b, sh);
        r[6] = __builtin_amdgcn_alignbyte(B.d, B.c, sh);
        r[7] = __builtin_amdgcn_alignbyte(B4, B.d, sh);
        r[8] = __builtin_amdgcn_alignbyte(H.b, H.a, sh);
        r[9] = __builtin_amdgcn_alignbyte(H.c, H.b, sh);
        r[10] = __builtin_amdgcn_alignbyte(H.d, H.c, sh);
        r[11] = __builtin_amdgcn_alignbyte(H4, H.d, sh);
        r[12] = __builtin_amdgcn_alignbyte(S1, S0, sh);
        r[13] = __builtin_amdgcn_alignbyte(S2, S1, sh);
        r[14] = D >> (8u * sh);
    }
    // The same registers from the repacked row group (repack_k): pieces A, B
    // and H of every item piece-major (ni x 16 bytes each), then the item's
    // four scale bytes sc[8n + i + 2k] (ni x 4), then each block's d (nb x 2).
    // r[12] then holds the four scales in bytes 0..3.
    __device__ static void load_rp(const uint8_t *grp, uint32_t it, uint32_t ni, uint32_t (&r)[NRAW])
    {
        const uint4 A = *(const uint4 *)(grp + it * 16u);
        const uint4 B = *(const uint4 *)(grp + (ni + it) * 16u);
        const uint4 H = *(const uint4 *)(grp + (2u * ni + it) * 16u);
        r[12] = *(const uint32_t *)(grp + 48u * ni + it * 4u);
        r[14] = *(const uint16_t *)(grp + 52u * ni + (it >> 2) * 2u);
        r[0] = A.x; r[1] = A.y; r[2] = A.z; r[3] = A.w;
        r[4] = B.x; r[5] = B.y; r[6] = B.z; r[7] = B.w;
        r[8] = H.x; r[9] = H.y; r[10] = H.z; r[11] = H.w;
        r[13] = 0u;
    }
    // sum q*x per 16-weight slot k with scale sc_k (RP: scales as load_rp
    // leaves them; otherwise as load does)
    template <bool RP>
    __device__ static void compute_t(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                     float (&out)[S])
    {
        const float d = h2f(r[14]);
        const uint32_t i8 = (it & 1u) * 8u;
        int u0[4] = {0, 0, 0, 0}, u1[4] = {0, 0, 0, 0}, s2[4] = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t A = r[t], B = r[4 + t], H = r[8 + t];
            const uint32_t q[4] = {andm(A, 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u),
                                   andm(B, 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u),
                                   andm(A >> 4, 0x0F0F0F0Fu) | (H & 0x30303030u),
                                   andm(B >> 4, 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                u0[k] = sdot4(q[k], x.p[k][0][t], u0[k]);
                u1[k] = sdot4(q[k], x.p[k][1][t], u1[k]);
                s2[k] = sdot4(q[k], x.p[k][2][t], s2[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // sc[8n + i + 2k]: byte (i + 2(k&1)) of dword r[12 + k/2], or byte k of r[12] (RP)
            const int sc = RP ? __builtin_amdgcn_sbfe((int)r[12], 8 * k, 8)
                              : __builtin_amdgcn_sbfe((int)r[12 + (k >> 1)], (int)(i8 + 16u * (k & 1)), 8);
            out[k] = (d * (float)sc) * __builtin_fmaf(-32.0f, x.sx[k], fix3(u0[k], u1[k], s2[k]) * x.ik[k]);
        }
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                   float (&out)[S])
    {
        compute_t<false>(r, x, it, out);
    }
    __device__ static void compute_rp(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t it,
                                      float (&out)[S])
    {
        compute_t<true>(r, x, it, out);
    }
};

// Q8_0 (quant.rs:106-113): item = two blocks (68 bytes, 4-byte aligned).
// Block 0's codes sit at byte 2 (realigned), block 1's at byte 36 (aligned);
// the signed codes meet the signed digits directly.
template <> struct Item<T_Q8_0> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 17, UNIT = 64;
    static constexpr bool PLANES = true, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 68u; }
    __device__ static void load(const uint8_t *ip, uint32_t, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)ip;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const U4a u = *(const U4a *)(p + 4 * v);
            r[4 * v] = u.a; r[4 * v + 1] = u.b; r[4 * v + 2] = u.c; r[4 * v + 3] = u.d;
        }
        r[16] = p[16];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t,
                                   float (&out)[S])
    {
        const float dd[2] = {h2f(r[0]), h2f(r[8] >> 16)};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t q = s == 0 ? __builtin_amdgcn_alignbyte(r[t + 1], r[t], 2u) : r[9 + t];
                a0 = sdot4(q, x.p[s][0][t], a0); a1 = sdot4(q, x.p[s][1][t], a1); a2 = sdot4(q, x.p[s][2][t], a2);
            }
            out[s] = dd[s] * (fix3(a0, a1, a2) * x.ik[s]);
        }
    }
    // The repacked row group (repack_k): piece k (16 bytes) of the item's 64
    // codes at (k*ni + it)*16, then the item's two d halves at 64ni + 4it.
    __device__ static void load_rp(const uint8_t *grp, uint32_t it, uint32_t ni, uint32_t (&r)[NRAW])
    {
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint4 v = *(const uint4 *)(grp + (k * ni + it) * 16u);
            r[4 * k] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
        }
        r[16] = *(const uint32_t *)(grp + 64u * ni + 4u * it);
    }
    __device__ static void compute_rp(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t,
                                      float (&out)[S])
    {
        const float dd[2] = {h2f(r[16]), h2f(r[16] >> 16)};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t q = r[8 * s + t];
                a0 = sdot4(q, x.p[s][0][t], a0); a1 = sdot4(q, x.p[s][1][t], a1); a2 = sdot4(q, x.p[s][2][t], a2);
            }
            out[s] = dd[s] * (fix3(a0, a1, a2) * x.ik[s]);
        }
    }
};

// Q4_0 (quant.rs:114-121): two blocks (36 bytes).  Interleaved nibble order:
// byte j holds element 2j (low nibble) and 2j+1 (high nibble); x planes are
// staged even-then-odd to match.
template <> struct Item<T_Q4_0> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 9, UNIT = 64;
    static constexpr bool PLANES = true, EVEN_ODD = true;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 36u; }
    __device__ static void load(const uint8_t *ip, uint32_t, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)ip;
        const U4a u0 = *(const U4a *)p, u1 = *(const U4a *)(p + 4);
        r[0] = u0.a; r[1] = u0.b; r[2] = u0.c; r[3] = u0.d;
        r[4] = u1.a; r[5] = u1.b; r[6] = u1.c; r[7] = u1.d;
        r[8] = p[8];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t,
                                   float (&out)[S])
    {
        const float dd[2] = {h2f(r[0]), h2f(r[4] >> 16)};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = s == 0 ? __builtin_amdgcn_alignbyte(r[t + 1], r[t], 2u) : r[5 + t];
                const uint32_t lo = andm(q, 0x0F0F0F0Fu), hi = hi_s(q);
                a0 = sdot4(lo, x.p[s][0][t], a0); a1 = sdot4(lo, x.p[s][1][t], a1); a2 = sdot4(lo, x.p[s][2][t], a2);
                b0 = sdot4(hi, x.p[s][0][4 + t], b0); b1 = sdot4(hi, x.p[s][1][4 + t], b1);
                b2 = sdot4(hi, x.p[s][2][4 + t], b2);
            }
            const float qy = __builtin_fmaf(__builtin_fmaf(128.0f, x.sy[s], fix3(b0, b1, b2)), 0.0625f,
                                            fix3(a0, a1, a2));
            out[s] = dd[s] * __builtin_fmaf(-8.0f, x.sx[s], qy * x.ik[s]);
        }
    }
};

// Q5_0 (quant.rs:122-136): two blocks (44 bytes).  Element i < 16: low nibble
// of qs[i]; i >= 16: high nibble of qs[i-16]; fifth bit = bit i of qh.
__device__ __forceinline__ uint32_t spread4(uint32_t v)  // bit k of v -> bit 8k+4
{
    return (((v & 15u) * 0x00204081u) & 0x01010101u) << 4;
}
template <> struct Item<T_Q5_0> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 11, UNIT = 64;
    static constexpr bool PLANES = true, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 44u; }
    __device__ static void load(const uint8_t *ip, uint32_t, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)ip;
        const U4a u0 = *(const U4a *)p, u1 = *(const U4a *)(p + 4);
        r[0] = u0.a; r[1] = u0.b; r[2] = u0.c; r[3] = u0.d;
        r[4] = u1.a; r[5] = u1.b; r[6] = u1.c; r[7] = u1.d;
        r[8] = p[8]; r[9] = p[9]; r[10] = p[10];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XP<S, SEG> &x, uint32_t,
                                   float (&out)[S])
    {
        const float dd[2] = {h2f(r[0]), h2f(r[5] >> 16)};
        const uint32_t qh[2] = {__builtin_amdgcn_alignbyte(r[1], r[0], 2u), r[6]};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = s == 0 ? __builtin_amdgcn_alignbyte(r[t + 2], r[t + 1], 2u) : r[7 + t];
                const uint32_t lo = andm(q, 0x0F0F0F0Fu) | spread4(qh[s] >> (4 * t));
                const uint32_t hi = andm(q >> 4, 0x0F0F0F0Fu) | spread4(qh[s] >> (16 + 4 * t));
                a0 = sdot4(lo, x.p[s][0][t], a0); a1 = sdot4(lo, x.p[s][1][t], a1); a2 = sdot4(lo, x.p[s][2][t], a2);
                a0 = sdot4(hi, x.p[s][0][4 + t], a0); a1 = sdot4(hi, x.p[s][1][4 + t], a1);
                a2 = sdot4(hi, x.p[s][2][4 + t], a2);
            }
            out[s] = dd[s] * __builtin_fmaf(-16.0f, x.sx[s], fix3(a0, a1, a2) * x.ik[s]);
        }
    }
};

// F16: 64 halves (128 bytes, 16-byte aligned); x stays f32.
template <> struct Item<T_F16> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 32, UNIT = 64;
    static constexpr bool PLANES = false, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 128u; }
    __device__ static void load(const uint8_t *ip, uint32_t, uint32_t (&r)[NRAW])
    {
        const uint4 *p = (const uint4 *)ip;
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint4 u = p[v];
            r[4 * v] = u.x; r[4 * v + 1] = u.y; r[4 * v + 2] = u.z; r[4 * v + 3] = u.w;
        }
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XF<S, SEG> &x, uint32_t,
                                   float (&out)[S])
    {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float a = 0.f, b = 0.f;
#pragma unroll
            for (int t = 0; t < 16; t++) {
                a = __builtin_fmaf(h2f(r[16 * s + t]), x.v[32 * s + 2 * t], a);
                b = __builtin_fmaf(h2f(r[16 * s + t] >> 16), x.v[32 * s + 2 * t + 1], b);
            }
            out[s] = a + b;
        }
    }
};

// F32: 32 floats (128 bytes); x stays f32.
template <> struct Item<T_F32> {
    static constexpr uint32_t IE = 32, S = 1, SEG = 32, NRAW = 32, UNIT = 32;
    static constexpr bool PLANES = false, EVEN_ODD = false;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t) { return it * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 128u; }
    __device__ static void load(const uint8_t *ip, uint32_t, uint32_t (&r)[NRAW])
    {
        const uint4 *p = (const uint4 *)ip;
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint4 u = p[v];
            r[4 * v] = u.x; r[4 * v + 1] = u.y; r[4 * v + 2] = u.z; r[4 * v + 3] = u.w;
        }
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const XF<S, SEG> &x, uint32_t,
                                   float (&out)[S])
    {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            a = __builtin_fmaf(__uint_as_float(r[2 * t]), x.v[2 * t], a);
            b = __builtin_fmaf(__uint_as_float(r[2 * t + 1]), x.v[2 * t + 1], b);
        }
        out[0] = a + b;
    }
};

// ------------------------------------------------------- row streaming
//
// Row groups: g = UNIT / gcd(cols, UNIT) consecutive rows hold whole units
// (superblocks for K-quants, item pairs of blocks otherwise), so every row
// group starts at a whole item and rows of a group share items only where a
// row boundary falls inside one (each slot of an item lies in one row).  A
// team of lanes owns whole row groups: lane i decodes item i of each of them,
// and a team spans 1..8 waves (wpt) when a row group has more than 64 items.
// Row groups are dealt to teams band-wise: team t takes t, t + NT, t + 2NT,
// ... (NT = teams in the grid), so at any moment the whole grid streams one
// contiguous band of the matrix.

// Items that can return the sum of their slots directly (one row per item)
template <class I, class = void> struct HasSum : std::false_type {};
template <class I> struct HasSum<I, std::void_t<decltype(&I::compute_sum)>> : std::true_type {};

// x as the kernel stages it in LDS: planes + records (quant types) or padded f32
__host__ __device__ constexpr uint32_t image_bytes(bool planes, uint32_t cols)
{
    return planes ? planes_bytes(cols) + (cols / 32) * 16u : (cols / 4 + cols / 64 + 1) * 16u;
}

constexpr int kMaxWG = 768;        // 12 waves: 3 per SIMD
constexpr int kStage = 8;          // 16-byte pieces of x each thread loads before the weights
constexpr int kDepth = 2;          // batches of loads in flight per team

// Largest workgroup of the stream kernel for type T: 128-weight items hold a
// 96-VGPR x slice and need the register budget of 2 waves per SIMD.
template <uint32_t T> constexpr int wg_max() { return Item<T>::IE == 128 ? 512 : kMaxWG; }

struct StreamArgs {
    const uint8_t *w;
    const float *x;
    float *y;
    uint32_t nbytes, group_bytes, rows, cols, g, n_groups, ni;
    uint32_t n_teams;              // NT
    uint32_t per_team;             // batches every team runs
    uint32_t wpt;                  // waves per team (TSUB == 0)
    uint32_t chunk;                // batches per partial-sum flush (TSUB == 0)
    uint32_t red_off;              // LDS byte offset of the partial-sum slots
    uint32_t ring_slot2;           // gemv_ring: LDS byte offset of the third ring slot
    // fused RMSNorm of the input (NORM kernels): x = rmsnorm(x + xb) * nw
    const float *xb;               // second addend (the residual branch), cols floats
    const float *nw;               // norm weights, cols floats
    float *sum_out;                // if not NULL, workgroup 0 stores x + xb here
    float eps;
    // gate/up pairs (GLU kernels): the matrix is [gate; up] with glu_half row
    // groups each; y[r] = silu(gate_r . x) * (up_r . x), rows / 2 floats
    uint32_t glu_half;
    // two-range attention merge (kProAttn): x = range 0's partial output, xb =
    // range 1's, ml = their (m, l) per head, [range][att_nh][2]; heads of
    // att_hd elements
    const float *ml;
    uint32_t att_nh, att_hd;
};

// ------------------------------------------------- non-finite x: slow rows
//
// The fixed-point x of the quant types cannot carry inf or NaN, and a segment
// holding one gets 1/k = NaN, which would make every row NaN.  The reference
// sums w * x[c] one product at a time in f32 (quant.rs:195-204), so a row that
// meets +inf gives +inf, -inf gives -inf, and NaN only where signs mix, a
// weight is zero or x holds a NaN.  The plain mat-vec kernels therefore find
// out whether any segment of x was non-finite (or so large that the
// fixed-point sums could overflow where f32 products do not: max |x| over a
// segment > 2^64) -- the stream and ring kernels from per-wave flags,
// gemv_wave from its NaN row sums -- and if so recompute every row they own
// with row_dot_f32: the f32 sum of one rounded product per element.  Its order
// differs from the reference's, which changes only finite results; whether a
// sum is finite, +inf, -inf or NaN does not depend on the order.
// sum over c of w(row, c) * x[c] in f32 (wave-cooperative: `row` is
// wave-uniform and every lane of the wave takes part; all lanes get the sum)
template <uint32_t T, bool RP>
__device__ float row_dot_f32(const StreamArgs &a, uint32_t row)
{
    constexpr uint32_t BS = block_elems(T), BB = block_bytes(T);
    const uint32_t lane = threadIdx.x & 63u;
    float acc = 0.f;
    if constexpr (RP) {
        const uint32_t gr = row / a.g, rr = row - gr * a.g;
        const uint8_t *grp = a.w + (size_t)gr * a.group_bytes;
        for (uint32_t c = lane; c < a.cols; c += 64u) {
            const uint32_t f = rr * a.cols + c;
            const float p = elem_t<T>(RpBlock<T>{grp, a.ni, f / BS}, f % BS) * a.x[c];
            acc += p;
        }
    } else {
        const uint64_t f0 = (uint64_t)row * a.cols;
        for (uint32_t c = lane; c < a.cols; c += 64u) {
            const uint64_t f = f0 + c;
            const float p = elem<T>(a.w + (f / BS) * BB, (uint32_t)(f % BS)) * a.x[c];
            acc += p;
        }
    }
    return wave_sum(acc);
}

// Plain mat-vec for contexts in QG_PRECISION_F32 (qg_set_precision): one
// wave per row, row_dot_f32 -- each product w * x rounded to f32 and summed
// in f32, the reference's arithmetic per product (quant.rs:195-204) in a
// lane-parallel order -- from the repacked layout (RP) or the GGUF one.
template <uint32_t T, bool RP>
__global__ void __launch_bounds__(256) gemv_f32(StreamArgs a)
{
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= a.rows) return;                                   // wave-uniform
    const float v = row_dot_f32<T, RP>(a, row);
    if ((threadIdx.x & 63u) == 0u) a.y[row] = v;
}

// Per-wave flags "this wave converted a diverting segment" (set before a
// workgroup barrier, read after it) and the test of all of them.
constexpr uint32_t kMaxWaves = 16;
__device__ __forceinline__ void divert_note(uint32_t *flags, bool mine)
{
    const bool any = __builtin_amdgcn_ballot_w64(mine) != 0;
    if ((threadIdx.x & 63u) == 0u) flags[threadIdx.x >> 6] = any ? 1u : 0u;
}
// (flags: kMaxWaves words, 16-byte aligned; read at once, slots past the
// workgroup's waves ignored)
__device__ __forceinline__ bool divert_any(const uint32_t *flags)
{
    const uint32_t nw = (blockDim.x + 63u) >> 6;
    const uint4 *f4 = (const uint4 *)flags;
    uint32_t v = 0;
#pragma unroll
    for (uint32_t q = 0; q < kMaxWaves / 4u; q++) {
        const uint4 u = f4[q];
        v |= (4u * q < nw ? u.x : 0u) | (4u * q + 1u < nw ? u.y : 0u) | (4u * q + 2u < nw ? u.z : 0u) |
             (4u * q + 3u < nw ? u.w : 0u);
    }
    return v != 0u;
}

// 16 bytes of v to p as an inline-asm store (not counted by the compiler's
// wait bookkeeping, like store_y)
__device__ __forceinline__ void store16(float *p, float4 v)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v r = {v.x, v.y, v.z, v.w};
    asm volatile("global_store_dwordx4 %0, %1, off" ::"v"(p), "v"(r) : "memory");
}

// y[row] = v as an inline-asm store.  The compiler does not count it among the
// vector memory operations it waits for, so the waits it places before using
// a batch's weights stay "all but the later batches" instead of falling back
// to "everything" after a data-dependent number of stores.  Uncounted stores
// only make those waits stricter (vmcnt completes in order), never too loose.
__device__ __forceinline__ void store_y(float *p, float v)
{
    asm volatile("global_store_dword %0, %1, off" ::"v"(p), "v"(v) : "memory");
}

// ------------------------------------------------------------ timeline
//
// Only in the build with -DQG_TIMELINE (libqgemv_timeline.so, `make
// timeline`): the LDS-ring, stream and wave-private kernels take
// s_memrealtime stamps at fixed points.  A stamp goes into lane `ev` of a VGPR (a select,
// no memory operation and no register indexing), and each stamping wave
// writes its lanes once, after its last load, wait and barrier, so the
// kernel's memory traffic and waits are those of the plain build.  Per
// workgroup, 64 stamps: compute wave 0 in 0..31 and, for the ring kernel,
// the first loader wave in 32..63; the stream and wave-private kernels put
// every wave's end in 32 + w and its entry in 48 + w instead (0 = never
// stamped).  gemv_wave, wave 0: 0 entry, 1 x and rows 0..3 requested, 2 x
// landed, 3 x converted and held in registers, 4 + 2s step s landed (rows
// 4s..4s+3), 5 + 2s step s computed, 12 the workgroup barrier passed, 13 y
// written.
#ifdef QG_TIMELINE
constexpr uint32_t kTlEv = 64, kTlWG = 2048;
__device__ uint64_t qg_tl_buf[kTlWG * kTlEv];
struct Timeline {
    uint64_t v = 0;
    __device__ __forceinline__ void stamp(uint32_t ev)
    {
        const uint64_t now = __builtin_amdgcn_s_memrealtime();
        v = (threadIdx.x & 63u) == ev ? now : v;
    }
    // lanes 0..31 of this wave to stamps base .. base + 31 of this workgroup
    __device__ __forceinline__ void write(uint32_t base)
    {
        const uint32_t l = threadIdx.x & 63u;
        if (l < 32u && blockIdx.x < kTlWG) qg_tl_buf[blockIdx.x * kTlEv + base + l] = v;
    }
};
// this wave's entry and end stamps (lane 0, waves 0..15)
__device__ __forceinline__ void tl_wave_marks(uint64_t entry)
{
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0u && w < 16u && blockIdx.x < kTlWG) {
        qg_tl_buf[blockIdx.x * kTlEv + 32u + w] = __builtin_amdgcn_s_memrealtime();
        qg_tl_buf[blockIdx.x * kTlEv + 48u + w] = entry;
    }
}
#define QG_TL_DECL Timeline tl_
#define QG_TL(ev) tl_.stamp(ev)
#define QG_TL_WRITE(base) tl_.write(base)
#define QG_TL_WAVE_DECL const uint64_t tl_entry_ = __builtin_amdgcn_s_memrealtime()
#define QG_TL_WAVE_END() tl_wave_marks(tl_entry_)
#else
#define QG_TL_DECL
#define QG_TL(ev) ((void)0)
#define QG_TL_WRITE(base) ((void)0)
#define QG_TL_WAVE_DECL
#define QG_TL_WAVE_END() ((void)0)
#endif

// Workgroup barrier that waits for this wave's LDS traffic only: global loads
// issued before it stay in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Loads of batch i of team t: R row groups t + (i*R + r)*NT, every load
// unconditional (row groups past the end read the matrix's first bytes and
// are masked out later) so that all of them are in flight together.  Byte
// offsets fit in 32 bits (the planner sends larger matrices elsewhere).
// GLU (R = 1): batches alternate gate row group j and up row group j,
// j = t + (i/2)*NT.
// RP: the matrix is in the repacked layout (repack_k), read with load_rp.
template <uint32_t T, int R, bool GLU = false, bool RP = false>
__device__ __forceinline__ void issue(const StreamArgs &a, uint32_t t, uint32_t i, uint32_t it,
                                      uint32_t ib, bool active, uint32_t (&raw)[R][Item<T>::NRAW])
{
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t grp, lim;
        if constexpr (GLU) {
            lim = t + (i >> 1) * a.n_teams;
            grp = lim + (i & 1u) * a.glu_half;
        } else {
            grp = t + (i * R + r) * a.n_teams;
            lim = grp;
        }
        if constexpr (RP) {
            // whole row groups only (the repack requires them)
            const bool ok = active && lim < (GLU ? a.glu_half : a.n_groups);
            Item<T>::load_rp(a.w + (ok ? grp * a.group_bytes : 0u), it, a.ni, raw[r]);
        } else {
            const uint32_t off = grp * a.group_bytes + ib;
            const bool ok = active && lim < (GLU ? a.glu_half : a.n_groups) && off < a.nbytes;
            Item<T>::load(a.w + (ok ? off : 0u), it, raw[r]);
        }
    }
}

template <class I, class = void> struct HasRp : std::false_type {};
template <class I> struct HasRp<I, std::void_t<decltype(&I::compute_rp)>> : std::true_type {};

// per-slot sums of an item (the repacked layout's register form where it differs)
template <class I, bool RP, class XT>
__device__ __forceinline__ void item_compute(const uint32_t (&r)[I::NRAW], const XT &x, uint32_t it,
                                             float (&acc)[I::S])
{
    if constexpr (RP && HasRp<I>::value) I::compute_rp(r, x, it, acc);
    else I::compute(r, x, it, acc);
}

// This lane's x slice for its item -- the S segments the item meets, as
// fixed-point digits and records -- from the planes staged in LDS; srow[s]:
// the row (within the row group) of slot s (0 with one row per group, G1,
// where no division is needed).  Every read is unconditional, so the
// compiler issues them together and waits once: an inactive lane reads the
// slice of its clamped item (it = 0), and its callers discard what such a
// lane computes.
template <class I, bool G1>
__device__ __forceinline__ void plane_slice(const uint8_t *lds, uint32_t meta, uint32_t it, bool active,
                                            uint32_t cols, XP<I::S, I::SEG> &xs, uint32_t (&srow)[I::S])
{
    constexpr int S = I::S, SEG = I::SEG;
    (void)active;
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t e = I::seg_elem(it, s);
        srow[s] = G1 ? 0u : e / cols;
        const uint32_t c = G1 ? e : e - srow[s] * cols;
        const uint32_t gs = c / 32u, h = (c / 16u) & 1u;
        const uint8_t *sp = lds + plane_off(gs) + (SEG == 16 ? 16u * h : 0u);
#pragma unroll
        for (int p = 0; p < 3; p++)
#pragma unroll
            for (int v = 0; v < SEG / 16; v++) {
                const uint4 q = *(const uint4 *)(sp + 32 * p + 16 * v);
                xs.p[s][p][4 * v] = q.x; xs.p[s][p][4 * v + 1] = q.y;
                xs.p[s][p][4 * v + 2] = q.z; xs.p[s][p][4 * v + 3] = q.w;
            }
        const float4 m = *(const float4 *)(lds + meta + 16u * gs);
        xs.ik[s] = m.x;
        xs.sx[s] = SEG == 32 ? m.y + m.z : (h ? m.z : m.y);
        xs.sy[s] = m.w;
    }
}

// CONV: a.x is x itself (f32) and the workgroup converts it to the
// fixed-point planes while the weight loads are in flight; otherwise a.x is
// the prepared image (quant types) or x (F16/F32).  XS: 16-byte pieces of x
// each thread loads before the weights.
// ------------------------------------------------------ stream GEMV kernel
//
// Persistent form of the team kernel.  A workgroup (TPW teams) stages x once,
// holds each lane's x slice in VGPRs and then streams its teams' batches of R
// row groups with D batches of loads in flight: batch i + D is issued as soon
// as batch i has been consumed, so compute runs while the matrix streams and
// no wave ever holds more than D batches of loads (more would stall the
// issue of every load behind a full memory queue).  Before the first batch
// only D batches are issued, so x is staged early.
//
// Teams of one wave or less (TSUB > 0) reduce with DPP and write y directly.
// Teams of several waves (TSUB == 0) park each wave's per-row partial sums in
// LDS slots and add them up every `chunk` batches (two workgroup barriers per
// chunk instead of per batch).

// Input prologues (PRO):
//   kProNorm: the input is rmsnorm(a.x + a.xb) * a.nw (math.rs:237-257, with
//             the residual add of transformer.rs:31-46 folded in): every
//             workgroup loads both addends and the weights, reduces the sum of
//             squares itself and converts the normalised vector; workgroup 0
//             also stores the residual sum.
//   kProSilu: the input is silu(a.x) * a.xb, elementwise (mlp.rs:36-43 with
//             math.rs:137-146).
//   kProAttn: the input is the attention output (attention.rs:101-119)
//             merged from two position ranges: a.x and a.xb hold each
//             range's unnormalised output, a.ml its (max, sum of
//             exponentials) per head, and x = w0 a.x + w1 a.xb with
//             w_r = exp(m_r - M) / (exp(m_0 - M) l_0 + exp(m_1 - M) l_1),
//             M = max(m_0, m_1).
// GLU: y[r] = silu(gate_r . x) * (up_r . x) over the [gate; up] matrix
// (mlp.rs:31-43): one team runs row group j of gate and row group j of up in
// consecutive batches (teams of one wave or less).
//
// stream_body runs workgroup `bid` of such a launch; gemv_stream is the
// kernel of one matrix, gemv_stream_pair runs two matrices in one grid.
template <uint32_t T, int TSUB, int R, int D, bool G1, bool CONV, int XS, int LB, int D0 = D,
          int PRO = kProPlain, bool GLU = false, bool RP = false>
__device__ __forceinline__ void stream_body(const StreamArgs &a, uint32_t bid)
{
    static_assert(!GLU || (R == 1 && TSUB != 0 && D % 2 == 0), "GLU pairs need teams of a wave or less");
    constexpr bool NORM = PRO == kProNorm, TWO = PRO != kProPlain;
    using I = Item<T>;
    constexpr int S = I::S, SEG = I::SEG, NR = I::NRAW;
    constexpr int RED = G1 ? R : R * 8;
    constexpr bool CV = CONV && I::PLANES;
    extern __shared__ float4 xl4[];
    uint8_t *lds = (uint8_t *)xl4;

    const uint32_t tid = threadIdx.x;
    const uint32_t TL = TSUB ? (uint32_t)TSUB : 64u * a.wpt;
    const uint32_t lt = tid % TL, tw = tid / TL, tpw = blockDim.x / TL;
    const bool active = lt < a.ni;
    const uint32_t it = active ? lt : 0u;
    const uint32_t ib = I::item_byte(it);
    const uint32_t team = bid * tpw + tw;
    const uint32_t g = G1 ? 1u : a.g;
    QG_TL_WAVE_DECL;
    QG_TL_DECL;
    QG_TL(0);

    // 1. x loads, then (once x is in) the first D batches of weight loads.
    // x is read in pieces: 16 elements (four float4) when the workgroup
    // converts it to planes (stage_planes16), one float4 otherwise; thread
    // tid takes pieces tid, tid + blockDim, ...
    constexpr uint32_t PW = CV ? 4u : 1u;
    static_assert(XS % PW == 0, "whole pieces in registers");
    constexpr int XR = XS / (int)PW;
    const uint32_t n16 = I::PLANES && !CV ? image_bytes(true, a.cols) / 16u : a.cols / 4u;
    const uint32_t npc = n16 / PW;              // pieces (cols % 32 == 0 for the planes)
    const uint4 *src = (const uint4 *)a.x;
    const uint32_t meta = planes_bytes(a.cols);
    // The weight loads are unconditional (clamped addresses): the compiler's
    // wait counting stays exact only when no such load sits on a conditional
    // path.  The x loads are the exception: only the ceil(npc / blockDim)
    // pieces the shape needs are issued (a uniform branch; each surplus load
    // costs address-unit time, and with a 3584-wide x and three input vectors
    // most would be surplus), and the wait below, visible to the compiler as
    // a wait for every load, closes them before any weight load.
    constexpr bool ATT = PRO == kProAttn;
    static_assert(!ATT || CV, "the attention merge converts x itself");
    uint4 xv[XS];
    uint4 bvv[TWO ? XS : 1], wvv[NORM ? XS : 1];
    float4 mlv[ATT ? XR : 1];                    // kProAttn: (m0, l0, m1, l1) of the piece's head
    const uint4 *srcb = (const uint4 *)a.xb, *srcw = (const uint4 *)a.nw;
    const float2 *ml2 = (const float2 *)a.ml;
    auto ml_of = [&](uint32_t c) {               // piece c = elements 16c .. 16c + 15
        const uint32_t h = 16u * c / a.att_hd;
        const float2 r0 = ml2[h], r1 = ml2[a.att_nh + h];
        return make_float4(r0.x, r0.y, r1.x, r1.y);
    };
    const uint32_t nxs = (npc + blockDim.x - 1u) / blockDim.x;
#pragma unroll
    for (int r = 0; r < XR; r++) {
        if ((uint32_t)r < nxs) {
            const uint32_t c = tid + r * blockDim.x, cc = c < npc ? c : npc - 1u;
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) {
                xv[r * PW + i] = src[cc * PW + i];
                if constexpr (TWO) bvv[r * PW + i] = srcb[cc * PW + i];
                if constexpr (NORM) wvv[r * PW + i] = srcw[cc * PW + i];
            }
            if constexpr (ATT) mlv[r] = ml_of(cc);
        }
    }
    // x first: issued behind the weight stream of the workgroups that started
    // earlier, x reaches the late ones after most of the matrix; waiting for
    // it here (the weights then overlap the conversion) is measurably faster.
    // The RMSNorm prologue is the exception: its three input vectors take
    // long enough to arrive that issuing the first batches behind them, with
    // no wait, is faster (decode +0.9 %); the compiler's own wait before the
    // conversion then covers x alone.
    // 0x0F70 = vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9 encoding).
    if constexpr (!NORM) __builtin_amdgcn_s_waitcnt(0x0F70);
    QG_TL(1);
    uint32_t raw[D][R][NR];
#pragma unroll
    for (int d = 0; d < D0; d++) issue<T, R, GLU, RP>(a, team, d, it, ib, active, raw[d]);
    QG_TL(2);

    // 2. stage x, then this lane's slice into VGPRs
    uint4 *l4 = (uint4 *)xl4;
    // the plain mat-vec diverts its rows to row_dot_f32 when any segment of x
    // is non-finite or huge (see row_dot_f32)
    constexpr bool DIV = PRO == kProPlain && CV;
    bool xdiv = false;
    __shared__ __align__(16) uint32_t dflags[DIV ? kMaxWaves : 1];
    auto put = [&](const uint4 (&u)[PW], uint32_t c) {
        if constexpr (CV) xdiv |= stage_planes16<I::EVEN_ODD>(u, c, lds, meta);
        else l4[I::PLANES ? c : c + (c >> 4)] = u[0];
    };
    // kProNorm: 1 / rms, applied to every segment's 1/k and sums after the
    // barrier that publishes the planes (see below)
    float nscale = 1.0f;
    __shared__ float nred[NORM ? LB / 64 : 1];
    if constexpr (NORM) {
        // x = a + b.  A segment's digits do not depend on a factor common to
        // its elements (k adapts to the segment maximum), so the planes are
        // converted from (a + b) * w at once, like a plain x, and the sum of
        // squares only has to be complete when the lanes read their slices:
        // no barrier between the weight issue and the conversion.
        static_assert(CV, "the RMSNorm prologue converts x itself");
        const bool w0 = bid == 0 && a.sum_out;
        auto addv = [](uint4 p, uint4 q) {
            const float4 u = __builtin_bit_cast(float4, p), v = __builtin_bit_cast(float4, q);
            return make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
        };
        auto sq = [](float s, float4 x) {
            s += x.x * x.x; s += x.y * x.y; s += x.z * x.z; s += x.w * x.w;
            return s;
        };
        auto mulw = [](float4 x, uint4 wq) {
            const float4 w = __builtin_bit_cast(float4, wq);
            return __builtin_bit_cast(uint4, make_float4(x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w));
        };
        float ss = 0.f;
        auto piece = [&](const uint4 (&xa)[PW], const uint4 (&xb)[PW], const uint4 (&w)[PW], uint32_t c) {
            uint4 u[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) {
                const float4 x = addv(xa[i], xb[i]);
                if (w0) store16(a.sum_out + 4 * (c * PW + i), x);
                ss = sq(ss, x);
                u[i] = mulw(x, w[i]);
            }
            put(u, c);
        };
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const uint32_t c = tid + r * blockDim.x;
            if (c < npc) {
                uint4 pa[PW], pb[PW], pw[PW];
#pragma unroll
                for (uint32_t i = 0; i < PW; i++) {
                    pa[i] = xv[r * PW + i]; pb[i] = bvv[r * PW + i]; pw[i] = wvv[r * PW + i];
                }
                piece(pa, pb, pw, c);
            }
        }
        for (uint32_t c = tid + XR * blockDim.x; c < npc; c += blockDim.x) {
            uint4 pa[PW], pb[PW], pw[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) {
                pa[i] = src[c * PW + i]; pb[i] = srcb[c * PW + i]; pw[i] = srcw[c * PW + i];
            }
            piece(pa, pb, pw, c);
        }
        ss = group_sum<64>(ss);
        if ((tid & 63u) == 63u) nred[tid >> 6] = ss;
    } else if constexpr (PRO == kProSilu) {
        auto piece = [&](const uint4 (&gq)[PW], const uint4 (&uq)[PW], uint32_t c) {
            uint4 u[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) {
                const float4 gv = __builtin_bit_cast(float4, gq[i]), uv = __builtin_bit_cast(float4, uq[i]);
                u[i] = __builtin_bit_cast(uint4, make_float4(silu1(gv.x) * uv.x, silu1(gv.y) * uv.y,
                                                             silu1(gv.z) * uv.z, silu1(gv.w) * uv.w));
            }
            put(u, c);
        };
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const uint32_t c = tid + r * blockDim.x;
            if (c < npc) {
                uint4 pg[PW], pu[PW];
#pragma unroll
                for (uint32_t i = 0; i < PW; i++) { pg[i] = xv[r * PW + i]; pu[i] = bvv[r * PW + i]; }
                piece(pg, pu, c);
            }
        }
        for (uint32_t c = tid + XR * blockDim.x; c < npc; c += blockDim.x) {
            uint4 pg[PW], pu[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) { pg[i] = src[c * PW + i]; pu[i] = srcb[c * PW + i]; }
            piece(pg, pu, c);
        }
    } else if constexpr (ATT) {
        auto piece = [&](const uint4 (&p0)[PW], const uint4 (&p1)[PW], float4 mv, uint32_t c) {
            // a range without positions has m = -inf, l = 0 and weight 0;
            // range 0 always holds position 0
            const float M = fmaxf(mv.x, mv.z);
            const float e0 = expf(mv.x - M), e1 = expf(mv.z - M);
            const float inv = 1.0f / (e0 * mv.y + e1 * mv.w);
            const float w0 = e0 * inv, w1 = e1 * inv;
            uint4 u[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) {
                const float4 f0 = __builtin_bit_cast(float4, p0[i]), f1 = __builtin_bit_cast(float4, p1[i]);
                u[i] = __builtin_bit_cast(uint4, make_float4(w0 * f0.x + w1 * f1.x, w0 * f0.y + w1 * f1.y,
                                                             w0 * f0.z + w1 * f1.z, w0 * f0.w + w1 * f1.w));
            }
            put(u, c);
        };
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const uint32_t c = tid + r * blockDim.x;
            if (c < npc) {
                uint4 q0[PW], q1[PW];
#pragma unroll
                for (uint32_t i = 0; i < PW; i++) { q0[i] = xv[r * PW + i]; q1[i] = bvv[r * PW + i]; }
                piece(q0, q1, mlv[r], c);
            }
        }
        for (uint32_t c = tid + XR * blockDim.x; c < npc; c += blockDim.x) {
            uint4 q0[PW], q1[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) { q0[i] = src[c * PW + i]; q1[i] = srcb[c * PW + i]; }
            piece(q0, q1, ml_of(c), c);
        }
    } else {
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const uint32_t c = tid + r * blockDim.x;
            if (c < npc) {
                uint4 u[PW];
#pragma unroll
                for (uint32_t i = 0; i < PW; i++) u[i] = xv[r * PW + i];
                put(u, c);
            }
        }
        for (uint32_t c = tid + XR * blockDim.x; c < npc; c += blockDim.x) {
            uint4 u[PW];
#pragma unroll
            for (uint32_t i = 0; i < PW; i++) u[i] = src[c * PW + i];
            put(u, c);
        }
    }
    QG_TL(3);
    if constexpr (DIV) divert_note(dflags, xdiv);
    lds_barrier();
    QG_TL(4);
    if constexpr (NORM) {
        // all the waves' sums read at once (one LDS wait), added in wave order;
        // the slots past the last wave add 0 to a sum of squares
        const uint32_t nwv = (blockDim.x + 63u) / 64u;
        float tot = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < (uint32_t)(LB / 64); i++) {
            const float v = nred[i];
            tot += i < nwv ? v : 0.f;
        }
        const float rms = sqrtf(tot / (float)a.cols + a.eps);
        nscale = 1.0f / rms;
    }

    using XT = typename std::conditional<I::PLANES, XP<S, SEG>, XF<S, SEG>>::type;
    XT xs;
    uint32_t srow[S];
    if constexpr (I::PLANES) {
        plane_slice<I, G1>(lds, meta, it, active, a.cols, xs, srow);
        if constexpr (NORM) {
            // the digits are those of x * rms; x = (digits / k) / rms
#pragma unroll
            for (int s = 0; s < S; s++) {
                xs.ik[s] *= nscale;
                xs.sx[s] *= nscale;
            }
        }
    } else {
        // F16 / F32: x in f32, float4 i at xl4[i + i/16]
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t e = I::seg_elem(it, s);
            srow[s] = G1 ? 0u : e / a.cols;
            const uint32_t j = (G1 ? e : e - srow[s] * a.cols) / 4;
            const float4 *xp = xl4 + j + (j >> 4);
#pragma unroll
            for (int v = 0; v < SEG / 4; v++) {
                const float4 f = active ? xp[v] : make_float4(0.f, 0.f, 0.f, 0.f);
                xs.v[s * SEG + 4 * v] = f.x; xs.v[s * SEG + 4 * v + 1] = f.y;
                xs.v[s * SEG + 4 * v + 2] = f.z; xs.v[s * SEG + 4 * v + 3] = f.w;
            }
        }
    }

    QG_TL(5);
    // the rest of the ring, now that no conversion work waits behind it
#pragma unroll
    for (int d = D0; d < D; d++) issue<T, R, GLU, RP>(a, team, d, it, ib, active, raw[d]);

    // 3. stream the batches
    float *red = (float *)(lds + a.red_off);
    const uint32_t wave = tid >> 6, lane = tid & 63u;
    auto flush = [&](uint32_t i0, uint32_t nb) {
        lds_barrier();
        for (uint32_t o = lt; o < nb * RED; o += TL) {
            const uint32_t b = o / RED, k = o % RED;
            const uint32_t r = G1 ? k : k / 8, gi = G1 ? 0 : k % 8;
            const uint32_t grp = team + ((i0 + b) * R + r) * a.n_teams, row = grp * g + gi;
            float sum = 0.f;
            for (uint32_t wv = 0; wv < a.wpt; wv++)
                sum += red[((tw * a.wpt + wv) * a.chunk + b) * RED + k];
            if (gi < g && grp < a.n_groups && row < a.rows) store_y(a.y + row, sum);
        }
        lds_barrier();
    };
    float gate[G1 ? 1 : 8] = {};   // GLU: the gate dot products of the pair in progress
    auto process = [&](const uint32_t (&rw)[R][NR], uint32_t i) {
        float v[RED];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if constexpr (G1) {
                // one row per group: rows past the end are computed from the
                // clamped loads and never written; inactive lanes add zero
                float t;
                if constexpr (HasSum<I>::value) {
                    t = I::compute_sum(rw[r], xs, it);
                } else {
                    float acc[S];
                    item_compute<I, RP>(rw[r], xs, it, acc);
                    t = 0.f;
#pragma unroll
                    for (int s = 0; s < S; s++) t += acc[s];
                }
                v[r] = active ? t : 0.f;
            } else {
                uint32_t grp, lim, lim_n;
                if constexpr (GLU) {
                    lim = team + (i >> 1) * a.n_teams;
                    grp = lim + (i & 1u) * a.glu_half;
                    lim_n = a.glu_half;
                } else {
                    grp = team + (i * R + r) * a.n_teams;
                    lim = grp;
                    lim_n = a.n_groups;
                }
                const bool ok = active && lim < lim_n && grp * a.group_bytes + ib < a.nbytes;
                float acc[S];
                item_compute<I, RP>(rw[r], xs, it, acc);
#pragma unroll
                for (int gi = 0; gi < 8; gi++) {
                    float t = 0.f;
#pragma unroll
                    for (int s = 0; s < S; s++) t += srow[s] == (uint32_t)gi ? acc[s] : 0.f;
                    v[r * 8 + gi] = ok ? t : 0.f;
                }
            }
        }
        if constexpr (GLU) {
            // group j of each half: rows j*g + gi of gate, then of up
            const uint32_t j = team + (i >> 1) * a.n_teams;
#pragma unroll
            for (int gi = 0; gi < (G1 ? 1 : 8); gi++) {
                if (!G1 && (uint32_t)gi >= g) continue;
                const float sum = group_sum<TSUB>(v[gi]);
                const uint32_t row = j * g + gi;
                if ((i & 1u) == 0) gate[gi] = sum;
                else if (lt == (uint32_t)TSUB - 1u && j < a.glu_half && row < a.rows / 2u)
                    store_y(a.y + row, silu1(gate[gi]) * sum);
            }
        } else if constexpr (TSUB != 0) {
#pragma unroll
            for (int k = 0; k < RED; k++) {
                const uint32_t r = G1 ? k : k / 8, gi = G1 ? 0 : k % 8;
                if (!G1 && gi >= g) continue;
                const float sum = group_sum<TSUB>(v[k]);
                const uint32_t grp = team + (i * R + r) * a.n_teams, row = grp * g + gi;
                if (lt == (uint32_t)TSUB - 1u && grp < a.n_groups && row < a.rows) store_y(a.y + row, sum);
            }
        } else {
            const uint32_t slot = i % a.chunk;
#pragma unroll
            for (int k = 0; k < RED; k++) {
                const float sum = group_sum<64>(v[k]);
                if (lane == 63u) red[(wave * a.chunk + slot) * RED + k] = sum;
            }
            if (slot + 1 == a.chunk || i + 1 == a.per_team) flush(i - slot, slot + 1);
        }
    };
    // Whole rounds of D batches while a full round follows; then the last
    // 1..D batches, with no loads (a round's loads past per_team fetch clamped
    // addresses and are never used)
    // Wave priority alternates batch by batch between the two waves that share
    // a SIMD (waves w and w + 4), the younger one first: the older wave would
    // otherwise win every VALU arbitration and the younger one finish its last
    // batches alone, with half the SIMD's loads in flight (decode +0.5 %; the
    // older wave first, or the younger one always first, measured slower).
    uint32_t i = 0;
    for (; i + D < a.per_team; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            if (((i + d) ^ (tid >> 8)) & 1u) __builtin_amdgcn_s_setprio(1); else __builtin_amdgcn_s_setprio(0);
            process(raw[d], i + d);
            QG_TL(6u + min(i + d, 24u));
            issue<T, R, GLU, RP>(a, team, i + d + D, it, ib, active, raw[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < D; d++)
        if (i + d < a.per_team) {
            process(raw[d], i + d);
            QG_TL(6u + min(i + d, 24u));
        }
    if constexpr (DIV) {
        if (divert_any(dflags)) {
            // every row this workgroup wrote, again in f32, after its first
            // stores (this wave's: vmcnt; the others': the barrier)
            __builtin_amdgcn_s_waitcnt(0x0F70);
            lds_barrier();
            const uint32_t nq = tpw * a.per_team * (uint32_t)R * g, nwv = blockDim.x >> 6;
            for (uint32_t q = tid >> 6; q < nq; q += nwv) {
                const uint32_t gi = q % g, r = (q / g) % (uint32_t)R, bi = (q / (g * R)) % a.per_team;
                const uint32_t tq = q / (g * R * a.per_team);
                const uint32_t grp = bid * tpw + tq + (bi * R + r) * a.n_teams, row = grp * g + gi;
                if (grp < a.n_groups && row < a.rows) {
                    const float v = row_dot_f32<T, RP>(a, row);
                    if ((tid & 63u) == 0u) a.y[row] = v;
                }
            }
        }
    }
    QG_TL(31);
    if ((tid >> 6) == 0u) QG_TL_WRITE(0);
    QG_TL_WAVE_END();
}

template <uint32_t T, int TSUB, int R, int D, bool G1, bool CONV, int XS, int LB, int D0 = D,
          int PRO = kProPlain, bool GLU = false, bool RP = false>
__global__ void __launch_bounds__(LB) gemv_stream(StreamArgs a)
{
    stream_body<T, TSUB, R, D, G1, CONV, XS, LB, D0, PRO, GLU, RP>(a, blockIdx.x);
}

// Two matrices with the same input, each with its own type and plan, in one
// launch: workgroups [0, grid1) run a1 (type T1, teams of TS1 lanes), the rest
// run a2 (T2, TS2) -- for a projection whose parts have different types
// ([Q;K] Q4_K beside V Q6_K in the Q4_K_M mix), so the small part does not
// pay a launch and an x staging of its own.  RMSNorm prologue; G1A / G1B:
// one row per group in that part.
template <uint32_t T1, int TS1, bool G1A, bool RPA, uint32_t T2, int TS2, bool G1B, bool RPB, int LB>
__global__ void __launch_bounds__(LB) gemv_stream_pair(StreamArgs a1, StreamArgs a2, uint32_t grid1)
{
    if (blockIdx.x < grid1)
        stream_body<T1, TS1, 1, kDepth, G1A, true, kStage, LB, kDepth, kProNorm, false, RPA>(a1, blockIdx.x);
    else
        stream_body<T2, TS2, 1, kDepth, G1B, true, kStage, LB, kDepth, kProNorm, false, RPB>(a2, blockIdx.x - grid1);
}

// ---------------------------------------------------- LDS ring (wide rows)
//
// Plain mat-vec of a repacked matrix with one row per row group and teams of
// WPT waves (rows of 65..320 items): TPW teams of compute waves and two
// loader waves per workgroup.  The loaders copy the TPW rows of each stage --
// team t of workgroup b runs rows t G + b + i NT (G workgroups, NT teams), so
// a stage's rows are G apart and every stage of the grid lies in one band of
// NT rows (Qwen2-7B decode +0.4 % against TPW consecutive rows per workgroup)
// -- straight into an LDS ring of kRingSlots slots with global_load_lds_dwordx4, so the weight stream
// starts at kernel entry and no compute wave ever waits behind a weight load:
// the compute waves load and convert x at once, then read each item from the
// ring.  One workgroup barrier per stage publishes it; after it the loaders
// refill the slot the compute waves finished.  The first two stages go to
// slots 0 and 1 at entry; slot 2 is first written after the compute waves
// have copied their x slices, so it may overlay the x planes
// (StreamArgs::ring_slot2).  Loader l owns LINST KB of each slot (its TPW/2
// rows, each ceil(group_bytes / 16) 16-byte pieces -- the last piece reads
// into the next row group or the tail padding -- then padding): every one of
// its LINST copy instructions is issued,
// for clamped sources too, so its wait counts are exact, and what a clamped
// lane copies lands in the padding.  The same item arithmetic and reduction
// order (per-wave sums added wave 0 first) as gemv_stream, so y is
// bit-identical.
constexpr uint32_t kRingSlots = 3;

// s_waitcnt immediate for vmcnt(n), expcnt and lgkmcnt unconstrained (gfx9:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr uint32_t waitcnt_vm(uint32_t n) { return 0x0F70u | (n & 15u) | ((n >> 4) << 14); }

// 16 bytes per lane from gp into LDS at lds_base + 16 * lane (global_load_lds_dwordx4;
// lds_base is wave-uniform, an LDS byte address)
__device__ __forceinline__ void lds_dma16(const void *gp, uint32_t lds_base)
{
    __builtin_amdgcn_global_load_lds(gp, (__attribute__((address_space(3))) void *)(uintptr_t)lds_base, 16, 0, 0);
}

template <uint32_t T, int WPT, int TPW, int LINST>
__global__ void __launch_bounds__(64 * (WPT * TPW + 2)) gemv_ring(StreamArgs a)
{
    static_assert(TPW % 2 == 0 && TPW <= 4, "two loaders, one or two rows each");
    using I = Item<T>;
    constexpr int S = I::S, SEG = I::SEG, NR = I::NRAW;
    constexpr uint32_t NW = WPT * TPW, NT = 64u * NW;           // compute waves, threads
    constexpr uint32_t REGION = LINST * 1024u, SLOT = 2u * REGION;
    extern __shared__ float4 xl4[];
    uint8_t *lds = (uint8_t *)xl4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t gb = a.group_bytes, ring = a.red_off;
    auto slot_off = [&](uint32_t i) { const uint32_t k = i % kRingSlots; return k < 2u ? ring + k * SLOT : a.ring_slot2; };
    float *redf = (float *)(lds + ring + 2u * SLOT);            // 2 x NW per-wave sums
    // per-wave "x has a non-finite or huge segment" (see row_dot_f32)
    __shared__ __align__(16) uint32_t dflags[kMaxWaves];
    QG_TL_DECL;
    if (wave >= NW) {
        // loader l: the rows of teams l*TPW/2 .. (l+1)*TPW/2 - 1 of every stage
        const uint32_t l = wave - NW, np = (gb + 15u) / 16u;
        auto issue = [&](uint32_t i) {
            const uint32_t g0 = l * (TPW / 2) * gridDim.x + blockIdx.x + i * a.n_teams;
            const uint32_t dst = lds0 + slot_off(i) + l * REGION;
#pragma unroll
            for (uint32_t k = 0; k < (uint32_t)LINST; k++) {
                // 16-byte piece p of its rows: row r, piece pc; pieces past its
                // rows and rows past the matrix read clamped (valid) bytes into
                // the padding or into rows no lane stores
                const uint32_t p = k * 64u + lane;
                const uint32_t r = (TPW / 2 == 2 && p >= np) ? 1u : 0u;
                const uint32_t pc = min(p - r * np, np - 1u), grp = min(g0 + r * gridDim.x, a.n_groups - 1u);
                lds_dma16(a.w + grp * gb + pc * 16u, dst + k * 1024u);
            }
        };
        QG_TL(0);
#pragma unroll
        for (uint32_t i = 0; i < kRingSlots - 1u; i++)
            if (i < a.per_team) issue(i);
        QG_TL(1);
        divert_note(dflags, false);
        lds_barrier();                                                  // x staged
        QG_TL(2);
        for (uint32_t i = 0; i < a.per_team; i++) {
            // stage i landed: at most the next stage's copies still in flight
            if (a.per_team - 1u - i >= kRingSlots - 2u) __builtin_amdgcn_s_waitcnt(waitcnt_vm(LINST));
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            QG_TL(3u + min(i, 27u));
            lds_barrier();                                              // stage i published
            if (i + kRingSlots - 1u < a.per_team) issue(i + kRingSlots - 1u);
        }
        lds_barrier();
        QG_TL(31);
        if (wave == NW) QG_TL_WRITE(32);
        if (divert_any(dflags)) lds_barrier();                          // the compute waves' last y stores
        return;
    }
    QG_TL(0);
    const uint32_t tw = tid / (64u * WPT), lt = tid % (64u * WPT), wt = wave % WPT;
    const bool active = lt < a.ni;
    const uint32_t it = active ? lt : 0u;
    const uint32_t team = tw * gridDim.x + blockIdx.x;
    // x: 16-element pieces, converted by the compute threads
    const uint32_t npc = a.cols / 16u;
    const uint4 *src = (const uint4 *)a.x;
    const uint32_t meta = planes_bytes(a.cols);
    constexpr int XR = kStage / 4;
    uint4 xv[kStage];
    const uint32_t nxs = (npc + NT - 1u) / NT;
#pragma unroll
    for (int r = 0; r < XR; r++) {
        if ((uint32_t)r < nxs) {
            const uint32_t c = tid + r * NT, cc = c < npc ? c : npc - 1u;
#pragma unroll
            for (int i = 0; i < 4; i++) xv[4 * r + i] = src[4 * cc + i];
        }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    QG_TL(1);
    bool xdiv = false;
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const uint32_t c = tid + r * NT;
        if (c < npc) {
            uint4 u[4];
#pragma unroll
            for (int i = 0; i < 4; i++) u[i] = xv[4 * r + i];
            xdiv |= stage_planes16<I::EVEN_ODD>(u, c, lds, meta);
        }
    }
    for (uint32_t c = tid + XR * NT; c < npc; c += NT) {
        uint4 u[4];
#pragma unroll
        for (int i = 0; i < 4; i++) u[i] = src[4 * c + i];
        xdiv |= stage_planes16<I::EVEN_ODD>(u, c, lds, meta);
    }
    QG_TL(2);
    divert_note(dflags, xdiv);
    lds_barrier();
    QG_TL(3);
    XP<S, SEG> xs;
    uint32_t srow[S];
    plane_slice<I, true>(lds, meta, it, active, a.cols, xs, srow);
    auto flush = [&](uint32_t i) {                          // after a barrier: y of stage i
        if (wt == 0 && lane == 0) {
            const uint32_t grp = team + i * a.n_teams;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < WPT; w++) v += redf[(i & 1u) * NW + tw * WPT + w];
            if (grp < a.n_groups) store_y(a.y + grp, v);
        }
    };
    for (uint32_t i = 0; i < a.per_team; i++) {
        QG_TL(4u + 2u * min(i, 12u));
        lds_barrier();
        QG_TL(5u + 2u * min(i, 12u));
        if (i > 0) flush(i - 1);
        const uint8_t *row = lds + slot_off(i) + (tw / (TPW / 2)) * REGION + (tw % (TPW / 2)) * ((gb + 15u) & ~15u);
        uint32_t raw[NR];
        I::load_rp(row, it, a.ni, raw);
        float t;
        if constexpr (HasSum<I>::value) {
            t = I::compute_sum(raw, xs, it);
        } else {
            float acc[S];
            item_compute<I, true>(raw, xs, it, acc);
            t = 0.f;
#pragma unroll
            for (int s2 = 0; s2 < S; s2++) t += acc[s2];
        }
        t = active ? t : 0.f;
        t = group_sum<64>(t);
        if (lane == 63u) redf[(i & 1u) * NW + wave] = t;
    }
    QG_TL(30);
    lds_barrier();
    if (a.per_team > 0) flush(a.per_team - 1);
    if (divert_any(dflags)) {
        // the workgroup's rows again in f32, after the flushes' stores (this
        // wave's: vmcnt; the others': the barrier the loaders join too)
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        lds_barrier();
        const uint32_t nq = (uint32_t)TPW * a.per_team;
        for (uint32_t q = wave; q < nq; q += NW) {
            const uint32_t grp = (q % TPW) * gridDim.x + blockIdx.x + (q / TPW) * a.n_teams;
            if (grp < a.n_groups) {
                const float v = row_dot_f32<T, true>(a, grp);
                if (lane == 0u) a.y[grp] = v;
            }
        }
    }
    QG_TL(31);
    if (wave == 0) QG_TL_WRITE(0);
}

// ------------------------------------------- wave-private column streaming
//
// Plain mat-vec of repacked Q4_K rows of 12 or 14 items per eighth of a row
// (cols 12288 / 14336): a workgroup of eight waves owns 16 rows, b + G i for
// i = 0..15 (workgroup b of G), and wave w owns column chunk w (CJ items,
// CJ * 128 columns) of all 16.  Rows G apart rather than 16 consecutive ones:
// step s of every workgroup then falls in one band of 4G rows, so the grid
// reads one region of the matrix at a time (4096 x 14336: 8.55 -> 8.20 us,
// bit-identical; 4 consecutive rows per step at 4(b + G s) measured 8.65).
// Every wave moves its own bytes into its own LDS region with
// global_load_lds_dwordx4 and waits on its own vmcnt only -- no workgroup
// barrier until the final sum -- in steps of 4 rows.  The two waves of a SIMD
// (w and w + 4) run different schedules: the older one keeps one step in
// flight (the next step is requested the moment a step lands), the younger
// one two, and once x is converted the younger one has the higher wave
// priority.  Left to oldest-first arbitration with one step each, the younger
// waves computed behind the older ones and ended ~0.6 us after them, alone
// on their SIMDs (two steps for every wave starved them further: 9.3 us);
// this schedule measured 8.45 against 8.6-8.8 us back to back:
//   * x: the wave's 4*CJ segments of 32 elements, one 128-byte line per
//     lane, copied with a rotation (slot p of line L holds piece (p - L) mod 8)
//     so that the lane's own 8 reads of its line are free of bank conflicts;
//     lane (jj, r) = 4*jj + r converts segment r of item jj in registers
//     (stage_seg32, the same arithmetic as stage_planes16) and the four lanes
//     of a quad exchange their segments with DPP quad broadcasts, so each lane
//     holds the x slice of item jj (the 108 registers of XP<4, 32>);
//   * weights: the wave's part of a row is the item's block headers and its
//     four 16-byte pieces per item, 72 * CJ bytes gathered from the repacked
//     row by one copy instruction (lane l fetches piece l; the per-lane offset
//     within a row is computed once); row i of the workgroup lands in slot i
//     of the region (slot stride 1088 == 64 mod 256 bytes: the 16 lanes of a
//     read pass see 16 different bank groups);
//   * lane (jj, r) computes item jj of row 4s + r with Item<T_Q4_K>::compute_sum
//     (per item exactly the gemv_stream arithmetic), the 14 items of a row in
//     a wave are summed with two DPP row shifts, and after the one workgroup
//     barrier wave w adds the 32 partial sums of rows 2w and 2w + 1 with a
//     fixed DPP tree (one partial sum per lane).
// The copies are issued from inline asm: the compiler does not see them, so
// it adds no vmcnt(0) before this wave's later LDS reads (with the builtin it
// waits for every outstanding copy before each read).  The waits are exact
// immediates.  x lands in the slots of rows 8..15, which are requested only
// after the x reads (lgkmcnt(0)).
constexpr uint32_t kWaveRows = 16;          // rows per workgroup (4 steps of 4)
constexpr uint32_t kWaveSlot = 1088;        // LDS bytes per row slot
constexpr uint32_t kWaveLds = 8u * kWaveRows * kWaveSlot + kWaveRows * 32u * 4u;

// 16 bytes per lane from gp into LDS at lds_addr + 16 * lane (wave-uniform
// lds_addr), invisible to the compiler's wait bookkeeping.  lds_addr is an
// operand bound to M0 (the compiler writes M0 itself, so no reserved register
// is clobbered behind its back); the copy reads M0 one wait state after the
// write
__device__ __forceinline__ void lds_dma16_asm(const void *gp, uint32_t lds_addr)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "{m0}"(lds_addr) : "memory");
}
template <uint32_t N> __device__ __forceinline__ void wait_vm_n()
{
    static_assert(N < 64, "vmcnt holds 63");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 32-element segment converted in one lane, with the arithmetic and the
// summation trees of stage_planes16 for its two halves: P = the three digit
// planes (8 dwords each), ik = 1/k, sx = sum x, sy = sum Y.
// Unlike stage_planes16, a segment with max |x| > 2^64 also gets 1/k = NaN:
// gemv_wave tells a diverting workgroup by its NaN row sums.
__device__ __forceinline__ void stage_seg32(const float4 (&v)[8], uint32_t (&P)[3][8], float &ik, float &sx, float &sy)
{
    uint32_t mb = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) mb = max(mb, __float_as_uint(absmax4(v[i])));
    const float m = __uint_as_float(mb);
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; i++) t[i] = (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float s0 = (t[0] + t[1]) + (t[2] + t[3]), s1 = (t[4] + t[5]) + (t[6] + t[7]);
    const bool bad = !__builtin_isfinite(s0 + s1) || m > kDivertMax;
    const float k = (m > 0.f && !bad) ? fminf(kFix * __builtin_amdgcn_rcpf(m), kMaxK) : 0.f;
    ik = bad ? __builtin_nanf("") : (k > 0.f ? __builtin_amdgcn_rcpf(k) : 0.f);
    const int off = 0x8080 - kMagicBits;
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t Y0 = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].x, k, kMagic)) + off);
        const uint32_t Y1 = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].y, k, kMagic)) + off);
        const uint32_t Y2 = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].z, k, kMagic)) + off);
        const uint32_t Y3 = (uint32_t)(__float_as_int(__builtin_fmaf(v[i].w, k, kMagic)) + off);
        f[i] = (float)((int)((Y0 + Y1) + (Y2 + Y3)) - 4 * 0x8080);
        const uint32_t P01 = __builtin_amdgcn_perm(Y1, Y0, 0x05010400u);
        const uint32_t P23 = __builtin_amdgcn_perm(Y3, Y2, 0x05010400u);
        const uint32_t Q01 = __builtin_amdgcn_perm(Y1, Y0, 0x0C0C0602u);
        const uint32_t Q23 = __builtin_amdgcn_perm(Y3, Y2, 0x0C0C0602u);
        P[0][i] = __builtin_amdgcn_perm(P23, P01, 0x05040100u) ^ 0x80808080u;
        P[1][i] = __builtin_amdgcn_perm(P23, P01, 0x07060302u) ^ 0x80808080u;
        P[2][i] = __builtin_amdgcn_perm(Q23, Q01, 0x05040100u);
    }
    sx = s0 + s1;
    sy = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
}

// lane i of every quad receives lane S of its quad
template <int S> __device__ __forceinline__ uint32_t quad_bcast(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, S | (S << 2) | (S << 4) | (S << 6), 0xF, 0xF, false);
}
template <int S> __device__ __forceinline__ float quad_bcastf(float v)
{
    return __uint_as_float(quad_bcast<S>(__float_as_uint(v)));
}

template <uint32_t CJ>
__global__ void __launch_bounds__(512) gemv_wave(StreamArgs a)
{
    using I = Item<T_Q4_K>;
    constexpr uint32_t NSTEP = kWaveRows / 4u, SLOT = kWaveSlot, REG = kWaveRows * SLOT;
    constexpr uint32_t NPC = 72u * CJ / 16u;                 // 16-byte pieces of a wave's row part
    constexpr uint32_t XINST = CJ / 2u;                      // x: 4 CJ lines of 128 bytes, 8 per copy
    constexpr uint32_t XROW = kWaveRows - 8u;                // x lands in slots XROW..
    static_assert(CJ % 2 == 0 && NPC <= 64 && 4 * CJ <= 64 && XINST * 1024u <= 8u * SLOT, "shape");
    extern __shared__ float4 xl4[];
    uint8_t *lds = (uint8_t *)xl4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *reg = lds + w * REG;
    const uint32_t reg0 = lds0 + w * REG;
    float *red = (float *)(lds + 8u * REG);                  // [kWaveRows][8 waves x 4 DPP rows]
    QG_TL_WAVE_DECL;
    QG_TL_DECL;
    QG_TL(0);
    // x lines L = 8k + lane/8 (item L/4, segment L%4 of the wave's chunk)
    const float *xw = a.x + w * CJ * 128u;
#pragma unroll
    for (uint32_t k = 0; k < XINST; k++) {
        const uint32_t L = 8u * k + (lane >> 3), p = lane & 7u;
        lds_dma16_asm(xw + 32u * L + 4u * ((p - L) & 7u), reg0 + XROW * SLOT + 1024u * k);
    }
    // this lane's piece of a row part: the CJ/2 headers, then pieces k = 0..3
    // of the CJ items (repacked row: headers, then piece k of item it at
    // 16 * (ni/2) + (k * ni + it) * 16)
    uint32_t loff;
    {
        const uint32_t l = lane < NPC ? lane : NPC - 1u;
        const uint32_t m = l - CJ / 2u, k = m / CJ, t = m - k * CJ;
        loff = l < CJ / 2u ? (w * (CJ / 2u) + l) * 16u : (a.ni / 2u) * 16u + (k * a.ni + w * CJ + t) * 16u;
    }
    auto issue = [&](uint32_t i) {
        const uint32_t gr = min(blockIdx.x + i * gridDim.x, a.rows - 1u);
        lds_dma16_asm(a.w + (size_t)gr * a.group_bytes + loff, reg0 + i * SLOT);
    };
    // the younger wave of each SIMD (w >= 4) keeps two steps of rows in
    // flight, the older one one step: rows 0..7 or 0..3 now (slots 0..7;
    // x lands in slots 8..15)
    const bool two = w >= 4u;
#pragma unroll
    for (uint32_t i = 0; i < 4u; i++) issue(i);
    if (two) {
#pragma unroll
        for (uint32_t i = 4; i < 8u; i++) issue(i);
    }
    QG_TL(1);
    if (two) wait_vm_n<8u>();                                // x landed
    else wait_vm_n<4u>();
    QG_TL(2);
    const uint32_t jj = lane >> 2, r = lane & 3u;
    const bool active = jj < CJ && w * CJ + jj < a.ni;
    const uint32_t it = jj < CJ ? jj : 0u;
    XP<4, 32> xs;
    {
        float4 v[8];
        const uint8_t *xl = reg + XROW * SLOT + 128u * (lane < 4u * CJ ? lane : 0u);
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) v[k] = *(const float4 *)(xl + 16u * ((k + lane) & 7u));
        uint32_t P[3][8];
        float ik, sx, sy;
        stage_seg32(v, P, ik, sx, sy);
#pragma unroll
        for (int c = 0; c < 3; c++)
#pragma unroll
            for (int q = 0; q < 8; q++) {
                xs.p[0][c][q] = quad_bcast<0>(P[c][q]);
                xs.p[1][c][q] = quad_bcast<1>(P[c][q]);
                xs.p[2][c][q] = quad_bcast<2>(P[c][q]);
                xs.p[3][c][q] = quad_bcast<3>(P[c][q]);
            }
        xs.ik[0] = quad_bcastf<0>(ik); xs.ik[1] = quad_bcastf<1>(ik);
        xs.ik[2] = quad_bcastf<2>(ik); xs.ik[3] = quad_bcastf<3>(ik);
        xs.sx[0] = quad_bcastf<0>(sx); xs.sx[1] = quad_bcastf<1>(sx);
        xs.sx[2] = quad_bcastf<2>(sx); xs.sx[3] = quad_bcastf<3>(sx);
        xs.sy[0] = quad_bcastf<0>(sy); xs.sy[1] = quad_bcastf<1>(sy);
        xs.sy[2] = quad_bcastf<2>(sy); xs.sy[3] = quad_bcastf<3>(sy);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // x read before rows 8.. overwrite it
    }
    QG_TL(3);
    // from here on the younger wave wins VALU arbitration on its SIMD: left
    // to the default (oldest first) it computes behind the older one and
    // finishes its last steps alone
    if (two) __builtin_amdgcn_s_setprio(1);
#pragma unroll 1
    for (uint32_t s = 0; s < NSTEP; s++) {
        // step s landed (the younger wave: step s + 1 may still be in
        // flight), then the next step requested
        if (two) {
            if (s + 1u < NSTEP) wait_vm_n<4u>();
            else wait_vm_n<0u>();
            if (s + 2u < NSTEP) {
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) issue(4u * (s + 2u) + i);
            }
        } else {
            wait_vm_n<0u>();
            if (s + 1u < NSTEP) {
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) issue(4u * (s + 1u) + i);
            }
        }
        QG_TL(4u + 2u * s);
        const uint8_t *grp = reg + (4u * s + r) * SLOT;
        uint32_t raw[I::NRAW];
        {
            const uint4 h = *(const uint4 *)(grp + (it >> 1) * 16u);
            raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
            const uint8_t *q = grp + (CJ / 2u) * 16u + it * 16u;
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) {
                const uint4 v = *(const uint4 *)(q + k * CJ * 16u);
                raw[4 + 4 * k] = v.x; raw[5 + 4 * k] = v.y; raw[6 + 4 * k] = v.z; raw[7 + 4 * k] = v.w;
            }
        }
        float t = I::compute_sum(raw, xs, it);
        t = active ? t : 0.f;
        t += dpp<0x114>(t);                                  // row_shr:4
        t += dpp<0x118>(t);                                  // row_shr:8: lanes 12..15 hold rows r = 0..3
        if ((lane & 15u) >= 12u) red[(4u * s + r) * 32u + w * 4u + (lane >> 4)] = t;
        QG_TL(5u + 2u * s);
    }
    lds_barrier();
    QG_TL(12);
    // rows 2w and 2w + 1: their 32 partial sums one per lane, added by DPP.  A
    // segment of x that is non-finite or above 2^64 has 1/k = NaN, and then
    // every row sum of the workgroup is NaN: those rows are recomputed in f32
    // (row_dot_f32), as are rows made NaN by non-finite weights
    const uint32_t rr = 2u * w + (lane >> 5), row = blockIdx.x + rr * gridDim.x;
    const float v = group_sum<32>(red[rr * 32u + (lane & 31u)]);
    const bool mine = (lane & 31u) == 31u && row < a.rows;
    if (__builtin_amdgcn_ballot_w64(mine && __builtin_isnan(v)) == 0) {
        if (mine) store_y(a.y + row, v);
    } else {
        for (uint32_t i = 2u * w; i < 2u * w + 2u; i++) {
            const uint32_t r2 = blockIdx.x + i * gridDim.x;
            if (r2 < a.rows) {
                const float f = row_dot_f32<T_Q4_K, true>(a, r2);
                if (lane == 0u) a.y[r2] = f;
            }
        }
    }
    QG_TL(13);
    if (w == 0) QG_TL_WRITE(0);
    QG_TL_WAVE_END();
}

// ------------------------------------------------ no-allocation scratch
//
// The device scratch of qg_matvec_norm_glu_dev_noalloc: the normalised x and
// the [gate; up] outputs of its unfused path, kNoAllocScratchFloats floats
// per GPU for the life of the process.  Host code never passes this array's
// name to a kernel (on the host it is only a stand-in for the symbol): it
// passes the device address that scratch_address returns.
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

int scratch_address(int device, float **ptr)
{
    *ptr = nullptr;
    if (hipSetDevice(device) != hipSuccess) return -2;
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -2;
    *ptr = (float *)p;
    return 0;
}

// ------------------------------------------------------------ planning

static uint32_t gcd_u(uint64_t a, uint64_t b)
{
    while (b) { uint64_t t = a % b; a = b; b = t; }
    return (uint32_t)a;
}

template <uint32_t T, bool G1, int PRO, bool RP = false> static const void *stream_fn_g(uint32_t tsub)
{
    constexpr int R = 1, D = kDepth, LB = wg_max<T>();
    switch (tsub) {
    case 16: return (const void *)gemv_stream<T, 16, R, D, G1, true, kStage, LB, D, PRO, false, RP>;
    case 32: return (const void *)gemv_stream<T, 32, R, D, G1, true, kStage, LB, D, PRO, false, RP>;
    case 64: return (const void *)gemv_stream<T, 64, R, D, G1, true, kStage, LB, D, PRO, false, RP>;
    case 0: return (const void *)gemv_stream<T, 0, R, D, G1, true, kStage, LB, D, PRO, false, RP>;
    default: return nullptr;
    }
}

// [gate; up] kernels with the RMSNorm prologue (teams of one wave or less)
template <uint32_t T, bool G1, bool RP = false> static const void *stream_fn_glu(uint32_t tsub)
{
    constexpr int R = 1, D = kDepth, LB = wg_max<T>();
    switch (tsub) {
    case 16: return (const void *)gemv_stream<T, 16, R, D, G1, true, kStage, LB, D, kProNorm, true, RP>;
    case 32: return (const void *)gemv_stream<T, 32, R, D, G1, true, kStage, LB, D, kProNorm, true, RP>;
    case 64: return (const void *)gemv_stream<T, 64, R, D, G1, true, kStage, LB, D, kProNorm, true, RP>;
    default: return nullptr;
    }
}

// Types the upload repacks (repack_k): their items take 5 load instructions or
// more in the GGUF layout.
template <uint32_t T> constexpr bool repackable() { return T == T_Q8_0 || T == T_Q4_K || T == T_Q5_K || T == T_Q6_K; }

// Dynamic LDS a workgroup may use: the device's maximum less a reserve for
// the kernels' static arrays (per-wave flags and norm sums, < 256 bytes).
constexpr int kStaticLds = 256;
static int max_lds_bytes()
{
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 65536 - kStaticLds;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= kStaticLds)
        return 65536 - kStaticLds;
    return v - kStaticLds;
}

// Stream kernel plan (kind 1); leaves kind 0 (generic kernel) where it does
// not apply: cols % 32 != 0, row groups longer than 768 items, more than 8
// rows per group, byte offsets past 32 bits, or x larger than LDS.
template <uint32_t T> static void plan_stream(size_t rows, size_t cols, int n_cu, bool rp, Plan *p)
{
    using I = Item<T>;
    p->kind = 0;
    if (cols % 32 != 0 || rows == 0 || cols == 0) return;
    const uint64_t unit = I::UNIT;
    const uint64_t g = unit / gcd_u(cols, unit);
    const uint64_t gel = g * cols;
    const uint64_t ni = gel / I::IE;
    if (ni > (uint64_t)wg_max<T>() || g > 8) return;
    const uint64_t gbytes = gel / block_elems(T) * block_bytes(T);
    const uint64_t n_groups = (rows + g - 1) / g;
    if ((n_groups + 8) * gbytes + kTailPad >= 0xFFFFFFFFull) return;
    uint32_t tsub = 0, wpt = 1, tl;
    if (ni <= 64) { tsub = 16; while (tsub < ni) tsub <<= 1; tl = tsub; }
    else { wpt = (uint32_t)((ni + 63) / 64); tl = 64 * wpt; }
    // prologue variants for the quant types (F16/F32 x tiles leave no registers for them)
    constexpr int PN = I::PLANES ? kProNorm : kProPlain, PS = I::PLANES ? kProSilu : kProPlain;
    constexpr int PA = I::PLANES ? kProAttn : kProPlain;
    const void *fn = nullptr, *fn_norm = nullptr, *fn_silu = nullptr, *fn_norm_glu = nullptr, *fn_attn = nullptr;
    rp = rp && repackable<T>() && rows % g == 0;
    if constexpr (repackable<T>()) {
        if (rp) {
            fn = g == 1 ? stream_fn_g<T, true, kProPlain, true>(tsub) : stream_fn_g<T, false, kProPlain, true>(tsub);
            fn_norm = g == 1 ? stream_fn_g<T, true, PN, true>(tsub) : stream_fn_g<T, false, PN, true>(tsub);
            fn_silu = g == 1 ? stream_fn_g<T, true, PS, true>(tsub) : stream_fn_g<T, false, PS, true>(tsub);
            fn_norm_glu = g == 1 ? stream_fn_glu<T, true, true>(tsub) : stream_fn_glu<T, false, true>(tsub);
            // the attention merge input: one row per group only
            fn_attn = g == 1 ? stream_fn_g<T, true, PA, true>(tsub) : nullptr;
        }
    }
    if (!rp) {
        fn = g == 1 ? stream_fn_g<T, true, kProPlain>(tsub) : stream_fn_g<T, false, kProPlain>(tsub);
        // input prologues for the fixed-point types only
        if constexpr (I::PLANES) {
            fn_norm = g == 1 ? stream_fn_g<T, true, PN>(tsub) : stream_fn_g<T, false, PN>(tsub);
            fn_silu = g == 1 ? stream_fn_g<T, true, PS>(tsub) : stream_fn_g<T, false, PS>(tsub);
            fn_norm_glu = g == 1 ? stream_fn_glu<T, true>(tsub) : stream_fn_glu<T, false>(tsub);
            fn_attn = g == 1 ? stream_fn_g<T, true, PA>(tsub) : nullptr;
        }
    }
    if (!fn) return;
    const uint64_t ncu = n_cu > 0 ? (uint64_t)n_cu : 256;
    const uint32_t img = (image_bytes(I::PLANES, (uint32_t)cols) + 15u) & ~15u;
    const uint32_t red = g == 1 ? 1u : 8u;                 // partial sums per batch per wave
    const uint64_t nbat = n_groups;                        // R = 1 row group per batch
    // Full workgroups (768 threads) on every CU when there is enough work;
    // otherwise smaller workgroups, one team batch each, spread over the CUs.
    const uint32_t tpw_max = tl >= (uint32_t)wg_max<T>() ? 1u : (uint32_t)wg_max<T>() / tl;
    const uint32_t tpw_min = tl >= 64u ? 1u : 64u / tl;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, (int)(tpw_max * tl), img + 4096) != hipSuccess)
        occ = 0;
    if (occ <= 0) return;
    uint32_t tpw, per;
    if (nbat > ncu * (uint64_t)occ * tpw_max) {
        tpw = tpw_max;
        per = (uint32_t)((nbat + ncu * occ * tpw - 1) / (ncu * occ * tpw));
    } else {
        const uint64_t t = (nbat + ncu - 1) / ncu;         // teams per CU
        tpw = (uint32_t)(t < tpw_min ? tpw_min : t > tpw_max ? tpw_max : t);
        // whole waves only: the workgroup reductions count blockDim / 64 waves
        tpw = (tpw + tpw_min - 1) / tpw_min * tpw_min;
        per = 1;
    }
    const uint32_t grid = (uint32_t)((nbat + (uint64_t)tpw * per - 1) / ((uint64_t)tpw * per));
    if ((tpw * tl) % 64u != 0) return;
    // partial-sum slots for a chunk of batches (several-wave teams)
    const uint32_t nw = tpw * tl / 64u;
    const uint32_t room = (uint32_t)max_lds_bytes() > img ? (uint32_t)max_lds_bytes() - img : 0u;
    uint32_t chunk = per < 64u ? per : 64u;
    while (chunk > 1 && nw * chunk * red * 4u > room) chunk >>= 1;
    const uint32_t lds = img + (tsub == 0 ? nw * chunk * red * 4u : 0u);
    if (lds > (uint32_t)max_lds_bytes()) return;
    p->fn = fn;
    p->fn_norm = fn_norm;
    p->fn_silu = fn_silu;
    p->fn_norm_glu = fn_norm_glu;
    p->fn_attn = fn_attn;
    p->rp = rp;
    p->g = (uint32_t)g;
    p->ni = (uint32_t)ni;
    p->ts = tl;
    p->tsub = tsub;
    p->wpt = wpt;
    p->n_groups = (uint32_t)n_groups;
    p->group_bytes = gbytes;
    p->R = 1;
    p->n_batches = (uint32_t)nbat;
    p->per_team = per;
    p->block = tpw * tl;
    p->grid = grid;
    p->n_teams = grid * tpw;
    p->chunk = chunk;
    p->red_off = img;
    p->lds = lds;
    p->kind = 1;
    // the LDS ring kernel for the plain mat-vec of repacked rows with
    // several-wave teams, where a loader's rows fit its region and the LDS
    // holds the x planes, two slots (the third overlays the x planes when they
    // are large enough) and the per-wave sums
    p->fn_ring = nullptr;
    if constexpr (repackable<T>()) {
        const uint32_t rsz = (uint32_t)((gbytes + 15u) & ~15ull);     // a row in whole 16-byte pieces
        const void *rf = nullptr;
        uint32_t rt = 0, linst = 0;
        // (waves per team, teams per workgroup, KB per loader): two rows per
        // loader for two-wave teams, one row otherwise
        auto pick = [&](const void *f, uint32_t teams, uint32_t kb) {
            if (!rf && (teams / 2u) * rsz <= kb * 1024u) { rf = f; rt = teams; linst = kb; }
        };
        // (Q4_K: none -- its rows of two- and three-wave teams measured 2-13 %
        // faster on the stream kernel, e.g. 9.55 against 9.80 us at 4000 x
        // 14336, 12.6 against 13.1 us at 3584 x 18944)
        if constexpr (T == T_Q5_K || T == T_Q6_K) {
            if (wpt == 5) pick((const void *)gemv_ring<T, 5, 2, 16>, 2, 16);
            if (wpt == 4) pick((const void *)gemv_ring<T, 4, 2, 12>, 2, 12);
        } else if constexpr (T == T_Q8_0) {
            if (wpt == 5) pick((const void *)gemv_ring<T, 5, 2, 20>, 2, 20);
            if (wpt == 4) pick((const void *)gemv_ring<T, 4, 2, 16>, 2, 16);
        }
        if (rf && rp && g == 1 && tsub == 0) {
            const uint32_t slot = 2u * linst * 1024u, red_bytes = 128u;
            const bool xs = slot <= img;
            const uint32_t ring_lds = img + 2u * slot + red_bytes + (xs ? 0u : slot);
            if (ring_lds <= (uint32_t)max_lds_bytes()) {
                const uint64_t wgs = (n_groups + rt - 1) / rt;
                const uint32_t rg = (uint32_t)(wgs < ncu ? wgs : ncu);
                p->fn_ring = rf;
                p->ring_grid = rg;
                p->ring_block = 64u * (wpt * rt + 2u);
                p->ring_per = (uint32_t)((n_groups + (uint64_t)rt * rg - 1) / ((uint64_t)rt * rg));
                p->ring_lds = ring_lds;
                p->ring_slot2 = xs ? 0u : img + 2u * slot + red_bytes;
            }
        }
    }
    // the wave-private column kernel for repacked Q4_K rows of 8 * CJ items,
    // CJ = 12 or 14, when its 16-row workgroups cover every CU at least once
    p->fn_wave = nullptr;
    if constexpr (T == T_Q4_K) {
        const uint64_t wg = (rows + kWaveRows - 1) / kWaveRows;
        if (rp && g == 1 && wg >= ncu && kWaveLds <= (uint32_t)max_lds_bytes() && wg <= 0x7FFFFFFFull) {
            if (ni == 8u * 14u) p->fn_wave = (const void *)gemv_wave<14>;
            if (ni == 8u * 12u) p->fn_wave = (const void *)gemv_wave<12>;
            p->wave_grid = (uint32_t)wg;
        }
    }
}

int make_plan(uint32_t type, size_t rows, size_t cols, int n_cu, Plan *p, bool rp)
{
    *p = Plan{};
    if (rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull) return 0;
    switch (type) {
    case T_F32: plan_stream<T_F32>(rows, cols, n_cu, false, p); break;
    case T_F16: plan_stream<T_F16>(rows, cols, n_cu, false, p); break;
    case T_Q4_0: plan_stream<T_Q4_0>(rows, cols, n_cu, false, p); break;
    case T_Q5_0: plan_stream<T_Q5_0>(rows, cols, n_cu, false, p); break;
    case T_Q8_0: plan_stream<T_Q8_0>(rows, cols, n_cu, rp, p); break;
    case T_Q4_K: plan_stream<T_Q4_K>(rows, cols, n_cu, rp, p); break;
    case T_Q5_K: plan_stream<T_Q5_K>(rows, cols, n_cu, rp, p); break;
    case T_Q6_K: plan_stream<T_Q6_K>(rows, cols, n_cu, rp, p); break;
    default: return -1;
    }
    return 0;
}

bool repack_eligible(uint32_t type, const Plan &p, size_t rows)
{
    return (type == T_Q8_0 || type == T_Q4_K || type == T_Q5_K || type == T_Q6_K) && p.kind == 1 && p.g > 0 &&
           rows % p.g == 0;
}

// The repacked layout of a whole number of row groups, group by group (the
// same bytes -- for Q5_K the same bits -- rearranged so that a wave's loads
// of one piece are contiguous):
//   Q4_K (ni = 2 nb items of 128 weights): the nb 16-byte block headers, then
//        piece k (bytes 16k..16k+15 of the item's 64 quant bytes) of item it
//        at nb*16 + (k*ni + it)*16;
//   Q8_0 (item = 2 blocks, 64 codes): piece k (codes 16k..16k+15) of item it
//        at (k*ni + it)*16, then the two d halves of every item at 64ni + 4it;
//   Q5_K (ni = 4 nb items of 64 weights, j = 2 (it & 3)): the nb block
//        headers, piece k of the item's 32 quant bytes at nb*16 + (k*ni + it)*16,
//        then 8 bytes per item at nb*16 + 32ni + 8it: bits 8b + 2t' and
//        8b + 2t' + 1 of word w are bits j and j + 1 of qh[16w + 4t' + b];
//   Q6_K (ni = 4 nb items of 64 weights; item it = block it/4, half
//        n = (it/2)&1, i = it&1): ql[64n+16i..+16] at it*16,
//        ql[64n+32+16i..+16] at (ni+it)*16, qh[32n+16i..+16] at (2ni+it)*16,
//        the scales sc[8n+i+2k], k = 0..3, at 48ni + 4it + k, d at 52ni + 2b.
// One thread per item.
template <uint32_t T>
__global__ void __launch_bounds__(256) repack_k(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                uint64_t n_items, uint32_t ni, uint32_t group_bytes)
{
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_items) return;
    const uint64_t gidx = idx / ni;
    const uint32_t it = (uint32_t)(idx - gidx * ni);
    const uint8_t *sg = src + gidx * group_bytes;
    uint8_t *dg = dst + gidx * group_bytes;
    if constexpr (T == T_Q8_0) {
        const uint8_t *b = sg + it * 68u;          // blocks 2it, 2it + 1: d, then 32 codes each
        for (uint32_t k = 0; k < 64; k++) dg[((k >> 4) * ni + it) * 16u + (k & 15u)] = b[k < 32 ? 2u + k : 4u + k];
        dg[64u * ni + 4u * it] = b[0];
        dg[64u * ni + 4u * it + 1u] = b[1];
        dg[64u * ni + 4u * it + 2u] = b[34];
        dg[64u * ni + 4u * it + 3u] = b[35];
    } else if constexpr (T == T_Q4_K) {
        const uint8_t *b = sg + (it >> 1) * 144u;
        if ((it & 1u) == 0)
            for (int j = 0; j < 16; j++) dg[(it >> 1) * 16u + j] = b[j];
        for (uint32_t k = 0; k < 4; k++)
            for (int j = 0; j < 16; j++) dg[(ni >> 1) * 16u + (k * ni + it) * 16u + j] = b[16u + (it & 1u) * 64u + 16u * k + j];
    } else if constexpr (T == T_Q5_K) {
        const uint8_t *b = sg + (it >> 2) * 176u;
        const uint32_t H = (ni >> 2) * 16u, j = (it & 3u) * 2u;
        if ((it & 3u) == 0)
            for (int k = 0; k < 16; k++) dg[(it >> 2) * 16u + k] = b[k];
        for (uint32_t k = 0; k < 32; k++) dg[H + ((k >> 4) * ni + it) * 16u + (k & 15u)] = b[48u + (it & 3u) * 32u + k];
        uint32_t W[2] = {0u, 0u};
        for (uint32_t m = 0; m < 32; m++) {       // qh byte m = 16w + 4t' + b
            const uint32_t w = m >> 4, tp = (m >> 2) & 3u, bb = m & 3u, v = b[16u + m];
            W[w] |= ((v >> j) & 1u) << (8u * bb + 2u * tp);
            W[w] |= ((v >> (j + 1u)) & 1u) << (8u * bb + 2u * tp + 1u);
        }
        for (uint32_t k = 0; k < 8; k++) dg[H + 32u * ni + 8u * it + k] = (uint8_t)(W[k >> 2] >> (8u * (k & 3u)));
    } else {
        const uint8_t *b = sg + (it >> 2) * 210u;
        const uint32_t n = (it >> 1) & 1u, i = it & 1u;
        for (int j = 0; j < 16; j++) {
            dg[it * 16u + j] = b[64u * n + 16u * i + j];
            dg[(ni + it) * 16u + j] = b[64u * n + 32u + 16u * i + j];
            dg[(2u * ni + it) * 16u + j] = b[128u + 32u * n + 16u * i + j];
        }
        for (uint32_t k = 0; k < 4; k++) dg[48u * ni + 4u * it + k] = b[192u + 8u * n + i + 2u * k];
        if ((it & 3u) == 0) {
            dg[52u * ni + (it >> 2) * 2u] = b[208];
            dg[52u * ni + (it >> 2) * 2u + 1u] = b[209];
        }
    }
}

int launch_repack(uint32_t type, const Plan &p, const uint8_t *src, uint8_t *dst, ihipStream_t *stream)
{
    if (p.kind != 1 || p.ni == 0) return -1;
    const uint64_t n_items = (uint64_t)p.n_groups * p.ni;
    if (n_items == 0) return 0;
    const uint64_t blocks = (n_items + 255) / 256;
    if (blocks > 0x7FFFFFFFull) return -1;
    if (type == T_Q8_0)
        hipLaunchKernelGGL(repack_k<T_Q8_0>, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, src, dst,
                           n_items, p.ni, (uint32_t)p.group_bytes);
    else if (type == T_Q4_K)
        hipLaunchKernelGGL(repack_k<T_Q4_K>, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, src, dst,
                           n_items, p.ni, (uint32_t)p.group_bytes);
    else if (type == T_Q5_K)
        hipLaunchKernelGGL(repack_k<T_Q5_K>, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, src, dst,
                           n_items, p.ni, (uint32_t)p.group_bytes);
    else if (type == T_Q6_K)
        hipLaunchKernelGGL(repack_k<T_Q6_K>, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, src, dst,
                           n_items, p.ni, (uint32_t)p.group_bytes);
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// The GGUF layout of repacked row groups (the inverse of repack_k, one thread
// per item; for Q5_K the block's first item also rebuilds the 32 qh bytes
// from the four items' bit words).
template <uint32_t T>
__global__ void __launch_bounds__(256) unrepack_k(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                  uint64_t n_items, uint32_t ni, uint32_t group_bytes)
{
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_items) return;
    const uint64_t gidx = idx / ni;
    const uint32_t it = (uint32_t)(idx - gidx * ni);
    const uint8_t *sg = src + gidx * group_bytes;          // repacked group
    uint8_t *dg = dst + gidx * group_bytes;                // GGUF-layout group
    if constexpr (T == T_Q8_0) {
        uint8_t *b = dg + it * 68u;
        for (uint32_t k = 0; k < 64; k++) b[k < 32 ? 2u + k : 4u + k] = sg[((k >> 4) * ni + it) * 16u + (k & 15u)];
        b[0] = sg[64u * ni + 4u * it];
        b[1] = sg[64u * ni + 4u * it + 1u];
        b[34] = sg[64u * ni + 4u * it + 2u];
        b[35] = sg[64u * ni + 4u * it + 3u];
    } else if constexpr (T == T_Q4_K) {
        uint8_t *b = dg + (it >> 1) * 144u;
        if ((it & 1u) == 0)
            for (int j = 0; j < 16; j++) b[j] = sg[(it >> 1) * 16u + j];
        for (uint32_t k = 0; k < 4; k++)
            for (int j = 0; j < 16; j++) b[16u + (it & 1u) * 64u + 16u * k + j] = sg[(ni >> 1) * 16u + (k * ni + it) * 16u + j];
    } else if constexpr (T == T_Q5_K) {
        uint8_t *b = dg + (it >> 2) * 176u;
        const uint32_t H = (ni >> 2) * 16u;
        for (uint32_t k = 0; k < 32; k++) b[48u + (it & 3u) * 32u + k] = sg[H + ((k >> 4) * ni + it) * 16u + (k & 15u)];
        if ((it & 3u) == 0) {
            for (int k = 0; k < 16; k++) b[k] = sg[(it >> 2) * 16u + k];
            uint32_t W[4][2];
            for (uint32_t q = 0; q < 4; q++)
                for (uint32_t w = 0; w < 2; w++) {
                    const uint8_t *pw = sg + H + 32u * ni + 8u * (it + q) + 4u * w;
                    W[q][w] = (uint32_t)pw[0] | ((uint32_t)pw[1] << 8) | ((uint32_t)pw[2] << 16) | ((uint32_t)pw[3] << 24);
                }
            for (uint32_t m = 0; m < 32; m++) {          // qh byte m = 16w + 4t' + bb
                const uint32_t w = m >> 4, tp = (m >> 2) & 3u, bb = m & 3u;
                uint32_t v = 0;
                for (uint32_t q = 0; q < 4; q++)        // item q of the block holds bits 2q, 2q + 1
                    for (uint32_t h = 0; h < 2; h++) v |= ((W[q][w] >> (8u * bb + 2u * tp + h)) & 1u) << (2u * q + h);
                b[16u + m] = (uint8_t)v;
            }
        }
    } else {
        uint8_t *b = dg + (it >> 2) * 210u;
        const uint32_t n = (it >> 1) & 1u, i = it & 1u;
        for (int j = 0; j < 16; j++) {
            b[64u * n + 16u * i + j] = sg[it * 16u + j];
            b[64u * n + 32u + 16u * i + j] = sg[(ni + it) * 16u + j];
            b[128u + 32u * n + 16u * i + j] = sg[(2u * ni + it) * 16u + j];
        }
        for (uint32_t k = 0; k < 4; k++) b[192u + 8u * n + i + 2u * k] = sg[48u * ni + 4u * it + k];
        if ((it & 3u) == 0) {
            b[208] = sg[52u * ni + (it >> 2) * 2u];
            b[209] = sg[52u * ni + (it >> 2) * 2u + 1u];
        }
    }
}

int launch_unrepack(uint32_t type, const Plan &p, const uint8_t *src, uint8_t *dst, ihipStream_t *stream)
{
    if (p.kind != 1 || p.ni == 0 || !p.rp) return -1;
    const uint64_t n_items = (uint64_t)p.n_groups * p.ni;
    if (n_items == 0) return 0;
    const uint64_t blocks = (n_items + 255) / 256;
    if (blocks > 0x7FFFFFFFull) return -1;
    const dim3 grid((uint32_t)blocks), block(256);
    hipStream_t st = (hipStream_t)stream;
    const uint32_t gb = (uint32_t)p.group_bytes;
    switch (type) {
    case T_Q8_0: hipLaunchKernelGGL(unrepack_k<T_Q8_0>, grid, block, 0, st, src, dst, n_items, p.ni, gb); break;
    case T_Q4_K: hipLaunchKernelGGL(unrepack_k<T_Q4_K>, grid, block, 0, st, src, dst, n_items, p.ni, gb); break;
    case T_Q5_K: hipLaunchKernelGGL(unrepack_k<T_Q5_K>, grid, block, 0, st, src, dst, n_items, p.ni, gb); break;
    case T_Q6_K: hipLaunchKernelGGL(unrepack_k<T_Q6_K>, grid, block, 0, st, src, dst, n_items, p.ni, gb); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// ------------------------------------------------------------ launchers

static StreamArgs stream_args(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                               const float *x, float *y)
{
    StreamArgs a{};
    a.w = w; a.x = x; a.y = y; a.nbytes = (uint32_t)nbytes; a.group_bytes = (uint32_t)p.group_bytes;
    a.rows = (uint32_t)rows; a.cols = (uint32_t)cols; a.g = p.g; a.n_groups = p.n_groups;
    a.ni = p.ni; a.n_teams = p.n_teams; a.per_team = p.per_team; a.wpt = p.wpt;
    a.chunk = p.chunk; a.red_off = p.red_off;
    return a;
}

int launch_gemv(uint32_t type, const Plan &p, const uint8_t *w, size_t nbytes, size_t rows,
                size_t cols, const float *x, float *y, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (p.kind != 1 || !p.fn) return launch_gemv_generic(type, w, rows, cols, x, y, stream);
    StreamArgs a = stream_args(p, w, nbytes, rows, cols, x, y);
    void *args[] = {&a};
    if (p.fn_wave)
        return hipLaunchKernel(p.fn_wave, dim3(p.wave_grid), dim3(512), args, kWaveLds, st) == hipSuccess ? 0 : -2;
    if (p.fn_ring) {
        a.n_teams = (p.ring_block / 64u - 2u) / p.wpt * p.ring_grid;
        a.per_team = p.ring_per;
        a.ring_slot2 = p.ring_slot2;
        return hipLaunchKernel(p.fn_ring, dim3(p.ring_grid), dim3(p.ring_block), args, p.ring_lds, st) == hipSuccess
                   ? 0 : -2;
    }
    return hipLaunchKernel(p.fn, dim3(p.grid), dim3(p.block), args, p.lds, st) == hipSuccess ? 0 : -2;
}

int launch_gemv_silu(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *g, const float *u, float *y, ihipStream_t *stream)
{
    if (p.kind != 1 || !p.fn_silu || cols % 4 != 0) return -1;
    StreamArgs a = stream_args(p, w, nbytes, rows, cols, g, y);
    a.xb = u;
    void *args[] = {&a};
    return hipLaunchKernel(p.fn_silu, dim3(p.grid), dim3(p.block), args, p.lds, (hipStream_t)stream) ==
                   hipSuccess ? 0 : -2;
}

int launch_gemv_attn(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *part, const float *ml, uint32_t n_heads, uint32_t hd, float *y,
                     ihipStream_t *stream)
{
    if (p.kind != 1 || !p.fn_attn || hd == 0 || hd % 16 != 0 || (size_t)n_heads * hd != cols ||
        ((uintptr_t)part & 15u) != 0)
        return -1;
    StreamArgs a = stream_args(p, w, nbytes, rows, cols, part, y);
    a.xb = part + cols;
    a.ml = ml;
    a.att_nh = n_heads;
    a.att_hd = hd;
    void *args[] = {&a};
    return hipLaunchKernel(p.fn_attn, dim3(p.grid), dim3(p.block), args, p.lds, (hipStream_t)stream) ==
                   hipSuccess ? 0 : -2;
}

int launch_gemv_norm(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                     const float *xa, const float *xb, const float *nw, float eps, float *sum_out,
                     float *y, ihipStream_t *stream)
{
    if (p.kind != 1 || !p.fn_norm || cols % 4 != 0) return -1;
    StreamArgs a = stream_args(p, w, nbytes, rows, cols, xa, y);
    a.xb = xb; a.nw = nw; a.sum_out = sum_out; a.eps = eps;
    void *args[] = {&a};
    return hipLaunchKernel(p.fn_norm, dim3(p.grid), dim3(p.block), args, p.lds, (hipStream_t)stream) ==
                   hipSuccess ? 0 : -2;
}

// Teams keep the plan's batches per team, rounded up to whole (gate, up)
// pairs; the grid covers the glu_half pairs.
int launch_gemv_norm_glu(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                         const float *xa, const float *xb, const float *nw, float eps, float *sum_out,
                         float *y, ihipStream_t *stream)
{
    // each half a whole number of row groups
    if (p.kind != 1 || !p.fn_norm_glu || p.tsub == 0 || rows % (2u * p.g) != 0 || cols % 4 != 0) return -1;
    const uint32_t half = (uint32_t)(rows / 2 / p.g), tpw = p.block / p.ts;
    const uint32_t pairs = (p.per_team + 1) / 2;
    const uint32_t grid = (half + tpw * pairs - 1) / (tpw * pairs);
    StreamArgs a = stream_args(p, w, nbytes, rows, cols, xa, y);
    a.n_teams = grid * tpw;
    a.per_team = 2 * pairs;
    a.glu_half = half;
    a.xb = xb; a.nw = nw; a.sum_out = sum_out; a.eps = eps;
    void *args[] = {&a};
    return hipLaunchKernel(p.fn_norm_glu, dim3(grid), dim3(p.block), args, p.lds, (hipStream_t)stream) ==
                   hipSuccess ? 0 : -2;
}

// ------------------------------------------------------ pairs of matrices

constexpr int kPairBlock = 512;

template <uint32_t T1, uint32_t T2, bool G1> static const void *pair_fn_g(uint32_t ts1, uint32_t ts2)
{
    constexpr int LB = kPairBlock;
    constexpr bool R1 = repackable<T1>(), R2 = repackable<T2>();
    if (ts1 == 16 && ts2 == 16) return (const void *)gemv_stream_pair<T1, 16, G1, R1, T2, 16, G1, R2, LB>;
    if (ts1 == 16 && ts2 == 32) return (const void *)gemv_stream_pair<T1, 16, G1, R1, T2, 32, G1, R2, LB>;
    if (ts1 == 32 && ts2 == 32) return (const void *)gemv_stream_pair<T1, 32, G1, R1, T2, 32, G1, R2, LB>;
    if (ts1 == 32 && ts2 == 64) return (const void *)gemv_stream_pair<T1, 32, G1, R1, T2, 64, G1, R2, LB>;
    if (ts1 == 64 && ts2 == 64) return (const void *)gemv_stream_pair<T1, 64, G1, R1, T2, 64, G1, R2, LB>;
    return nullptr;
}

// Both parts one-row groups, or both multi-row groups (the 896-column rows of
// Qwen2-0.5B: two rows per group for the K-quants); the repackable types in
// their repacked layout (matrices wrapped from caller memory are not, and
// take two launches).
template <uint32_t T1, uint32_t T2> static const void *pair_fn(const Plan &p1, const Plan &p2)
{
    if (p1.rp != repackable<T1>() || p2.rp != repackable<T2>()) return nullptr;
    if (p1.g == 1 && p2.g == 1) return pair_fn_g<T1, T2, true>(p1.tsub, p2.tsub);
    if (p1.g > 1 && p2.g > 1) return pair_fn_g<T1, T2, false>(p1.tsub, p2.tsub);
    return nullptr;
}

static bool pair_part_ok(const Plan &p)
{
    return p.kind == 1 && p.tsub != 0 && kPairBlock % p.ts == 0;
}

// Workgroups of kPairBlock threads for a part of n_batches batches, per
// batches per team.
static uint32_t pair_grid(const Plan &p, uint32_t per)
{
    const uint32_t tpw = kPairBlock / p.ts;
    return (p.n_batches + tpw * per - 1) / (tpw * per);
}

// Resident workgroups of a pair kernel per CU (queried once per kernel).
static int pair_occupancy(const void *fn, uint32_t lds)
{
    static std::mutex mu;
    static std::map<std::pair<const void *, uint32_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({fn, lds});
    if (it != cache.end()) return it->second;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kPairBlock, lds) != hipSuccess || occ < 1) occ = 1;
    cache[{fn, lds}] = occ;
    return occ;
}

int launch_gemv_norm_pair(uint32_t t1, const Plan &p1, const uint8_t *w1, size_t nbytes1, size_t rows1, float *y1,
                          uint32_t t2, const Plan &p2, const uint8_t *w2, size_t nbytes2, size_t rows2, float *y2,
                          size_t cols, const float *xa, const float *xb, const float *nw, float eps,
                          float *sum_out, int n_cu, ihipStream_t *stream)
{
    const void *fn = nullptr;
    if (t1 == T_Q4_K && t2 == T_Q6_K) fn = pair_fn<T_Q4_K, T_Q6_K>(p1, p2);
    else if (t1 == T_Q5_K && t2 == T_Q6_K) fn = pair_fn<T_Q5_K, T_Q6_K>(p1, p2);
    if (!fn || cols % 4 != 0 || !pair_part_ok(p1) || !pair_part_ok(p2)) return -1;
    const uint32_t lds = p1.lds > p2.lds ? p1.lds : p2.lds;
    // both parts resident at once (a part that waits for the other's
    // workgroups to finish costs as much as a second launch): more batches
    // per team for the part with more workgroups until they fit
    const uint64_t slots = (uint64_t)(n_cu > 0 ? n_cu : 256) * (uint64_t)pair_occupancy(fn, lds);
    uint32_t per1 = p1.per_team ? p1.per_team : 1u, per2 = p2.per_team ? p2.per_team : 1u;
    uint32_t g1 = pair_grid(p1, per1), g2 = pair_grid(p2, per2);
    while ((uint64_t)g1 + g2 > slots && (g1 > 1 || g2 > 1)) {
        if (g1 >= g2) g1 = pair_grid(p1, ++per1);
        else g2 = pair_grid(p2, ++per2);
    }
    StreamArgs a1 = stream_args(p1, w1, nbytes1, rows1, cols, xa, y1);
    StreamArgs a2 = stream_args(p2, w2, nbytes2, rows2, cols, xa, y2);
    a1.n_teams = g1 * (kPairBlock / p1.ts);
    a2.n_teams = g2 * (kPairBlock / p2.ts);
    a1.per_team = per1;
    a2.per_team = per2;
    a1.xb = a2.xb = xb;
    a1.nw = a2.nw = nw;
    a1.eps = a2.eps = eps;
    a1.sum_out = sum_out;
    void *args[] = {&a1, &a2, &g1};
    return hipLaunchKernel(fn, dim3(g1 + g2), dim3(kPairBlock), args, lds, (hipStream_t)stream) == hipSuccess ? 0
                                                                                                             : -2;
}

template <uint32_t T>
static int launch_generic_t(const uint8_t *w, size_t rows, size_t cols, const float *x, float *y,
                            hipStream_t st)
{
    dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    hipLaunchKernelGGL((gemv_generic<T>), grid, block, 0, st, w, x, y, (uint32_t)rows,
                       (uint32_t)cols);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <uint32_t T, bool RP> static int launch_f32_t(const StreamArgs &a, hipStream_t st)
{
    hipLaunchKernelGGL((gemv_f32<T, RP>), dim3((a.rows + 3u) / 4u), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_gemv_f32(uint32_t type, const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                    const float *x, float *y, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (rows == 0) return 0;
    if (rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull || nbytes > 0xFFFFFFFFull) return -1;
    const StreamArgs a = stream_args(p, w, nbytes, rows, cols, x, y);
    if (p.rp) {
        switch (type) {
        case T_Q8_0: return launch_f32_t<T_Q8_0, true>(a, st);
        case T_Q4_K: return launch_f32_t<T_Q4_K, true>(a, st);
        case T_Q5_K: return launch_f32_t<T_Q5_K, true>(a, st);
        case T_Q6_K: return launch_f32_t<T_Q6_K, true>(a, st);
        default: return -1;
        }
    }
    switch (type) {
    case T_F32: return launch_f32_t<T_F32, false>(a, st);
    case T_F16: return launch_f32_t<T_F16, false>(a, st);
    case T_Q4_0: return launch_f32_t<T_Q4_0, false>(a, st);
    case T_Q5_0: return launch_f32_t<T_Q5_0, false>(a, st);
    case T_Q8_0: return launch_f32_t<T_Q8_0, false>(a, st);
    case T_Q4_K: return launch_f32_t<T_Q4_K, false>(a, st);
    case T_Q5_K: return launch_f32_t<T_Q5_K, false>(a, st);
    case T_Q6_K: return launch_f32_t<T_Q6_K, false>(a, st);
    default: return -1;
    }
}

int launch_gemv_generic(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const float *x,
                        float *y, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (rows == 0) return 0;
    if (rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull) return -1;
    switch (type) {
    case T_F32: return launch_generic_t<T_F32>(w, rows, cols, x, y, st);
    case T_F16: return launch_generic_t<T_F16>(w, rows, cols, x, y, st);
    case T_Q4_0: return launch_generic_t<T_Q4_0>(w, rows, cols, x, y, st);
    case T_Q5_0: return launch_generic_t<T_Q5_0>(w, rows, cols, x, y, st);
    case T_Q8_0: return launch_generic_t<T_Q8_0>(w, rows, cols, x, y, st);
    case T_Q4_K: return launch_generic_t<T_Q4_K>(w, rows, cols, x, y, st);
    case T_Q5_K: return launch_generic_t<T_Q5_K>(w, rows, cols, x, y, st);
    case T_Q6_K: return launch_generic_t<T_Q6_K>(w, rows, cols, x, y, st);
    default: return -1;
    }
}

static unsigned grid_for(uint64_t n)
{
    uint64_t g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : g > 65536 ? 65536 : g);
}

template <uint32_t T>
static int launch_dequant_t(const uint8_t *w, size_t n, float *out, hipStream_t st)
{
    hipLaunchKernelGGL((dequant_k<T>), dim3(grid_for(n)), dim3(256), 0, st, w, (uint64_t)n, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_dequant(uint32_t type, const uint8_t *w, size_t n, float *out, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) return 0;
    switch (type) {
    case T_F32: return launch_dequant_t<T_F32>(w, n, out, st);
    case T_F16: return launch_dequant_t<T_F16>(w, n, out, st);
    case T_Q4_0: return launch_dequant_t<T_Q4_0>(w, n, out, st);
    case T_Q5_0: return launch_dequant_t<T_Q5_0>(w, n, out, st);
    case T_Q8_0: return launch_dequant_t<T_Q8_0>(w, n, out, st);
    case T_Q4_K: return launch_dequant_t<T_Q4_K>(w, n, out, st);
    case T_Q5_K: return launch_dequant_t<T_Q5_K>(w, n, out, st);
    case T_Q6_K: return launch_dequant_t<T_Q6_K>(w, n, out, st);
    default: return -1;
    }
}

template <uint32_t T>
static int launch_deq_row_t(const uint8_t *w, size_t rows, size_t cols, size_t row, const uint32_t *d_row,
                            uint32_t nrows, float *out, size_t ldo, hipStream_t st)
{
    const uint64_t bs = block_elems(T);
    const uint64_t n = (cols + bs - 1) / bs * bs;
    hipLaunchKernelGGL((deq_row_k<T>), dim3(grid_for(n), nrows), dim3(256), 0, st, w, (uint64_t)rows,
                       (uint64_t)cols, (uint64_t)row, d_row, out, (uint64_t)ldo);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

static int launch_dequantize_row_any(uint32_t type, const uint8_t *w, size_t rows, size_t cols, size_t row,
                              const uint32_t *d_row, uint32_t nrows, float *out, size_t ldo, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (cols == 0 || nrows == 0) return 0;
    if (nrows > 65535u) return -1;
    switch (type) {
    case T_F32: return launch_deq_row_t<T_F32>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_F16: return launch_deq_row_t<T_F16>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q4_0: return launch_deq_row_t<T_Q4_0>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q5_0: return launch_deq_row_t<T_Q5_0>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q8_0: return launch_deq_row_t<T_Q8_0>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q4_K: return launch_deq_row_t<T_Q4_K>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q5_K: return launch_deq_row_t<T_Q5_K>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    case T_Q6_K: return launch_deq_row_t<T_Q6_K>(w, rows, cols, row, d_row, nrows, out, ldo, st);
    default: return -1;
    }
}

int launch_dequantize_row(uint32_t type, const uint8_t *w, size_t rows, size_t cols, size_t row,
                          float *out, ihipStream_t *stream)
{
    return launch_dequantize_row_any(type, w, rows, cols, row, nullptr, 1, out, 0, stream);
}

int launch_dequantize_row_dev(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const uint32_t *d_row,
                              float *out, ihipStream_t *stream)
{
    return launch_dequantize_row_any(type, w, rows, cols, 0, d_row, 1, out, 0, stream);
}

int launch_dequantize_rows_dev(uint32_t type, const uint8_t *w, size_t rows, size_t cols, const uint32_t *d_rows,
                               uint32_t n, float *out, size_t ldo, ihipStream_t *stream)
{
    return launch_dequantize_row_any(type, w, rows, cols, 0, d_rows, n, out, ldo, stream);
}

int launch_fill(float *out, size_t n, float v, ihipStream_t *stream)
{
    if (n == 0) return 0;
    hipLaunchKernelGGL(fill_k, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, out,
                       (uint64_t)n, v);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_silu_mul(const float *g, const float *u, float *out, size_t n, ihipStream_t *stream)
{
    if (n == 0) return 0;
    hipLaunchKernelGGL(silu_mul_k, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, g, u, out, (uint64_t)n);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_rmsnorm(const float *a, const float *b, float *sum_out, const float *w, float *out, size_t n,
                   float eps, ihipStream_t *stream)
{
    if (n == 0) return 0;
    if (n > 0xFFFFFFFFull) return -1;
    hipLaunchKernelGGL(rmsnorm_k, dim3(1), dim3(kNormBlock), 0, (hipStream_t)stream, a, b, sum_out, w, out,
                       (uint32_t)n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace qg

#ifdef QG_TIMELINE
#include "qgemv.h"

// The stamps of the last instrumented launch (libqgemv_timeline.so only):
// n values, 64 per workgroup, and the stamp clock in kHz.
extern "C" int qg_timeline_read(uint64_t *out, size_t n, int *clock_khz)
{
    const size_t cap = (size_t)qg::kTlWG * qg::kTlEv;
    if (!out) return QG_ERR_INVALID_ARG;
    if (n > cap) n = cap;
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(qg::qg_tl_buf), n * sizeof(uint64_t), 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return QG_ERR_HIP;
    int dev = 0;
    if (clock_khz && (hipGetDevice(&dev) != hipSuccess ||
                      hipDeviceGetAttribute(clock_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess))
        return QG_ERR_HIP;
    return QG_OK;
}

extern "C" int qg_timeline_clear(void)
{
    static uint64_t zero[qg::kTlWG * qg::kTlEv];
    return hipMemcpyToSymbol(HIP_SYMBOL(qg::qg_tl_buf), zero, sizeof zero, 0, hipMemcpyHostToDevice) == hipSuccess
               ? QG_OK
               : QG_ERR_HIP;
}
#endif
