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
//   gemv_team<T,..>   the fast path: a "team" of lanes owns one row group,
//                     each lane one 64-weight item (32 for F32) whose x slice
//                     stays in VGPRs for every row group the team visits
#include <hip/hip_runtime.h>

#include "qg_common.h"

namespace qg {

// ---------------------------------------------------------------- helpers

// Opaque AND/XOR: hides the mask from the instruction combiner, which would
// otherwise turn "(w & 0x0F0F0F0F) >> 8k & 0xFF" into one v_bfe per byte
// instead of one v_and per four bytes feeding v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t andm(uint32_t a, uint32_t m)
{
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(a));
    return r;
}
__device__ __forceinline__ uint32_t xorm(uint32_t a, uint32_t m)
{
    uint32_t r;
    asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(a));
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

// ------------------------------------------- bit-exact element decoders
// elem<T>(block, i) = value i of the block, as src/quant.rs:82-149 computes it.

template <uint32_t T> __device__ float elem(const uint8_t *b, uint32_t i);

template <> __device__ __forceinline__ float elem<T_F32>(const uint8_t *b, uint32_t)
{
    return __uint_as_float(*(const uint32_t *)b);
}
template <> __device__ __forceinline__ float elem<T_F16>(const uint8_t *b, uint32_t)
{
    return h2f_exact(rd16(b));
}
template <> __device__ __forceinline__ float elem<T_Q8_0>(const uint8_t *b, uint32_t i)
{
    const float d = h2f_exact(rd16(b));                          // quant.rs:107
    return d * (float)(int8_t)b[2 + i];                          // quant.rs:110
}
template <> __device__ __forceinline__ float elem<T_Q4_0>(const uint8_t *b, uint32_t i)
{
    const float d = h2f_exact(rd16(b));
    const uint32_t v = b[2 + i / 2];                             // quant.rs:117-118 (interleaved)
    const int nib = (i & 1u) ? (int)(v >> 4) : (int)(v & 15u);
    return d * (float)(nib - 8);
}
template <> __device__ __forceinline__ float elem<T_Q5_0>(const uint8_t *b, uint32_t i)
{
    const float d = h2f_exact(rd16(b));
    const uint32_t qh = rd16(b + 2) | (rd16(b + 4) << 16);
    const uint32_t xl = i < 16u ? (b[6 + i] & 15u) : (uint32_t)(b[6 + i - 16] >> 4);
    const uint32_t xh = ((qh >> i) & 1u) << 4;                   // quant.rs:126-135
    return d * (float)((int)(xl | xh) - 16);
}
template <> __device__ __forceinline__ float elem<T_Q4_K>(const uint8_t *b, uint32_t i)
{
    const float d = h2f_exact(rd16(b)), dmin = h2f_exact(rd16(b + 2));
    const uint32_t j = i >> 5, l = i & 31u;
    const uint8_t *s = b + 4;
    uint32_t sc, m;
    k4sm(j, s[0] | (s[1] << 8) | (s[2] << 16) | ((uint32_t)s[3] << 24),
         s[4] | (s[5] << 8) | (s[6] << 16) | ((uint32_t)s[7] << 24),
         s[8] | (s[9] << 8) | (s[10] << 16) | ((uint32_t)s[11] << 24), sc, m);
    const uint32_t q = b[16 + (j >> 1) * 32 + l];
    const uint32_t nib = (j & 1u) ? (q >> 4) : (q & 15u);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;        // quant.rs:218-219
    return d1 * (float)nib - m1;                                 // quant.rs:224-225
}
template <> __device__ __forceinline__ float elem<T_Q5_K>(const uint8_t *b, uint32_t i)
{
    const float d = h2f_exact(rd16(b)), dmin = h2f_exact(rd16(b + 2));
    const uint32_t j = i >> 5, l = i & 31u;
    const uint8_t *s = b + 4;
    uint32_t sc, m;
    k4sm(j, s[0] | (s[1] << 8) | (s[2] << 16) | ((uint32_t)s[3] << 24),
         s[4] | (s[5] << 8) | (s[6] << 16) | ((uint32_t)s[7] << 24),
         s[8] | (s[9] << 8) | (s[10] << 16) | ((uint32_t)s[11] << 24), sc, m);
    const uint32_t q = b[48 + (j >> 1) * 32 + l];
    const uint32_t lo = (j & 1u) ? (q >> 4) : (q & 15u);
    const uint32_t hi = ((b[16 + l] >> j) & 1u) ? 16u : 0u;     // u1/u2 = bit j, quant.rs:238-260
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    return d1 * (float)(lo + hi) - m1;
}
template <> __device__ __forceinline__ float elem<T_Q6_K>(const uint8_t *b, uint32_t i)
{
    const uint32_t n = i >> 7, rr = i & 127u, k = rr >> 5, l = rr & 31u, is = l >> 4;
    const uint32_t qlb = b[64 * n + l + 32 * (k & 1u)];
    const uint32_t nib = k >= 2u ? (qlb >> 4) : (qlb & 15u);
    const uint32_t hb = (b[128 + 32 * n + l] >> (2 * k)) & 3u;
    const int q = (int)(nib | (hb << 4));
    const float sc = (float)(int8_t)b[192 + 8 * n + is + 2 * k];
    const float d = h2f_exact(rd16(b + 208));
    return d * sc * (float)(q - 32);                             // quant.rs:286-289
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

// quant.rs:152-174: writes only the positions the reference writes.
template <uint32_t T>
__global__ void __launch_bounds__(256) deq_row_k(const uint8_t *__restrict__ w, uint64_t rows,
                                                 uint64_t cols, uint64_t row,
                                                 float *__restrict__ out)
{
    constexpr uint64_t BS = block_elems(T), BB = block_bytes(T);
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

__global__ void fill_k(float *out, uint64_t n, float v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = v;
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

// ------------------------------------------------------ team GEMV items
//
// An item is the unit one lane decodes per row group: 64 consecutive-in-block
// weights (32 for F32), split into S segments of SEG weights that each lie in
// one row.  Every quant type is reduced to unsigned codes u (one byte each,
// converted with v_cvt_f32_ubyte) so that a segment contributes
//     scale * (sum u*x) - offset_or_min * (sum x)
// with sum x precomputed once per lane (x never changes during a launch).

template <uint32_t T> struct Item;

// Q4_K (quant.rs:210-228): item = (block, pair p): sub-blocks 2p (low nibbles)
// and 2p+1 (high nibbles) of qs[32p .. 32p+32].
template <> struct Item<T_Q4_K> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 12, UNIT = 256;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 2) * 256u + (it & 3u) * 64u + s * 32u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 2) * 144u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint8_t *b = gb + (it >> 2) * 144u;
        const uint4 h = *(const uint4 *)b;
        const uint4 *q = (const uint4 *)(b + 16u + (it & 3u) * 32u);
        const uint4 q0 = q[0], q1 = q[1];
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = q0.x; r[5] = q0.y; r[6] = q0.z; r[7] = q0.w;
        r[8] = q1.x; r[9] = q1.y; r[10] = q1.z; r[11] = q1.w;
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t it, float (&out)[S])
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        const uint32_t j = (it & 3u) * 2u;
        uint32_t sc0, m0, sc1, m1;
        k4sm(j, r[1], r[2], r[3], sc0, m0);
        k4sm(j + 1u, r[1], r[2], r[3], sc1, m1);
        float a = 0.f, b = 0.f, a2 = 0.f, b2 = 0.f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t lo = andm(r[4 + t], 0x0F0F0F0Fu), hi = andm(r[4 + t], 0xF0F0F0F0u);
            a = __builtin_fmaf(ub(lo, 0), xs[4 * t + 0], a);
            b = __builtin_fmaf(ub(hi, 0), xs[32 + 4 * t + 0], b);
            a2 = __builtin_fmaf(ub(lo, 1), xs[4 * t + 1], a2);
            b2 = __builtin_fmaf(ub(hi, 1), xs[32 + 4 * t + 1], b2);
            a = __builtin_fmaf(ub(lo, 2), xs[4 * t + 2], a);
            b = __builtin_fmaf(ub(hi, 2), xs[32 + 4 * t + 2], b);
            a2 = __builtin_fmaf(ub(lo, 3), xs[4 * t + 3], a2);
            b2 = __builtin_fmaf(ub(hi, 3), xs[32 + 4 * t + 3], b2);
        }
        a += a2;
        b += b2;
        out[0] = __builtin_fmaf(d * (float)sc0, a, -(dmin * (float)m0) * sx[0]);
        out[1] = __builtin_fmaf(d * (float)sc1 * 0.0625f, b, -(dmin * (float)m1) * sx[1]);
    }
};

// Q5_K (quant.rs:231-262): as Q4_K plus the fifth bit, bit j of qh[l].
template <> struct Item<T_Q5_K> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 20, UNIT = 256;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 2) * 256u + (it & 3u) * 64u + s * 32u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 2) * 176u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint8_t *b = gb + (it >> 2) * 176u;
        const uint4 h = *(const uint4 *)b;
        const uint4 *qh = (const uint4 *)(b + 16u);
        const uint4 *q = (const uint4 *)(b + 48u + (it & 3u) * 32u);
        const uint4 h0 = qh[0], h1 = qh[1], q0 = q[0], q1 = q[1];
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = h0.x; r[5] = h0.y; r[6] = h0.z; r[7] = h0.w;
        r[8] = h1.x; r[9] = h1.y; r[10] = h1.z; r[11] = h1.w;
        r[12] = q0.x; r[13] = q0.y; r[14] = q0.z; r[15] = q0.w;
        r[16] = q1.x; r[17] = q1.y; r[18] = q1.z; r[19] = q1.w;
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t it, float (&out)[S])
    {
        const float d = h2f(r[0]), dmin = h2f(r[0] >> 16);
        const uint32_t j = (it & 3u) * 2u;
        uint32_t sc0, m0, sc1, m1;
        k4sm(j, r[1], r[2], r[3], sc0, m0);
        k4sm(j + 1u, r[1], r[2], r[3], sc1, m1);
        float a = 0.f, b = 0.f, a2 = 0.f, b2 = 0.f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t w = r[12 + t], hb = r[4 + t];
            const uint32_t qa = andm(w, 0x0F0F0F0Fu) | (((hb >> j) & 0x01010101u) << 4);
            const uint32_t qb = andm(w >> 4, 0x0F0F0F0Fu) | (((hb >> (j + 1u)) & 0x01010101u) << 4);
            a = __builtin_fmaf(ub(qa, 0), xs[4 * t + 0], a);
            b = __builtin_fmaf(ub(qb, 0), xs[32 + 4 * t + 0], b);
            a2 = __builtin_fmaf(ub(qa, 1), xs[4 * t + 1], a2);
            b2 = __builtin_fmaf(ub(qb, 1), xs[32 + 4 * t + 1], b2);
            a = __builtin_fmaf(ub(qa, 2), xs[4 * t + 2], a);
            b = __builtin_fmaf(ub(qb, 2), xs[32 + 4 * t + 2], b);
            a2 = __builtin_fmaf(ub(qa, 3), xs[4 * t + 3], a2);
            b2 = __builtin_fmaf(ub(qb, 3), xs[32 + 4 * t + 3], b2);
        }
        a += a2;
        b += b2;
        out[0] = __builtin_fmaf(d * (float)sc0, a, -(dmin * (float)m0) * sx[0]);
        out[1] = __builtin_fmaf(d * (float)sc1, b, -(dmin * (float)m1) * sx[1]);
    }
};

// Q6_K (quant.rs:265-292): item = (block, half n, i = l/16): 4 segments of 16,
// elements 128n + 32k + 16i + (0..15), k = 0..3.  Blocks are 210 bytes, so
// fields sit at 2-byte alignment: load aligned dword windows and realign
// with v_alignbyte.
template <> struct Item<T_Q6_K> {
    static constexpr uint32_t IE = 64, S = 4, SEG = 16, NRAW = 15, UNIT = 256;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s)
    {
        return (it >> 2) * 256u + ((it >> 1) & 1u) * 128u + s * 32u + (it & 1u) * 16u;
    }
    __device__ static uint32_t item_byte(uint32_t it) { return (it >> 2) * 210u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint8_t *b = gb + (it >> 2) * 210u;
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
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t it, float (&out)[S])
    {
        const float d = h2f(r[14]);
        const uint32_t i8 = (it & 1u) * 8u;
        float dot[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t A = r[t], B = r[4 + t], H = r[8 + t];
            const uint32_t q[4] = {andm(A, 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u),
                                   andm(B, 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u),
                                   andm(A >> 4, 0x0F0F0F0Fu) | (H & 0x30303030u),
                                   andm(B >> 4, 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
            for (int k = 0; k < 4; k++)
#pragma unroll
                for (int bb = 0; bb < 4; bb++)
                    dot[k] = __builtin_fmaf(ub(q[k], bb), xs[16 * k + 4 * t + bb], dot[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // sc[8n + i + 2k]: byte (i + 2(k&1)) of dword r[12 + k/2]
            const int sc = __builtin_amdgcn_sbfe((int)r[12 + (k >> 1)], (int)(i8 + 16u * (k & 1)), 8);
            out[k] = (d * (float)sc) * __builtin_fmaf(-32.0f, sx[k], dot[k]);
        }
    }
};

// Q8_0 (quant.rs:106-113): item = two blocks (68 bytes, 4-byte aligned).
// Block 0's codes sit at byte 2 (realigned), block 1's at byte 36 (aligned).
// Signed codes become unsigned with ^0x80: q = u - 128.
template <> struct Item<T_Q8_0> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 17, UNIT = 64;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 68u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)(gb + it * 68u);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const U4a u = *(const U4a *)(p + 4 * v);
            r[4 * v] = u.a; r[4 * v + 1] = u.b; r[4 * v + 2] = u.c; r[4 * v + 3] = u.d;
        }
        r[16] = p[16];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t, float (&out)[S])
    {
        const float d0 = h2f(r[0]), d1 = h2f(r[8] >> 16);
        float a = 0.f, b = 0.f, a2 = 0.f, b2 = 0.f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t u0 = xorm(__builtin_amdgcn_alignbyte(r[t + 1], r[t], 2u), 0x80808080u);
            const uint32_t u1 = xorm(r[9 + t], 0x80808080u);
            a = __builtin_fmaf(ub(u0, 0), xs[4 * t + 0], a);
            b = __builtin_fmaf(ub(u1, 0), xs[32 + 4 * t + 0], b);
            a2 = __builtin_fmaf(ub(u0, 1), xs[4 * t + 1], a2);
            b2 = __builtin_fmaf(ub(u1, 1), xs[32 + 4 * t + 1], b2);
            a = __builtin_fmaf(ub(u0, 2), xs[4 * t + 2], a);
            b = __builtin_fmaf(ub(u1, 2), xs[32 + 4 * t + 2], b);
            a2 = __builtin_fmaf(ub(u0, 3), xs[4 * t + 3], a2);
            b2 = __builtin_fmaf(ub(u1, 3), xs[32 + 4 * t + 3], b2);
        }
        a += a2;
        b += b2;
        out[0] = d0 * __builtin_fmaf(-128.0f, sx[0], a);
        out[1] = d1 * __builtin_fmaf(-128.0f, sx[1], b);
    }
};

// Q4_0 (quant.rs:114-121): two blocks (36 bytes).  Interleaved nibble order:
// byte j holds element 2j (low nibble) and 2j+1 (high nibble).
template <> struct Item<T_Q4_0> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 9, UNIT = 64;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 36u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)(gb + it * 36u);
        const U4a u0 = *(const U4a *)p, u1 = *(const U4a *)(p + 4);
        r[0] = u0.a; r[1] = u0.b; r[2] = u0.c; r[3] = u0.d;
        r[4] = u1.a; r[5] = u1.b; r[6] = u1.c; r[7] = u1.d;
        r[8] = p[8];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t, float (&out)[S])
    {
        const float dd[2] = {h2f(r[0]), h2f(r[4] >> 16)};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float e = 0.f, o = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = s == 0 ? __builtin_amdgcn_alignbyte(r[t + 1], r[t], 2u) : r[5 + t];
                const uint32_t lo = andm(q, 0x0F0F0F0Fu), hi = andm(q, 0xF0F0F0F0u);
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    e = __builtin_fmaf(ub(lo, bb), xs[32 * s + 8 * t + 2 * bb], e);
                    o = __builtin_fmaf(ub(hi, bb), xs[32 * s + 8 * t + 2 * bb + 1], o);
                }
            }
            out[s] = dd[s] * (__builtin_fmaf(o, 0.0625f, e) - 8.0f * sx[s]);
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
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 44u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint32_t *p = (const uint32_t *)(gb + it * 44u);
        const U4a u0 = *(const U4a *)p, u1 = *(const U4a *)(p + 4);
        r[0] = u0.a; r[1] = u0.b; r[2] = u0.c; r[3] = u0.d;
        r[4] = u1.a; r[5] = u1.b; r[6] = u1.c; r[7] = u1.d;
        r[8] = p[8]; r[9] = p[9]; r[10] = p[10];
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&sx)[S], uint32_t, float (&out)[S])
    {
        const float dd[2] = {h2f(r[0]), h2f(r[5] >> 16)};
        const uint32_t qh[2] = {__builtin_amdgcn_alignbyte(r[1], r[0], 2u), r[6]};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float a = 0.f, b = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = s == 0 ? __builtin_amdgcn_alignbyte(r[t + 2], r[t + 1], 2u) : r[7 + t];
                const uint32_t lo = andm(q, 0x0F0F0F0Fu) | spread4(qh[s] >> (4 * t));
                const uint32_t hi = andm(q >> 4, 0x0F0F0F0Fu) | spread4(qh[s] >> (16 + 4 * t));
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    a = __builtin_fmaf(ub(lo, bb), xs[32 * s + 4 * t + bb], a);
                    b = __builtin_fmaf(ub(hi, bb), xs[32 * s + 16 + 4 * t + bb], b);
                }
            }
            out[s] = dd[s] * __builtin_fmaf(-16.0f, sx[s], a + b);
        }
    }
};

// F16: 64 halves (128 bytes, 16-byte aligned).
template <> struct Item<T_F16> {
    static constexpr uint32_t IE = 64, S = 2, SEG = 32, NRAW = 32, UNIT = 64;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t s) { return it * 64u + s * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 128u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint4 *p = (const uint4 *)(gb + it * 128u);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint4 u = p[v];
            r[4 * v] = u.x; r[4 * v + 1] = u.y; r[4 * v + 2] = u.z; r[4 * v + 3] = u.w;
        }
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&)[S], uint32_t, float (&out)[S])
    {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float a = 0.f, b = 0.f;
#pragma unroll
            for (int t = 0; t < 16; t++) {
                a = __builtin_fmaf(h2f(r[16 * s + t]), xs[32 * s + 2 * t], a);
                b = __builtin_fmaf(h2f(r[16 * s + t] >> 16), xs[32 * s + 2 * t + 1], b);
            }
            out[s] = a + b;
        }
    }
};

// F32: 32 floats (128 bytes).
template <> struct Item<T_F32> {
    static constexpr uint32_t IE = 32, S = 1, SEG = 32, NRAW = 32, UNIT = 32;
    __device__ static uint32_t seg_elem(uint32_t it, uint32_t) { return it * 32u; }
    __device__ static uint32_t item_byte(uint32_t it) { return it * 128u; }
    __device__ static void load(const uint8_t *gb, uint32_t it, uint32_t (&r)[NRAW])
    {
        const uint4 *p = (const uint4 *)(gb + it * 128u);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint4 u = p[v];
            r[4 * v] = u.x; r[4 * v + 1] = u.y; r[4 * v + 2] = u.z; r[4 * v + 3] = u.w;
        }
    }
    __device__ static void compute(const uint32_t (&r)[NRAW], const float (&xs)[S * SEG],
                                   const float (&)[S], uint32_t, float (&out)[S])
    {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            a = __builtin_fmaf(__uint_as_float(r[2 * t]), xs[2 * t], a);
            b = __builtin_fmaf(__uint_as_float(r[2 * t + 1]), xs[2 * t + 1], b);
        }
        out[0] = a + b;
    }
};

template <uint32_t T> constexpr int rows_per_batch()
{
    return T == T_Q4_K ? 4 : T == T_Q4_0 ? 4 : T == T_Q5_0 ? 4 : T == T_F16 || T == T_F32 ? 1 : 2;
}

// ------------------------------------------------------- team GEMV kernel

struct TeamArgs {
    const uint8_t *w;
    const float *x;
    float *y;
    uint64_t nbytes, group_bytes;
    uint32_t rows, cols, g, n_groups, ni, n_teams, n_batches;
};

// TSUB > 0: teams of TSUB lanes inside 256-thread workgroups (several teams per
// wave when TSUB < 64).  TSUB == 0: one team per workgroup of blockDim.x lanes
// (up to 8 waves), reduced across waves through LDS.
template <uint32_t T, int TSUB>
__global__ void __launch_bounds__(TSUB ? 256 : 512) gemv_team(TeamArgs a)
{
    using I = Item<T>;
    constexpr int S = I::S, SEG = I::SEG, R = rows_per_batch<T>();
    const uint32_t tid = threadIdx.x;
    const uint32_t lt = TSUB ? (tid & (uint32_t)(TSUB - 1)) : tid;
    const uint32_t team = TSUB ? blockIdx.x * (256u / TSUB) + tid / TSUB : blockIdx.x;
    const bool active = lt < a.ni;

    float xs[S * SEG], sx[S];
    uint32_t srow[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        sx[s] = 0.f;
        srow[s] = 0xFFFFFFFFu;
#pragma unroll
        for (int e = 0; e < SEG; e++) xs[s * SEG + e] = 0.f;
    }
    if (active) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t e = I::seg_elem(lt, s);
            srow[s] = e / a.cols;
            const float4 *xp = (const float4 *)(a.x + (e - srow[s] * a.cols));
#pragma unroll
            for (int v = 0; v < SEG / 4; v++) {
                const float4 f = xp[v];
                xs[s * SEG + 4 * v] = f.x; xs[s * SEG + 4 * v + 1] = f.y;
                xs[s * SEG + 4 * v + 2] = f.z; xs[s * SEG + 4 * v + 3] = f.w;
            }
            float t = 0.f;
#pragma unroll
            for (int e2 = 0; e2 < SEG; e2++) t += xs[s * SEG + e2];
            sx[s] = t;
        }
    }
    const uint64_t ib = I::item_byte(lt);
    __shared__ float red[TSUB ? 1 : 8][R * 8];

    for (uint32_t bt = team; bt < a.n_batches; bt += a.n_teams) {
        uint32_t raw[R][I::NRAW];
        bool ok[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t grp = bt * R + r;
            const uint64_t gbase = (uint64_t)grp * a.group_bytes;
            ok[r] = active && grp < a.n_groups && gbase + ib < a.nbytes;
            if (ok[r]) I::load(a.w + gbase, lt, raw[r]);
        }
        float acc[R][S];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (ok[r]) {
                I::compute(raw[r], xs, sx, lt, acc[r]);
            } else {
#pragma unroll
                for (int s = 0; s < S; s++) acc[r][s] = 0.f;
            }
        }
        if (TSUB) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t grp = bt * R + r;
                if (grp >= a.n_groups) break;                   // team-uniform
                for (uint32_t gi = 0; gi < a.g; gi++) {
                    float v = 0.f;
#pragma unroll
                    for (int s = 0; s < S; s++) v += srow[s] == gi ? acc[r][s] : 0.f;
#pragma unroll
                    for (int o = TSUB / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, TSUB);
                    const uint32_t row = grp * a.g + gi;
                    if (lt == 0 && row < a.rows) a.y[row] = v;
                }
            }
        } else {
            const uint32_t wave = tid >> 6, lane = tid & 63u;
#pragma unroll
            for (int r = 0; r < R; r++) {
                for (uint32_t gi = 0; gi < a.g; gi++) {
                    float v = 0.f;
#pragma unroll
                    for (int s = 0; s < S; s++) v += srow[s] == gi ? acc[r][s] : 0.f;
                    v = wave_sum(v);
                    if (lane == 0) red[wave][r * a.g + gi] = v;
                }
            }
            __syncthreads();
            if (tid < R * a.g) {
                const uint32_t r = tid / a.g, gi = tid - r * a.g, grp = bt * R + r;
                float s = 0.f;
                for (uint32_t wv = 0; wv < (blockDim.x >> 6); wv++) s += red[wv][tid];
                const uint32_t row = grp * a.g + gi;
                if (grp < a.n_groups && row < a.rows) a.y[row] = s;
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------ planning

static uint32_t gcd_u(uint64_t a, uint64_t b)
{
    while (b) { uint64_t t = a % b; a = b; b = t; }
    return (uint32_t)a;
}

template <uint32_t T> static void plan_team(size_t rows, size_t cols, int n_cu, Plan *p)
{
    using I = Item<T>;
    constexpr uint32_t R = rows_per_batch<T>();
    p->kind = 0;
    if (cols % 32 != 0 || rows == 0 || cols == 0) return;
    const uint64_t unit = I::UNIT;                       // elements per aligned row-group unit
    const uint64_t g = unit / gcd_u(cols, unit);
    const uint64_t gel = g * cols;
    const uint64_t ni = gel / I::IE;
    if (ni > 512 || g > 8) return;
    uint32_t ts;
    if (ni <= 64) { ts = 4; while (ts < ni) ts <<= 1; }
    else ts = (uint32_t)((ni + 63) / 64 * 64);
    p->g = (uint32_t)g;
    p->ni = (uint32_t)ni;
    p->ts = ts;
    p->tsub = ts <= 64 ? ts : 0;
    p->n_groups = (uint32_t)((rows + g - 1) / g);
    p->group_bytes = gel / block_elems(T) * block_bytes(T);
    const uint64_t n_batches = (p->n_groups + R - 1) / R;
    // aim for ~16 waves per CU resident, then balance batches per team
    const uint64_t waves_target = (uint64_t)(n_cu > 0 ? n_cu : 256) * 16;
    const uint64_t teams_target = ts <= 64 ? waves_target * (64 / ts) : waves_target / (ts / 64);
    const uint64_t per_team = (n_batches + teams_target - 1) / (teams_target ? teams_target : 1);
    uint64_t n_teams = (n_batches + per_team - 1) / per_team;
    const uint32_t tpb = p->tsub ? 256u / ts : 1u;
    p->block = p->tsub ? 256u : ts;
    p->grid = (uint32_t)((n_teams + tpb - 1) / tpb);
    p->n_teams = p->grid * tpb;
    p->kind = 1;
}

int make_plan(uint32_t type, size_t rows, size_t cols, int n_cu, Plan *p)
{
    *p = Plan{};
    if (rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull) return 0;
    switch (type) {
    case T_F32: plan_team<T_F32>(rows, cols, n_cu, p); break;
    case T_F16: plan_team<T_F16>(rows, cols, n_cu, p); break;
    case T_Q4_0: plan_team<T_Q4_0>(rows, cols, n_cu, p); break;
    case T_Q5_0: plan_team<T_Q5_0>(rows, cols, n_cu, p); break;
    case T_Q8_0: plan_team<T_Q8_0>(rows, cols, n_cu, p); break;
    case T_Q4_K: plan_team<T_Q4_K>(rows, cols, n_cu, p); break;
    case T_Q5_K: plan_team<T_Q5_K>(rows, cols, n_cu, p); break;
    case T_Q6_K: plan_team<T_Q6_K>(rows, cols, n_cu, p); break;
    default: return -1;
    }
    return 0;
}

// ------------------------------------------------------------ launchers

template <uint32_t T>
static int launch_team_t(const Plan &p, const uint8_t *w, size_t nbytes, size_t rows, size_t cols,
                         const float *x, float *y, hipStream_t st)
{
    TeamArgs a;
    a.w = w; a.x = x; a.y = y; a.nbytes = nbytes; a.group_bytes = p.group_bytes;
    a.rows = (uint32_t)rows; a.cols = (uint32_t)cols; a.g = p.g; a.n_groups = p.n_groups;
    a.ni = p.ni; a.n_teams = p.n_teams;
    a.n_batches = (p.n_groups + rows_per_batch<T>() - 1) / rows_per_batch<T>();
    dim3 grid(p.grid), block(p.block);
    switch (p.tsub) {
    case 4: hipLaunchKernelGGL((gemv_team<T, 4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((gemv_team<T, 8>), grid, block, 0, st, a); break;
    case 16: hipLaunchKernelGGL((gemv_team<T, 16>), grid, block, 0, st, a); break;
    case 32: hipLaunchKernelGGL((gemv_team<T, 32>), grid, block, 0, st, a); break;
    case 64: hipLaunchKernelGGL((gemv_team<T, 64>), grid, block, 0, st, a); break;
    case 0: hipLaunchKernelGGL((gemv_team<T, 0>), grid, block, 0, st, a); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_gemv(uint32_t type, const Plan &p, const uint8_t *w, size_t nbytes, size_t rows,
                size_t cols, const float *x, float *y, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (p.kind != 1) return launch_gemv_generic(type, w, rows, cols, x, y, stream);
    switch (type) {
    case T_F32: return launch_team_t<T_F32>(p, w, nbytes, rows, cols, x, y, st);
    case T_F16: return launch_team_t<T_F16>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q4_0: return launch_team_t<T_Q4_0>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q5_0: return launch_team_t<T_Q5_0>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q8_0: return launch_team_t<T_Q8_0>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q4_K: return launch_team_t<T_Q4_K>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q5_K: return launch_team_t<T_Q5_K>(p, w, nbytes, rows, cols, x, y, st);
    case T_Q6_K: return launch_team_t<T_Q6_K>(p, w, nbytes, rows, cols, x, y, st);
    default: return -1;
    }
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
static int launch_deq_row_t(const uint8_t *w, size_t rows, size_t cols, size_t row, float *out,
                            hipStream_t st)
{
    const uint64_t bs = block_elems(T);
    const uint64_t n = (cols + bs - 1) / bs * bs;
    hipLaunchKernelGGL((deq_row_k<T>), dim3(grid_for(n)), dim3(256), 0, st, w, (uint64_t)rows,
                       (uint64_t)cols, (uint64_t)row, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_dequantize_row(uint32_t type, const uint8_t *w, size_t rows, size_t cols, size_t row,
                          float *out, ihipStream_t *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (cols == 0) return 0;
    switch (type) {
    case T_F32: return launch_deq_row_t<T_F32>(w, rows, cols, row, out, st);
    case T_F16: return launch_deq_row_t<T_F16>(w, rows, cols, row, out, st);
    case T_Q4_0: return launch_deq_row_t<T_Q4_0>(w, rows, cols, row, out, st);
    case T_Q5_0: return launch_deq_row_t<T_Q5_0>(w, rows, cols, row, out, st);
    case T_Q8_0: return launch_deq_row_t<T_Q8_0>(w, rows, cols, row, out, st);
    case T_Q4_K: return launch_deq_row_t<T_Q4_K>(w, rows, cols, row, out, st);
    case T_Q5_K: return launch_deq_row_t<T_Q5_K>(w, rows, cols, row, out, st);
    case T_Q6_K: return launch_deq_row_t<T_Q6_K>(w, rows, cols, row, out, st);
    default: return -1;
    }
}

int launch_fill(float *out, size_t n, float v, ihipStream_t *stream)
{
    if (n == 0) return 0;
    hipLaunchKernelGGL(fill_k, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, out,
                       (uint64_t)n, v);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace qg
