// qg_prefill.hip -- batched prefill: the prompt's tokens through one layer at
// a time (include/qgmodel.h, qg_model_prefill), the multi-token form of the
// decode step of qg_model.hip.
//
// The reference feeds the prompt one token at a time (model.rs:361-365,
// Transformer::forward per token).  Here every projection of a chunk of up
// to kPfMaxTokens tokens is one GEMM on the matrix cores:
//
//   * pf_split_k: each token's input vector x (the RMSNorm's numerator (h + o)
//     * nw of the residual stream, the attention output, or silu(g) * u)
//     scaled per 256-element group g by a power of two 2^e_g (the group's
//     largest magnitude into [512, 1024)) and split into two f16 pieces
//     xs = x 2^e_g = hi + lo (hi the rounding of xs, lo the rounding of what
//     hi leaves: 22 significant bits together), written chunk by chunk in the
//     layout of the GEMM's LDS buffers; per 32-element segment the sum of xs
//     (as two f16 pieces); per group 2^-e_g; with the norm, the partial sums
//     of squares per group (the consumer of the GEMM's output applies
//     1 / rms);
//   * pf_gemm_k: y[t][r] = sum over blocks of 2^-e_g (d D + sum over the
//     block's sub-blocks of -dmin m S) with D = sum over the block's
//     elements of xs B from chained v_mfma_f32_16x16x32_f16 (A: 16 tokens x
//     32 elements of one piece, B: 32 weights x 16 rows).  B holds integers
//     that f16 represents exactly -- sc q for Q4_K / Q5_K (at most 63 * 31),
//     the two parts 16 a q' and b q' of sc q' (sc = 16 a + b) for Q6_K, q for
//     Q8_0 -- so every product is exact and accumulates in f32; d 2^-e_g
//     multiplies D once per block (per sub-block for Q8_0; per chunk where a
//     row's blocks straddle the groups) and the K-quant min terms -dmin sum
//     m S are one v_mfma_f32_16x16x16_f16 per 4 sub-blocks (A: S, the sums of
//     xs, as two f16 pieces; B: m, exact);
//   * pf_qkv_post_k, pf_attention_k: bias, RoPE and KV append of every token
//     (attention.rs:66-90), causal attention of every token over the cache up
//     to its own slot (attention.rs:93-121), as the decode path.
//
// MFMA operand layout (v_mfma_f32_16x16x32_f16 and _bf16, checked on
// gfx950): lane l holds A[l % 16][8 (l/16) .. +8), B[8 (l/16) .. +8)[l % 16]
// and D[4 (l/16) + i][l % 16], i = 0..3.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "qg_common.h"

namespace qgp {

using qg::T_Q4_K;
using qg::T_Q5_K;
using qg::T_Q6_K;
using qg::T_Q8_0;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t h16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xFFFFu));
}

// the dword-aligned address at or below p
__device__ __forceinline__ const uint32_t *adown(const uint8_t *p)
{
    return (const uint32_t *)(p - ((uintptr_t)p & 3u));
}
// 4 bytes at byte offset s (0..3) of the dword pair (a, b)
__device__ __forceinline__ uint32_t abyte(uint32_t b, uint32_t a, uint32_t s)
{
    return __builtin_amdgcn_alignbyte(b, a, s);
}

// quant.rs:606-615 for the four sub-blocks jb .. jb + 3 (jb = 0 or 4; it may
// differ between lanes) at once: byte i of sc4 / m4 is the scale / min of
// sub-block jb + i, from the 12-byte pack held in the dwords q0, q1, q2
// (j < 4: q[j] & 63, q[j+4] & 63; j >= 4: (q[j+4] & 15) | (q[j-4] >> 6) << 4,
// (q[j+4] >> 4) | (q[j] >> 6) << 4), without branches
__device__ __forceinline__ void k4sm4(uint32_t jb, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t &sc4,
                                      uint32_t &m4)
{
    const uint32_t lo = 0u - (uint32_t)(jb < 4u);
    sc4 = (q0 & 0x3F3F3F3Fu & lo) | (((q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u)) & ~lo);
    m4 = (q1 & 0x3F3F3F3Fu & lo) | ((((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u)) & ~lo);
}

// The same for the sub-blocks 2 ph, 2 ph + 1, 4 + 2 ph, 5 + 2 ph (ph = 0 or
// 1: half ph of each of the block's two 128-element halves)
__device__ __forceinline__ void k4sm_ph(uint32_t ph, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t &sc4,
                                        uint32_t &m4)
{
    const uint32_t sel = 0x05040100u + ph * 0x02020202u;
    sc4 = __builtin_amdgcn_perm((q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u), q0 & 0x3F3F3F3Fu, sel);
    m4 = __builtin_amdgcn_perm(((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u), q1 & 0x3F3F3F3Fu, sel);
}

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 h) { return __builtin_bit_cast(uint32_t, h); }

// the f16 pairs 1024 + c of the byte codes of c: bytes 0, 1 and bytes 2, 3
// (1024 + c for c < 1024 is the f16 with bits 0x6400 | c)
__device__ __forceinline__ h2 mag_lo(uint32_t c) { return as_h2(__builtin_amdgcn_perm(0x64646464u, c, 0x04010400u)); }
__device__ __forceinline__ h2 mag_hi(uint32_t c) { return as_h2(__builtin_amdgcn_perm(0x64646464u, c, 0x04030402u)); }

// the f16 pair (v, v) of an integer |v| <= 2048 (exact)
__device__ __forceinline__ h2 hpair(int v)
{
    const _Float16 f = (_Float16)(int16_t)v;
    return h2{f, f};
}

// sc q for the 8 codes in the bytes of c0, c1 (q < 256, sc q <= 2048): one
// fused (1024 + q) sc - 1024 sc per pair, exact since the result is
__device__ __forceinline__ uint4 scaled_codes(uint32_t c0, uint32_t c1, h2 s, h2 o)
{
    return make_uint4(as_u(__builtin_elementwise_fma(mag_lo(c0), s, o)),
                      as_u(__builtin_elementwise_fma(mag_hi(c0), s, o)),
                      as_u(__builtin_elementwise_fma(mag_lo(c1), s, o)),
                      as_u(__builtin_elementwise_fma(mag_hi(c1), s, o)));
}

// A K-quant sub-block's B operand from its 8 codes (bytes of c0, c1) and the
// scale in byte kk of sc4 (the f16 pair (sc, sc) as 1024 + sc - 1024)
__device__ __forceinline__ uint4 kquant_b(uint32_t c0, uint32_t c1, uint32_t sc4, uint32_t kk)
{
    const h2 s = as_h2(__builtin_amdgcn_perm(0x64646464u, sc4, 0x04000400u | (kk * 0x00010001u))) -
                 h2{1024.0f16, 1024.0f16};
    return scaled_codes(c0, c1, s, s * h2{-1024.0f16, -1024.0f16});
}

// The min terms' B operand (v_mfma_f32_16x16x16_f16, K slot 2 kk + p = piece
// p of the sums of the chunk's sub-block kk): lane kq < 2 holds the mins of
// sub-blocks 2 kq, 2 kq + 1 (bytes of m4), each twice, as exact f16; kq >= 2
// zero.  Returned as two dwords.
__device__ __forceinline__ uint2 kquant_minb(uint32_t m4, uint32_t kq)
{
    const uint32_t b = 2u * (kq & 1u);
    const h2 one = h2{1024.0f16, 1024.0f16};
    const uint32_t lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, m4, 0x04000400u | (b * 0x00010001u))) - one);
    const uint32_t hi =
        as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, m4, 0x04000400u | ((b + 1u) * 0x00010001u))) - one);
    return kq < 2u ? make_uint2(lo, hi) : make_uint2(0u, 0u);
}

// Q6_K: codes q (6 bits) of c0, c1 as q' = q - 32, times the two parts of
// the signed scale sc = 16 a + b (a = sc >> 4, 0 <= b < 16): B1 = 16 a q'
// (a multiple of 16 of magnitude <= 4096 with at most 9 significant bits)
// and B2 = b q' (<= 480), each exact; B1 + B2 = sc q'
__device__ __forceinline__ void q6_b(uint32_t c0, uint32_t c1, int sc, uint4 &b1, uint4 &b2)
{
    const h2 A = hpair(16 * (sc >> 4)), B = hpair(sc & 15);
    const h2 off = h2{-1056.0f16, -1056.0f16};
    const h2 q0 = mag_lo(c0) + off, q1 = mag_hi(c0) + off, q2 = mag_lo(c1) + off, q3 = mag_hi(c1) + off;
    b1 = make_uint4(as_u(q0 * A), as_u(q1 * A), as_u(q2 * A), as_u(q3 * A));
    b2 = make_uint4(as_u(q0 * B), as_u(q1 * B), as_u(q2 * B), as_u(q3 * B));
}

// Q8_0: 8 signed byte codes as f16 (1024 + (q + 128) - 1152, exact)
__device__ __forceinline__ uint4 q8_b(uint32_t c0, uint32_t c1)
{
    const h2 off = h2{-1152.0f16, -1152.0f16};
    c0 ^= 0x80808080u;
    c1 ^= 0x80808080u;
    return make_uint4(as_u(mag_lo(c0) + off), as_u(mag_hi(c0) + off), as_u(mag_lo(c1) + off),
                      as_u(mag_hi(c1) + off));
}

// Per-type access to a chunk of 4 sub-blocks that lies inside one block
// (sub-blocks jb .. jb + 3 of it, jb = 0 or 4; for Q8_0, whose blocks are
// single sub-blocks, 4 consecutive blocks).  The lane (kq = lane / 16) needs
// codes 8 kq .. 8 kq + 7 of each sub-block, for the row of its column.
//   load(blk, jb, kq) / load_rp(G, b, jb, kq, ni): the raw dwords, from the
//     GGUF block at blk (every byte read lies in the matrix or its tail pad)
//     or from block b of the repacked row group G (ni items);
//   decode(c, jb, kk, kq, bq): the B operands of sub-block kk of the chunk;
//   dscale(c, kk): the scale that multiplies D (per block; per sub-block
//     for Q8_0);
//   minb(c, jb, kq, dmin): the min terms' B operand (kquant_minb) and dmin
//     (MIN types).
// NB: B operands per sub-block.
template <uint32_t T> struct PfH;

// Q4_K (quant.rs:210-228): 8 sub-blocks per 144-byte block; sub-block j is
// the low (j even) or high (j odd) nibbles of qs[32 (j/2) .. +32); the value
// is d sc q - dmin m.
template <> struct PfH<T_Q4_K> {
    static constexpr int NB = 1;
    static constexpr bool MIN = true;
    static constexpr uint32_t BB = 144;
    struct C {
        uint4 h;            // d, dmin, the 12 scale bytes
        uint2 v0, v1;       // the lane's code bytes of sub-block pairs jb/2 and jb/2 + 1
    };
    using CR = C;
    __device__ static C load(const uint8_t *blk, uint32_t jb, uint32_t kq)
    {
        const uint8_t *q = blk + 16u + 16u * jb + 8u * kq;
        return C{*(const uint4 *)blk, *(const uint2 *)q, *(const uint2 *)(q + 32u)};
    }
    // repack_k's row group: the ni/2 block heads, then piece k' (16 bytes)
    // of item it at 8 ni + (k' ni + it) 16; item it = the quant bytes
    // 64 (it & 1) .. +64 of block it / 2
    __device__ static CR load_rp(const uint8_t *G, uint32_t b, uint32_t jb, uint32_t kq, uint32_t ni)
    {
        const uint8_t *q = G + 8u * ni + (size_t)(((kq >> 1) * ni + 2u * b + (jb >> 2)) << 4) + 8u * (kq & 1u);
        return C{*(const uint4 *)(G + 16u * b), *(const uint2 *)q, *(const uint2 *)(q + 32u * ni)};
    }
    __device__ static void decode(const C &c, uint32_t jb, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t sh = 4u * (kk & 1u);
        uint32_t sc4, m4;
        k4sm4(jb, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b((v.x >> sh) & 0x0F0F0F0Fu, (v.y >> sh) & 0x0F0F0F0Fu, sc4, kk);
    }
    __device__ static void decode_rp(const CR &c, uint32_t jb, uint32_t kk, uint32_t kq, uint4 (&bq)[NB])
    {
        decode(c, jb, kk, kq, bq);
    }
    __device__ static float dscale(const C &c, uint32_t) { return h2f(c.h.x); }
    __device__ static uint2 minb(const C &c, uint32_t jb, uint32_t kq, float &dmin)
    {
        uint32_t sc4, m4;
        k4sm4(jb, c.h.y, c.h.z, c.h.w, sc4, m4);
        dmin = h2f(c.h.x >> 16);
        return kquant_minb(m4, kq);
    }
    // Phase chunks (see pf_gemm_rows): sub-blocks 2 ph, 2 ph + 1 (pair ph of
    // the block's first item) and 4 + 2 ph, 5 + 2 ph (pair ph of its second)
    __device__ static C load_ph(const uint8_t *blk, uint32_t ph, uint32_t kq)
    {
        const uint8_t *q = blk + 16u + 32u * ph + 8u * kq;
        return C{*(const uint4 *)blk, *(const uint2 *)q, *(const uint2 *)(q + 64u)};
    }
    __device__ static C load_rp_ph(const uint8_t *G, uint32_t b, uint32_t ph, uint32_t kq, uint32_t ni)
    {
        const uint8_t *q =
            G + 8u * ni + (size_t)(((2u * ph + (kq >> 1)) * ni + 2u * b) << 4) + 8u * (kq & 1u);
        return C{*(const uint4 *)(G + 16u * b), *(const uint2 *)q, *(const uint2 *)(q + 16u)};
    }
    __device__ static void decode_ph(const C &c, uint32_t ph, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t sh = 4u * (kk & 1u);
        uint32_t sc4, m4;
        k4sm_ph(ph, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b((v.x >> sh) & 0x0F0F0F0Fu, (v.y >> sh) & 0x0F0F0F0Fu, sc4, kk);
    }
    __device__ static uint2 minb_ph(const C &c, uint32_t ph, uint32_t kq, float &dmin)
    {
        uint32_t sc4, m4;
        k4sm_ph(ph, c.h.y, c.h.z, c.h.w, sc4, m4);
        dmin = h2f(c.h.x >> 16);
        return kquant_minb(m4, kq);
    }
};

// Q5_K (quant.rs:231-262): as Q4_K with a fifth bit, bit j of qh[l].
template <> struct PfH<T_Q5_K> {
    static constexpr int NB = 1;
    static constexpr bool MIN = true;
    static constexpr uint32_t BB = 176;
    struct C {
        uint4 h;
        uint2 v0, v1;       // as Q4_K (qs at 48)
        uint2 qh;           // qh[8 kq .. +8]
    };
    __device__ static C load(const uint8_t *blk, uint32_t jb, uint32_t kq)
    {
        const uint8_t *q = blk + 48u + 16u * jb + 8u * kq;
        return C{*(const uint4 *)blk, *(const uint2 *)q, *(const uint2 *)(q + 32u),
                 *(const uint2 *)(blk + 16u + 8u * kq)};
    }
    __device__ static void decode(const C &c, uint32_t jb, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t sh = 4u * (kk & 1u), j = jb + kk;
        const uint32_t c0 = ((v.x >> sh) & 0x0F0F0F0Fu) | (((c.qh.x >> j) & 0x01010101u) << 4);
        const uint32_t c1 = ((v.y >> sh) & 0x0F0F0F0Fu) | (((c.qh.y >> j) & 0x01010101u) << 4);
        uint32_t sc4, m4;
        k4sm4(jb, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b(c0, c1, sc4, kk);
    }
    // repack_k's row group: the ni/4 block heads, piece k' of item it's 32
    // quant bytes at 16 (ni/4) + (k' ni + it) 16, then 8 bytes per item at
    // 4 ni + 32 ni + 8 it: bits 8 bb + 2 t' + q of word w are bit
    // 2 (it & 3) + q of qh[16 w + 4 t' + bb]; item it = block it / 4,
    // sub-blocks 2 (it & 3) and 2 (it & 3) + 1
    struct CR {
        uint4 h;
        uint2 v0, v1;       // items 4 b + jb/2 and the next
        uint32_t w0, w1;
    };
    __device__ static CR load_rp(const uint8_t *G, uint32_t b, uint32_t jb, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = 4u * b + (jb >> 1), H = 4u * ni;
        const uint8_t *q = G + H + (size_t)(((kq >> 1) * ni + it) << 4) + 8u * (kq & 1u);
        const uint8_t *w = G + H + 32u * ni + 8u * it + 4u * (kq >> 1);
        return CR{*(const uint4 *)(G + 16u * b), *(const uint2 *)q, *(const uint2 *)(q + 16u),
                  *(const uint32_t *)w, *(const uint32_t *)(w + 8u)};
    }
    __device__ static void decode_rp(const CR &c, uint32_t jb, uint32_t kk, uint32_t kq, uint4 (&bq)[NB])
    {
        // code 8 kq + e: qh byte 16 w + 4 t' + bb with w = kq / 2, t' =
        // 2 (kq & 1) + e / 4, bb = e % 4, so its bit j sits at 8 (e % 4) + s
        // (+ 2 for e >= 4), s = 4 (kq & 1) + (j & 1)
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t w = kk < 2u ? c.w0 : c.w1;
        const uint32_t sh = 4u * (kk & 1u), s = 4u * (kq & 1u) + (kk & 1u);
        const uint32_t c0 = ((v.x >> sh) & 0x0F0F0F0Fu) | (((w >> s) & 0x01010101u) << 4);
        const uint32_t c1 = ((v.y >> sh) & 0x0F0F0F0Fu) | (((w >> (s + 2u)) & 0x01010101u) << 4);
        uint32_t sc4, m4;
        k4sm4(jb, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b(c0, c1, sc4, kk);
    }
    // phase chunks (as Q4_K): pairs ph and 2 + ph
    __device__ static C load_ph(const uint8_t *blk, uint32_t ph, uint32_t kq)
    {
        const uint8_t *q = blk + 48u + 32u * ph + 8u * kq;
        return C{*(const uint4 *)blk, *(const uint2 *)q, *(const uint2 *)(q + 64u),
                 *(const uint2 *)(blk + 16u + 8u * kq)};
    }
    __device__ static void decode_ph(const C &c, uint32_t ph, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t sh = 4u * (kk & 1u), j = 2u * ph + (kk & 1u) + 4u * (kk >> 1);
        const uint32_t c0 = ((v.x >> sh) & 0x0F0F0F0Fu) | (((c.qh.x >> j) & 0x01010101u) << 4);
        const uint32_t c1 = ((v.y >> sh) & 0x0F0F0F0Fu) | (((c.qh.y >> j) & 0x01010101u) << 4);
        uint32_t sc4, m4;
        k4sm_ph(ph, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b(c0, c1, sc4, kk);
    }
    __device__ static CR load_rp_ph(const uint8_t *G, uint32_t b, uint32_t ph, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = 4u * b + ph, H = 4u * ni;
        const uint8_t *q = G + H + (size_t)(((kq >> 1) * ni + it) << 4) + 8u * (kq & 1u);
        const uint8_t *w = G + H + 32u * ni + 8u * it + 4u * (kq >> 1);
        return CR{*(const uint4 *)(G + 16u * b), *(const uint2 *)q, *(const uint2 *)(q + 32u),
                  *(const uint32_t *)w, *(const uint32_t *)(w + 16u)};
    }
    __device__ static void decode_ph(const CR &c, uint32_t ph, uint32_t kk, uint32_t kq, uint4 (&bq)[NB])
    {
        const uint2 v = kk < 2u ? c.v0 : c.v1;
        const uint32_t w = kk < 2u ? c.w0 : c.w1;
        const uint32_t sh = 4u * (kk & 1u), s = 4u * (kq & 1u) + (kk & 1u);
        const uint32_t c0 = ((v.x >> sh) & 0x0F0F0F0Fu) | (((w >> s) & 0x01010101u) << 4);
        const uint32_t c1 = ((v.y >> sh) & 0x0F0F0F0Fu) | (((w >> (s + 2u)) & 0x01010101u) << 4);
        uint32_t sc4, m4;
        k4sm_ph(ph, c.h.y, c.h.z, c.h.w, sc4, m4);
        bq[0] = kquant_b(c0, c1, sc4, kk);
    }
    template <class X> __device__ static uint2 minb_ph(const X &c, uint32_t ph, uint32_t kq, float &dmin)
    {
        uint32_t sc4, m4;
        k4sm_ph(ph, c.h.y, c.h.z, c.h.w, sc4, m4);
        dmin = h2f(c.h.x >> 16);
        return kquant_minb(m4, kq);
    }
    __device__ static float dscale(const C &c, uint32_t) { return h2f(c.h.x); }
    __device__ static float dscale(const CR &c, uint32_t) { return h2f(c.h.x); }
    template <class X> __device__ static uint2 minb(const X &c, uint32_t jb, uint32_t kq, float &dmin)
    {
        uint32_t sc4, m4;
        k4sm4(jb, c.h.y, c.h.z, c.h.w, sc4, m4);
        dmin = h2f(c.h.x >> 16);
        return kquant_minb(m4, kq);
    }
};

// Q6_K (quant.rs:265-292): 210-byte blocks (2-byte aligned), halves n of 128
// elements; within a half, sub-block k4 (32 elements, l = 0..31) takes the
// low (k4 < 2) or high nibbles of ql[64 n + 32 (k4 & 1) + l], bits 2 k4 of
// qh[32 n + l], and scale sc[8 n + l/16 + 2 k4]; the value is
// d sc (q - 32).  A chunk is one half (n = jb / 4).  Reads stay inside the
// block but for the dwords holding d and the last scales, which can end up
// to 3 bytes past the last block (inside the buffer's tail pad).
template <> struct PfH<T_Q6_K> {
    static constexpr int NB = 2;
    static constexpr bool MIN = false;
    static constexpr uint32_t BB = 210;
    struct C {
        uint32_t l0[3], l1[3], qh[3], s[3], d, sb;
    };
    __device__ static C load(const uint8_t *blk, uint32_t jb, uint32_t kq)
    {
        const uint32_t n = jb >> 2;
        const uint32_t *p0 = adown(blk + 64u * n + 8u * kq), *p1 = adown(blk + 64u * n + 32u + 8u * kq);
        const uint32_t *ph = adown(blk + 128u + 32u * n + 8u * kq), *ps = adown(blk + 192u + 8u * n + (kq >> 1));
        C c;
#pragma unroll
        for (int i = 0; i < 3; i++) {
            c.l0[i] = p0[i];
            c.l1[i] = p1[i];
            c.qh[i] = ph[i];
            c.s[i] = ps[i];
        }
        c.d = *adown(blk + 208u);
        c.sb = (uint32_t)((uintptr_t)blk & 3u);
        return c;
    }
    __device__ static void decode(const C &c, uint32_t, uint32_t kk, uint32_t kq, uint4 (&bq)[NB])
    {
        // the block starts at byte sb = 0 or 2 of a dword: ql and qh at
        // offsets 0 mod 4 from it; the scale window at sb + kq/2
        const uint32_t sb = c.sb, sl = (kk >> 1) * 4u, shh = 2u * kk;
        const uint32_t *L = (kk & 1u) ? c.l1 : c.l0;
        const uint32_t L0 = abyte(L[1], L[0], sb), L1 = abyte(L[2], L[1], sb);
        const uint32_t H0 = abyte(c.qh[1], c.qh[0], sb), H1 = abyte(c.qh[2], c.qh[1], sb);
        const uint32_t c0 = ((L0 >> sl) & 0x0F0F0F0Fu) | (((H0 >> shh) & 0x03030303u) << 4);
        const uint32_t c1 = ((L1 >> sl) & 0x0F0F0F0Fu) | (((H1 >> shh) & 0x03030303u) << 4);
        const uint32_t so = (sb + (kq >> 1)) & 3u;
        const uint32_t W = kk < 2u ? abyte(c.s[1], c.s[0], so) : abyte(c.s[2], c.s[1], so);
        const int sc = (int)(int8_t)((W >> (16u * (kk & 1u))) & 0xFFu);     // sc[8n + kq/2 + 2 kk]
        q6_b(c0, c1, sc, bq[0], bq[1]);
    }
    __device__ static float dscale(const C &c, uint32_t) { return h2f(c.d >> (8u * c.sb)); }
    // repack_k's row group: item it = block it/4, half n = (it/2) & 1,
    // i = it & 1 -- l in 16 i .. 16 i + 15 of the half; ql[64n+16i..+16] at
    // 16 it, ql[64n+32+16i..+16] at 16 (ni + it), qh[32n+16i..+16] at
    // 16 (2 ni + it), sc[8n+i+2k] at 48 ni + 4 it + k, d at 52 ni + 2 b
    struct CR {
        uint2 la, lb, qh;
        uint32_t sc, d;
    };
    __device__ static CR load_rp(const uint8_t *G, uint32_t b, uint32_t jb, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = 4u * b + 2u * (jb >> 2) + (kq >> 1), o = 8u * (kq & 1u);
        return CR{*(const uint2 *)(G + 16u * it + o), *(const uint2 *)(G + 16u * (ni + it) + o),
                  *(const uint2 *)(G + 16u * (2u * ni + it) + o), *(const uint32_t *)(G + 48u * ni + 4u * it),
                  (uint32_t)*(const uint16_t *)(G + 52u * ni + 2u * b)};
    }
    __device__ static void decode_rp(const CR &c, uint32_t, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        const uint2 L = (kk & 1u) ? c.lb : c.la;
        const uint32_t sl = (kk >> 1) * 4u, shh = 2u * kk;
        const uint32_t c0 = ((L.x >> sl) & 0x0F0F0F0Fu) | (((c.qh.x >> shh) & 0x03030303u) << 4);
        const uint32_t c1 = ((L.y >> sl) & 0x0F0F0F0Fu) | (((c.qh.y >> shh) & 0x03030303u) << 4);
        q6_b(c0, c1, (int)(int8_t)((c.sc >> (8u * kk)) & 0xFFu), bq[0], bq[1]);
    }
    __device__ static float dscale(const CR &c, uint32_t) { return h2f(c.d); }
    template <class X> __device__ static uint2 minb(const X &, uint32_t, uint32_t, float &dmin)
    {
        dmin = 0.0f;
        return make_uint2(0u, 0u);
    }
};

// Q8_0 (quant.rs:106-113): one 34-byte block (2-byte aligned) per sub-block,
// value d q; a chunk is 4 blocks.
template <> struct PfH<T_Q8_0> {
    static constexpr int NB = 1;
    static constexpr bool MIN = false;
    static constexpr uint32_t BB = 34;
    struct C {
        uint32_t q[4][3], d[4], sb;
    };
    __device__ static C load(const uint8_t *blk, uint32_t, uint32_t kq)
    {
        C c;
#pragma unroll
        for (uint32_t b = 0; b < 4u; b++) {
            const uint32_t *pq = adown(blk + 34u * b + 2u + 8u * kq);
            c.q[b][0] = pq[0];
            c.q[b][1] = pq[1];
            c.q[b][2] = pq[2];
            c.d[b] = *adown(blk + 34u * b);
        }
        c.sb = (uint32_t)((uintptr_t)blk & 3u);
        return c;
    }
    __device__ static void decode(const C &c, uint32_t, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        // block kk starts at byte (sb + 2 kk) & 3 of a dword, its codes
        // (block + 2 + 8 kq) 2 bytes later
        const uint32_t sq = (c.sb + 2u * kk + 2u) & 3u;
        bq[0] = q8_b(abyte(c.q[kk][1], c.q[kk][0], sq), abyte(c.q[kk][2], c.q[kk][1], sq));
    }
    __device__ static float dscale(const C &c, uint32_t kk) { return h2f(c.d[kk] >> (8u * ((c.sb + 2u * kk) & 3u))); }
    // repack_k's row group: item it = blocks 2 it, 2 it + 1; piece k'
    // (codes 16 k' .. +16) at (k' ni + it) 16, the two d halves at
    // 64 ni + 4 it
    struct CR {
        uint2 q[4];
        uint32_t d0, d1;
    };
    __device__ static CR load_rp(const uint8_t *G, uint32_t b, uint32_t, uint32_t kq, uint32_t ni)
    {
        CR c;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const uint32_t bb = b + i, kp = 2u * (bb & 1u) + (kq >> 1);
            c.q[i] = *(const uint2 *)(G + (size_t)((kp * ni + (bb >> 1)) << 4) + 8u * (kq & 1u));
        }
        c.d0 = *(const uint32_t *)(G + 64u * ni + 4u * (b >> 1));
        c.d1 = *(const uint32_t *)(G + 64u * ni + 4u * (b >> 1) + 4u);
        return c;
    }
    __device__ static void decode_rp(const CR &c, uint32_t, uint32_t kk, uint32_t, uint4 (&bq)[NB])
    {
        bq[0] = q8_b(c.q[kk].x, c.q[kk].y);
    }
    __device__ static float dscale(const CR &c, uint32_t kk) { return h2f((kk < 2u ? c.d0 : c.d1) >> (16u * (kk & 1u))); }
    template <class X> __device__ static uint2 minb(const X &, uint32_t, uint32_t, float &dmin)
    {
        dmin = 0.0f;
        return make_uint2(0u, 0u);
    }
};

#ifndef QG_PF_R
#define QG_PF_R 2
#endif
#ifndef QG_PF_WAVES
#define QG_PF_WAVES 4
#endif
#ifndef QG_PF_WG_TARGET
#define QG_PF_WG_TARGET 1024
#endif
#ifndef QG_PF_FILL
#define QG_PF_FILL 256
#endif
constexpr uint32_t kPfKC = 4;                                // sub-blocks per staged chunk
constexpr uint32_t kPfSliceMax = 8;                          // K-split slices per GEMM at most
constexpr uint32_t kPfR = QG_PF_R;                           // 16-row tiles per wave
constexpr uint32_t kPfWaves = QG_PF_WAVES;                   // waves per workgroup
constexpr uint32_t kPfRows = 16u * kPfR * kPfWaves;          // rows per workgroup tile
constexpr uint32_t kPfBufX = kPfKC * 2u * 64u * 64u;         // bytes of x pieces per buffer
constexpr uint32_t kPfBufS = kPfBufX + kPfKC * 256u;         // ... and of the sums, then the group scales
constexpr uint32_t kPfBuf = kPfBufS + 256u;
constexpr uint32_t kPfLds = 2u * kPfBuf;                     // two buffers

// 16 bytes per lane from global memory straight into LDS at byte m0 + 16 lane
// (global_load_lds_dwordx4, issued from asm: the compiler does not track it,
// the waits for it are explicit; lds_addr is an operand bound to M0, which
// the compiler writes itself)
__device__ __forceinline__ void pf_dma16(const void *gp, uint32_t lds_addr)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "{m0}"(lds_addr) : "memory");
}

// 4 bytes per lane, to LDS at byte m0 + 4 lane (global_load_lds_dword)
__device__ __forceinline__ void pf_dma4(const void *gp, uint32_t lds_addr)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gp), "{m0}"(lds_addr) : "memory");
}

// The registers of x are (re)defined here: an empty asm statement that reads
// and writes them keeps its place among the other asm statements, so no
// computation on x moves above it (above a wait or barrier just before).
template <class X> __device__ __forceinline__ void pf_pin(X &x)
{
    static_assert(sizeof(X) % 4 == 0, "whole dwords");
    uint32_t w[sizeof(X) / 4];
    __builtin_memcpy(w, &x, sizeof(X));
#pragma unroll
    for (uint32_t i = 0; i < sizeof(X) / 4; i++) asm volatile("" : "+v"(w[i]));
    __builtin_memcpy(&x, w, sizeof(X));
}

// slot position of token t's slots in its 64-byte LDS row: the 16-byte
// reads of tokens t..t+7 (t % 8 == 0) at one slot cover 8 distinct 16-byte
// bank groups mod 128 bytes, those of t..t+15 16 distinct groups mod 256
__device__ __forceinline__ uint32_t pf_swz(uint32_t t) { return ((t >> 1) ^ (t >> 3)) & 3u; }

// The x pieces are stored chunk by chunk (kPfKC sub-blocks of all
// kPfMaxTokens token slots) as the image of an LDS buffer: 1 KB block
// u = (kk * 2 + c) * 4 + g holds piece c of sub-block kk for tokens
// 16 g .. 16 g + 15, token t's 64 bytes as four 16-byte slots, slot s
// (elements 8 s .. 8 s + 7) at position s ^ pf_swz(t) so that the A-operand
// reads of 8 or 16 consecutive tokens at one slot hit distinct banks.  Byte
// offset of (chunk, u, t % 16, position):
__device__ __forceinline__ size_t pf_xoff(uint32_t chunk, uint32_t u, uint32_t t16, uint32_t pos)
{
    return (size_t)chunk * (kPfKC * 8u * 1024u) + u * 1024u + t16 * 64u + pos * 16u;
}

// Issue part `part` (of kPfKC) of the copies of chunk kc into the buffer at
// LDS byte address b0: x blocks u = 8 part .. 8 part + 7 (each one
// contiguous KB), with part 0 the chunk's 4 x 64 sums, with part 1 the 64
// token scales 2^-e_g of its 256-element group (scl: the scales of group 0).
__device__ __forceinline__ void pf_stage(const uint8_t *__restrict__ xp, const float *__restrict__ rec,
                                         const float *__restrict__ scl, uint32_t kc, uint32_t b0, uint32_t wave,
                                         uint32_t lane, uint32_t part)
{
#pragma unroll
    for (uint32_t v = 0; v < 8u / kPfWaves; v++) {
        const uint32_t u = 8u * part + v * kPfWaves + wave;
        pf_dma16(xp + pf_xoff(kc / kPfKC, u, 0, 0) + 16u * lane, b0 + u * 1024u);
    }
    if (part == 0 && wave == 0) pf_dma16(rec + (size_t)kc * 64u + 4u * lane, b0 + kPfBufX);
    if (part == 1 && wave == 0) pf_dma4(scl + (size_t)(kc / 8u) * 64u + lane, b0 + kPfBufS);
}

// The same for a phase chunk (block b, half ph): its sub-blocks kk' = 0, 1
// are sub-blocks 2 ph, 2 ph + 1 of the block's first chunk image (2 b), kk'
// = 2, 3 those of the second (2 b + 1); the buffer gets the layout of a
// plain chunk.
__device__ __forceinline__ void pf_stage_ph(const uint8_t *__restrict__ xp, const float *__restrict__ rec,
                                            const float *__restrict__ scl, uint32_t b, uint32_t ph, uint32_t b0,
                                            uint32_t wave, uint32_t lane, uint32_t part)
{
    const uint32_t src_kk = 2u * ph + (part & 1u), chunk = 2u * b + (part >> 1);
#pragma unroll
    for (uint32_t v = 0; v < 8u / kPfWaves; v++) {
        const uint32_t u = 8u * part + v * kPfWaves + wave;          // (part * 2 + c) * 4 + g
        pf_dma16(xp + pf_xoff(chunk, ((src_kk * 2u + ((u >> 2) & 1u)) << 2) + (u & 3u), 0, 0) + 16u * lane,
                 b0 + u * 1024u);
    }
    if (part == 0 && wave == 0) {
        const uint32_t kk = lane >> 4, sub = 8u * b + 4u * (kk >> 1) + 2u * ph + (kk & 1u);
        pf_dma16(rec + (size_t)sub * 64u + 4u * (lane & 15u), b0 + kPfBufX);
    }
    if (part == 1 && wave == 0) pf_dma4(scl + (size_t)b * 64u + lane, b0 + kPfBufS);
}

// One workgroup's share of a grouped GEMM: rows row0 .. row0 + 16 kPfR
// (waves past the matrix still stage), K slice k0 .. k1 (multiples of
// kPfKC), all the chunk's tokens.  x: the chunk images at xp (pf_xoff); per
// sub-block k the sums rec[64 k + t]; 2^-e_g of token t's 256-element group
// g at rec[64 nseg + 64 g + t].  Chunks of kPfKC sub-blocks (with their
// sums and their group's 2^-e_g) are copied into two LDS buffers in turn,
// the next chunk's copy and weight loads in flight while this one is
// computed.  Every chunk lies inside one block of each row
// (cols % 128 == 0 and slices of whole chunks: a row starts at a multiple of
// 4 sub-blocks).  D[4 kq + i][c16] of an MFMA is token 16 tt + 4 kq + i of
// row r0 + c16.  LAY, the weight layout: 0 GGUF, rows straddling blocks; 1
// GGUF, every row starts a block (nseg % 8 == 0, or Q8_0); 2 repacked
// (repack_k), one row per row group; 3 repacked, gg rows per group of gb
// bytes (ni items).  In layouts 1 and 2 every row is at the same sub-block
// of its block, and the block ends are the same for the whole wave.
template <uint32_t T, int LAY>
__device__ __forceinline__ void pf_gemm_rows(const uint8_t *__restrict__ w, uint32_t rows, uint32_t row0,
                                             uint32_t nseg, uint32_t k0, uint32_t k1,
                                             const uint16_t *__restrict__ xp, const float *__restrict__ rec,
                                             uint32_t ntok, uint32_t n, uint8_t *lds, float *__restrict__ y,
                                             uint32_t ldy, uint32_t gg, uint64_t gb, uint32_t ni)
{
    using P = PfH<T>;
    constexpr int R = (int)kPfR;
    constexpr bool RPL = LAY >= 2, AL = LAY == 1 || LAY == 2, Q8 = T == T_Q8_0;
    // phase order (Q4_K, Q5_K with whole-block rows): chunk slot c of a
    // group of nbg <= 4 blocks is half c / nbg of block c % nbg -- the four
    // first halves, then the four second halves -- so that a row's repacked
    // pieces in use at a time lie in 2 of the layout's 4 code regions (the
    // lines of the other two would not stay in L2 until their next use)
    constexpr bool PH = (T == T_Q4_K || T == T_Q5_K) && AL;
    using Ck = std::conditional_t<RPL, typename P::CR, typename P::C>;
    const uint8_t *xb8 = (const uint8_t *)xp;
    const float *scl = rec + (size_t)nseg * 64u;                     // 2^-e_g of group 0
    const uint32_t lane = threadIdx.x & 63u, kq = lane >> 4, c16 = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
    const bool active = row0 < rows;                                  // wave-uniform
    const uint32_t swz = kq ^ pf_swz(c16);                           // this lane's slot position
    // per row tile: the row's first sub-block (GGUF: flat index; repacked:
    // within its row group) and its base (GGUF layout 1: its first block;
    // repacked: its group)
    uint64_t fb[R];
    const uint8_t *rb[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const uint32_t r = min(row0 + 16u * i + c16, rows - 1u);
        if constexpr (RPL) {
            fb[i] = LAY == 2 ? 0u : (uint64_t)(r % gg) * nseg;
            rb[i] = w + (size_t)(LAY == 2 ? r : r / gg) * gb;
        } else {
            fb[i] = (uint64_t)r * nseg;
            rb[i] = w + (Q8 ? fb[i] : fb[i] / 8u) * P::BB;
        }
    }
    // block and half of the phase chunk at sub-block kc
    auto slot = [&](uint32_t kc, uint32_t &b, uint32_t &ph) {
        const uint32_t c = kc / kPfKC, g4 = c >> 3, nbg = min(4u, nseg / 8u - 4u * g4), s8 = c & 7u;
        ph = s8 >= nbg ? 1u : 0u;
        b = 4u * g4 + s8 - ph * nbg;
    };
    // chunk kc of row tile i (kc < k1: clamped by the caller)
    auto cload = [&](int i, uint32_t kc) -> Ck {
        if constexpr (PH) {
            uint32_t b, ph;
            slot(kc, b, ph);
            if constexpr (RPL) return P::load_rp_ph(rb[i], b, ph, kq, ni);
            else return P::load_ph(rb[i] + (size_t)b * P::BB, ph, kq);
        }
        const uint64_t f = fb[i] + kc;
        const uint32_t jb = Q8 ? 0u : (uint32_t)(f & 7u);
        if constexpr (RPL) {
            return P::load_rp(rb[i], (uint32_t)(Q8 ? f : f >> 3), jb, kq, ni);
        } else if constexpr (LAY == 1) {
            return P::load(rb[i] + (size_t)(Q8 ? kc : kc >> 3) * P::BB, jb, kq);
        } else {
            return P::load(w + (Q8 ? f : f >> 3) * P::BB, jb, kq);
        }
    };
    v4f acc[R][4], D[R][4];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int tt = 0; tt < 4; tt++) acc[i][tt] = D[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
    if (k0 < k1) {
        // The operands of chunk kc (B, scales) are decoded from its weight
        // registers during chunk kc - kPfKC, between that chunk's MFMAs; the
        // weights of chunk kc + kPfKC are loaded at the start of chunk kc.
        // The waits are compiler-visible (s_waitcnt builtin), so no use of a
        // loaded register waits for the copies issued after it.
        struct Ops {
            uint4 bq[kPfKC][R][P::NB];
            float dsc[R][Q8 ? kPfKC : 1];
            uint2 bm[R];                                              // min terms: B operand, dmin
            float dmn[R];
            uint32_t jb[R];
        };
        // sub-block kk's B operands of the chunk kc held in cw; its scales
        auto decode_kk = [&](const Ck (&cw)[R], uint32_t kc, uint32_t kk, Ops &o) {
            if constexpr (PH) {
                uint32_t b, ph;
                slot(kc, b, ph);
#pragma unroll
                for (int i = 0; i < R; i++) P::decode_ph(cw[i], ph, kk, kq, o.bq[kk][i]);
                return;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const uint32_t jb = Q8 ? 0u : AL ? (kc & 7u) : (uint32_t)((fb[i] + kc) & 7u);
                if constexpr (RPL) P::decode_rp(cw[i], jb, kk, kq, o.bq[kk][i]);
                else P::decode(cw[i], jb, kk, kq, o.bq[kk][i]);
            }
        };
        auto decode_sc = [&](const Ck (&cw)[R], uint32_t kc, Ops &o) {
            if constexpr (PH) {
                uint32_t b, ph;
                slot(kc, b, ph);
#pragma unroll
                for (int i = 0; i < R; i++) {
                    o.jb[i] = 4u;                                     // every chunk ends its D
                    o.dsc[i][0] = P::dscale(cw[i], 0u);
                    if constexpr (P::MIN) o.bm[i] = P::minb_ph(cw[i], ph, kq, o.dmn[i]);
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                o.jb[i] = Q8 ? 0u : AL ? (kc & 7u) : (uint32_t)((fb[i] + kc) & 7u);
#pragma unroll
                for (uint32_t kk = 0; kk < (Q8 ? kPfKC : 1u); kk++) o.dsc[i][kk] = P::dscale(cw[i], kk);
                o.bm[i] = P::minb(cw[i], o.jb[i], kq, o.dmn[i]);
            }
        };
        auto stage = [&](uint32_t kc, uint32_t b0, uint32_t part) {
            if constexpr (PH) {
                uint32_t b, ph;
                slot(kc, b, ph);
                pf_stage_ph(xb8, rec, scl, b, ph, b0, wave, lane, part);
            } else {
                pf_stage(xb8, rec, scl, kc, b0, wave, lane, part);
            }
        };
#pragma unroll
        for (uint32_t part = 0; part < kPfKC; part++) stage(k0, lds0, part);
        Ck cw[R];
#pragma unroll
        for (int i = 0; i < R; i++) cw[i] = cload(i, k0);
        __builtin_amdgcn_s_waitcnt(0x0F70);                           // vmcnt(0)
        Ops op;
#pragma unroll
        for (uint32_t kk = 0; kk < kPfKC; kk++) decode_kk(cw, k0, kk, op);
        decode_sc(cw, k0, op);
#pragma unroll
        for (int i = 0; i < R; i++) cw[i] = cload(i, min(k0 + kPfKC, k1 - kPfKC));
        uint32_t buf = 0;
        for (uint32_t kc = k0; kc < k1; kc += kPfKC, buf ^= 1u) {
            __builtin_amdgcn_s_waitcnt(0x0F70);                       // this wave's copies of chunk kc, the weights of the next
            __syncthreads();                                          // everyone's copies; the other buffer is free
#pragma unroll
            for (int i = 0; i < R; i++) pf_pin(cw[i]);                // decoded below, not above the wait
            // the next chunk's copies and the weights of the one after, spread
            // over the sub-blocks below (the copies of the last chunk repeat it
            // into the buffer no one reads any more)
            const uint32_t kx = min(kc + kPfKC, k1 - kPfKC), kw = min(kc + 2u * kPfKC, k1 - kPfKC);
            const uint32_t bnext = lds0 + (buf ^ 1u) * kPfBuf;
            Ck cw2[R];
            Ops on;
            const uint32_t kn = min(kc + kPfKC, k1 - kPfKC);
            decode_sc(cw, kn, on);
            {   // (waves past the matrix compute too -- clamped rows, never stored -- so that
                // this phase stays one block of straight-line code)
                const uint8_t *xb = lds + buf * kPfBuf;
                // 2^-e_g of the chunk's 256-element group for the lane's 16
                // tokens 16 tt + 4 kq + e
                float sg[4][4];
                {
                    const float4 *sp = (const float4 *)(xb + kPfBufS);
#pragma unroll
                    for (uint32_t tt = 0; tt < 4; tt++) {
                        const float4 q = sp[4u * tt + kq];
                        sg[tt][0] = q.x; sg[tt][1] = q.y; sg[tt][2] = q.z; sg[tt][3] = q.w;
                    }
                }
                // min terms: A = the sums of the chunk's sub-blocks 2 (kq & 1),
                // 2 (kq & 1) + 1 as f16 pieces (K slots 2 kk + piece; zero for kq >= 2)
                v4f Dm[R][4];
                if constexpr (P::MIN) {
                    const uint32_t *su = (const uint32_t *)(xb + kPfBufX) + 2u * (kq & 1u) * 64u + c16;
#pragma unroll
                    for (uint32_t tt = 0; tt < 4; tt++) {
                        const uint32_t s0 = su[16u * tt], s1 = su[64u + 16u * tt];
                        const h4 a = __builtin_bit_cast(h4, kq < 2u ? make_uint2(s0, s1) : make_uint2(0u, 0u));
#pragma unroll
                        for (int i = 0; i < R; i++)
                            Dm[i][tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, __builtin_bit_cast(h4, op.bm[i]),
                                                                               v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    }
                }
#pragma unroll
                for (uint32_t kk = 0; kk < kPfKC; kk++) {
                    stage(kx, bnext, kk);
#pragma unroll
                    for (int i = 0; i < R; i++)
                        if ((uint32_t)i % kPfKC == kk) cw2[i] = cload(i, kw);
                    // the sub-block's A operands (every token tile, both
                    // pieces), then its MFMAs piece by piece, so that the
                    // MFMAs on one accumulator are 4 R NB issues apart
                    h8 av[2][4];
#pragma unroll
                    for (uint32_t tt = 0; tt < 4; tt++) {
                        const uint8_t *xa = xb + (((kk * 2u * 64u + 16u * tt + c16) * 4u + swz) << 4);
                        av[0][tt] = *(const h8 *)xa;
                        av[1][tt] = *(const h8 *)(xa + 64u * 64u);
                    }
#pragma unroll
                    for (int pc = 0; pc < 2; pc++)
#pragma unroll
                        for (uint32_t tt = 0; tt < 4; tt++)
#pragma unroll
                            for (int i = 0; i < R; i++)
#pragma unroll
                                for (int h = 0; h < P::NB; h++)
                                    D[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                        av[pc][tt], __builtin_bit_cast(h8, op.bq[kk][i][h]), D[i][tt], 0, 0, 0);
                    decode_kk(cw, kn, kk, on);                        // the next chunk's, between the MFMAs
                    pf_pin(on.bq[kk]);                                // (here, not sunk to the loop's end)
                    if constexpr (Q8) {                               // a scale per sub-block
#pragma unroll
                        for (int i = 0; i < R; i++)
#pragma unroll
                            for (int tt = 0; tt < 4; tt++) {
#pragma unroll
                                for (int e = 0; e < 4; e++)
                                    acc[i][tt][e] = __builtin_fmaf(op.dsc[i][kk] * sg[tt][e], D[i][tt][e], acc[i][tt][e]);
                                D[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
                            }
                    }
                }
                if constexpr (PH) {
                    // every chunk ends its D: d D and the chunk's -dmin m S
                    // terms (the v_mfma_f32_16x16x16_f16 products taken before
                    // this chunk's main MFMAs), times 2^-e_g
#pragma unroll
                    for (int i = 0; i < R; i++)
#pragma unroll
                        for (uint32_t tt = 0; tt < 4; tt++) {
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                const float u = __builtin_fmaf(op.dsc[i][0], D[i][tt][e], -op.dmn[i] * Dm[i][tt][e]);
                                acc[i][tt][e] = __builtin_fmaf(sg[tt][e], u, acc[i][tt][e]);
                            }
                            D[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
                        }
                } else {
                    if constexpr (P::MIN) {
                        // the chunk's -dmin m S terms, from the v_mfma_f32_16x16x16_f16
                        // products taken before this chunk's main MFMAs
#pragma unroll
                        for (int i = 0; i < R; i++)
#pragma unroll
                            for (uint32_t tt = 0; tt < 4; tt++)
#pragma unroll
                                for (int e = 0; e < 4; e++)
                                    acc[i][tt][e] =
                                        __builtin_fmaf(-op.dmn[i] * sg[tt][e], Dm[i][tt][e], acc[i][tt][e]);
                    }
                    if constexpr (!Q8) {
                        if constexpr (AL) {
                            // a row's block ends with this chunk (jb = 4), or the
                            // slice does; the block's two chunks share a group
                            if (op.jb[0] == 4u || kc + kPfKC >= k1) {
#pragma unroll
                                for (int i = 0; i < R; i++)
#pragma unroll
                                    for (int tt = 0; tt < 4; tt++) {
#pragma unroll
                                        for (int e = 0; e < 4; e++)
                                            acc[i][tt][e] = __builtin_fmaf(op.dsc[i][0] * sg[tt][e], D[i][tt][e],
                                                                           acc[i][tt][e]);
                                        D[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
                                    }
                            }
                        } else {
                            // rows whose blocks straddle the 256-element groups:
                            // every chunk ends D
#pragma unroll
                            for (int i = 0; i < R; i++)
#pragma unroll
                                for (int tt = 0; tt < 4; tt++) {
#pragma unroll
                                    for (int e = 0; e < 4; e++)
                                        acc[i][tt][e] =
                                            __builtin_fmaf(op.dsc[i][0] * sg[tt][e], D[i][tt][e], acc[i][tt][e]);
                                    D[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
                                }
                        }
                    }
                }
            }
            op = on;
#pragma unroll
            for (int i = 0; i < R; i++) cw[i] = cw2[i];
        }
    }
    if (!active) return;
#pragma unroll
    for (int i = 0; i < R; i++) {
        const uint32_t r = row0 + 16u * i + c16;
        if (r >= rows) continue;
#pragma unroll
        for (uint32_t tt = 0; tt < 4; tt++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t t = 16u * tt + 4u * kq + (uint32_t)e;
                if (t < ntok) __builtin_nontemporal_store(acc[i][tt][e], &y[(size_t)t * ldy + r]);
            }
        }
    }
}

// One matrix of a grouped GEMM launch: its rows, workgroup tiles of
// kPfRows rows, and where row 0 of token 0 of slice 0 of its output goes.
struct PfJob {
    const uint8_t *w;
    float *y;
    uint32_t type, rows, tiles;
    uint32_t g, ni;        // repacked layout: rows per row group, items per group
    uint64_t gb;           // ... and bytes per group
};
struct PfJobs {
    PfJob j0, j1, j2;
    uint32_t n;
};

// Grouped, K-split GEMM over matrices of type T: blockIdx.x runs over the row
// tiles of jobs j0, j1, j2 in turn, blockIdx.y over the slices of sps
// sub-blocks (a multiple of kPfKC); slice s of a job writes its partial
// products to y + s * sstride (the consumer sums the slices in order
// s = 0, 1, ...).  kPfWaves waves of 16 kPfR rows per workgroup.
template <uint32_t T, int LAY>
__global__ void __launch_bounds__(64 * kPfWaves) pf_gemm_k(PfJobs jobs, uint32_t nseg, uint32_t sps,
                                                 const uint16_t *__restrict__ xp, const float *__restrict__ rec,
                                                 uint32_t ntok, uint32_t n, uint32_t ldy, uint64_t sstride)
{
    extern __shared__ float4 pf_lds4[];
    uint32_t tile = blockIdx.x;
    PfJob J = jobs.j0;
    if (tile >= J.tiles) {
        tile -= J.tiles;
        J = jobs.j1;
        if (tile >= J.tiles) {
            tile -= J.tiles;
            J = jobs.j2;
        }
    }
    const uint32_t row0 = tile * kPfRows + (threadIdx.x >> 6) * (16u * kPfR);
    const uint32_t k0 = min(nseg, blockIdx.y * sps), k1 = min(nseg, k0 + sps);
    pf_gemm_rows<T, LAY>(J.w, J.rows, row0, nseg, k0, k1, xp, rec, ntok, n, (uint8_t *)pf_lds4,
                         J.y + (size_t)blockIdx.y * sstride, ldy, J.g, J.gb, J.ni);
}

// ---------------------------------------------------------------- planes
//
// The input vector x of token blockIdx.y -- mode 0: x = a; mode 1: x = (a +
// b) * nw, the RMSNorm's numerator, with a + b stored to sum_out when given
// and the partial sums of (a + b)^2 per 256-element group in ss_out; mode 2:
// x = silu(a r) * (b r), r = 1 / rms of the norm whose partial sums are at
// `pre` (r = 1 without) -- as the two f16 pieces of xs = x 2^e_g, every
// 256-element group g with its own e_g (in the GEMM's chunk images,
// pf_xoff), the sums of xs per 32-element segment (two f16 pieces), and
// 2^-e_g.  A GEMM over such an x gives y = W x' with x' = (a + b) * nw in mode
// 1: the consumer of y multiplies it by 1 / rms (math.rs:237-257: the norm's
// factor is common to the row, so it moves past the product), from the
// partial sums (pf_inv_rms).  a and b may be the K-split slices of a GEMM
// (na, nb <= kPfMaxSlices slices sstride floats apart, summed in slice
// order).  One launch of pf_planes_blk(n) workgroups per token over 8-element
// pieces: 32 threads hold a 256-element group and find its maximum through
// lane shuffles, 4 threads a 32-element segment.  A group with a non-finite
// x gets 2^-e_g = NaN (every output of its token NaN).  sum_out must not alias
// a or b.
constexpr uint32_t kPfMaxSlices = 16;
constexpr uint32_t kPfPlanesT = 256;                         // threads per workgroup

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

// p[0] + p[sstride] + ... over ns <= kPfMaxSlices slices, all loads issued first
__device__ __forceinline__ float sum_slices(const float *p, uint32_t ns, uint64_t sstride)
{
    float u[kPfMaxSlices];
#pragma unroll
    for (uint32_t s = 0; s < kPfMaxSlices; s++)
        if (s < ns) u[s] = p[s * sstride];
    float r = u[0];
#pragma unroll
    for (uint32_t s = 1; s < kPfMaxSlices; s++)
        if (s < ns) r += u[s];
    return r;
}

// elements i .. i + 7 (i % 8 == 0) of the sum of ns slices, all loads issued first
__device__ __forceinline__ void sum8_slices(const float *p, uint32_t ns, uint64_t sstride, float (&v)[8])
{
    float4 u[kPfMaxSlices][2];
#pragma unroll
    for (uint32_t s = 0; s < kPfMaxSlices; s++)
        if (s < ns) {
            u[s][0] = *(const float4 *)(p + s * sstride);
            u[s][1] = *(const float4 *)(p + s * sstride + 4);
        }
    float4 r0 = u[0][0], r1 = u[0][1];
#pragma unroll
    for (uint32_t s = 1; s < kPfMaxSlices; s++)
        if (s < ns) {
            r0.x += u[s][0].x; r0.y += u[s][0].y; r0.z += u[s][0].z; r0.w += u[s][0].w;
            r1.x += u[s][1].x; r1.y += u[s][1].y; r1.z += u[s][1].z; r1.w += u[s][1].w;
        }
    v[0] = r0.x; v[1] = r0.y; v[2] = r0.z; v[3] = r0.w;
    v[4] = r1.x; v[5] = r1.y; v[6] = r1.z; v[7] = r1.w;
}

// x[i] (before the norm) of the piece at e0: a + b (mode 1), silu(a) * b (2), a (0)
__device__ __forceinline__ void pf_input8(const float *at, uint32_t na, const float *bt, uint32_t nb,
                                          uint64_t sstride, uint32_t mode, uint32_t e0, float (&v)[8])
{
    sum8_slices(at + e0, na, sstride, v);
    if (bt) {
        float u[8];
        sum8_slices(bt + e0, nb, sstride, u);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = mode == 2 ? silu1(v[e]) * u[e] : v[e] + u[e];
    }
}

// sum (or maximum) of v over the workgroup, through red[0 .. waves)
template <bool MAX>
__device__ __forceinline__ float pf_block_reduce(float v, float *red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float u = __shfl_xor(v, o, 64);
        v = MAX ? fmaxf(v, u) : v + u;
    }
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (uint32_t i = 1; i < blockDim.x / 64u; i++) r = MAX ? fmaxf(r, red[i]) : r + red[i];
    __syncthreads();
    return r;
}

// workgroups per token for rows of n elements: one 8-element piece per thread
__host__ __device__ constexpr uint32_t pf_planes_blk(uint32_t n) { return (n / 8u + kPfPlanesT - 1u) / kPfPlanesT; }

// 1 / rms of token t from the partial sums of squares of its ng groups
// (math.rs:253-255): lane g of every wave loads groups g, g + 64, ..., the
// wave adds them with a fixed butterfly, and lane 0's sum is taken, so every
// thread gets the same value, run after run.
__device__ __forceinline__ float pf_inv_rms(const float *__restrict__ ss, uint32_t ng, uint32_t t, uint32_t n,
                                            float eps)
{
    const float *p = ss + (size_t)t * ng;
    const uint32_t lane = threadIdx.x & 63u;
    float r = 0.f;
    for (uint32_t g = lane; g < ng; g += 64u) r += p[g];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) r += __shfl_xor(r, o, 64);
    r = __shfl(r, 0, 64);
    return 1.0f / sqrtf(r / (float)n + eps);
}

__global__ void __launch_bounds__(kPfPlanesT) pf_split_k(const float *__restrict__ a, uint32_t na,
                                                         const float *__restrict__ b, uint32_t nb, uint64_t sstride,
                                                         float *__restrict__ sum_out, const float *__restrict__ nw,
                                                         uint32_t n, uint32_t lda, uint32_t mode,
                                                         const float *__restrict__ pre, uint32_t pre_ng,
                                                         uint32_t pre_n, float eps, float *__restrict__ ss_out,
                                                         uint16_t *__restrict__ xp, float *__restrict__ rec)
{
    const uint32_t t = blockIdx.y, j = blockIdx.x * kPfPlanesT + threadIdx.x, ng = (n + 255u) / 256u;
    const bool live = j < n / 8u;
    const uint32_t e0 = live ? 8u * j : 0u;
    float v[8];
    bool bad = false;
    float ss = 0.f;
    {
        const float *at = a + (size_t)t * lda, *bt = b ? b + (size_t)t * lda : nullptr;
        sum8_slices(at + e0, na, sstride, v);
        if (bt) {
            float u[8];
            sum8_slices(bt + e0, nb, sstride, u);
            if (mode == 2) {
                const float r = pre ? pf_inv_rms(pre, pre_ng, t, pre_n, eps) : 1.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = silu1(v[e] * r) * (u[e] * r);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] += u[e];
            }
        }
        if (mode == 1) {
            if (sum_out && live) {
                float *so = sum_out + (size_t)t * lda + e0;
                *(float4 *)so = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(so + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                ss += v[e] * v[e];
                v[e] = v[e] * nw[e0 + e];
            }
        }
    }
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        bad |= !__builtin_isfinite(v[e]);
        m = fmaxf(m, fabsf(v[e]));
    }
    if (!live) {
        m = 0.f;
        ss = 0.f;
        bad = false;
    }
    // the group's maximum, sum of squares and badness over its 32 lanes
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o, 64));
        ss += __shfl_xor(ss, o, 64);
        bad |= __shfl_xor((int)bad, o, 64) != 0;
    }
    // 2^e_g brings the group's largest magnitude into [512, 1024)
    int E = 0;
    (void)frexpf(m, &E);
    const int e = bad ? 0 : m > 0.f ? min(max(10 - E, -126), 126) : 0;
    const float sc = ldexpf(1.0f, e);
    if (live) {
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = v[k] * sc;
        uint32_t wh[4], wl[4];
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const _Float16 h0 = (_Float16)v[k], h1 = (_Float16)v[k + 1];
            const _Float16 l0 = (_Float16)(v[k] - (float)h0), l1 = (_Float16)(v[k + 1] - (float)h1);
            wh[k >> 1] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            wl[k >> 1] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        // piece c of slot j & 3 of sub-block j / 4, in the GEMM's chunk image
        const uint32_t k = j >> 2, t16 = t & 15u;
        uint8_t *p0 = (uint8_t *)xp + pf_xoff(k / kPfKC, (k % kPfKC) * 8u + (t >> 4), t16, (j & 3u) ^ pf_swz(t16));
        *(uint4 *)p0 = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        *(uint4 *)(p0 + 4u * 1024u) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    }
    // per quarter (x0 + x1) + (x2 + x3) ..., per half the two quarters, the segment the two halves
    const float qsum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    const float hsum = qsum + __shfl_xor(qsum, 1, 64);
    const float seg = hsum + __shfl_xor(hsum, 2, 64);
    if (live && (j & 3u) == 0u) {                                     // as two f16 pieces, hi | lo << 16
        const _Float16 sh = (_Float16)seg, sl = (_Float16)(seg - (float)sh);
        ((uint32_t *)rec)[(size_t)(j >> 2) * 64u + t] =
            (uint32_t)__builtin_bit_cast(uint16_t, sh) | ((uint32_t)__builtin_bit_cast(uint16_t, sl) << 16);
    }
    if (live && (j & 31u) == 0u) {
        const uint32_t g = j >> 5;
        rec[(size_t)(n / 32u) * 64u + (size_t)g * 64u + t] = bad ? __builtin_nanf("") : ldexpf(1.0f, -e);
        if (mode == 1) ss_out[(size_t)t * ng + g] = ss;
    }
}

// out[i] = sum over slices s of x[s * sstride + i], i < n
__global__ void __launch_bounds__(256) pf_sum_k(const float *__restrict__ x, uint32_t ns, uint64_t sstride, uint32_t n,
                                                float *__restrict__ out)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = sum_slices(x + i, ns, sstride);
}

// ----------------------------------------------------- attention, post-ops

// Bias add, RoPE and KV append of token t of the chunk (position pos0 + t,
// cache slot slot0 + t); q, k, v of a token are contiguous with stride ldq,
// summed over the ns K-split slices of the QKV GEMM (sstride floats apart);
// the rotated q goes to slice 0.  The expressions of the decode path's
// qkv_post_k.
__global__ void __launch_bounds__(256) pf_qkv_post_k(float *__restrict__ qkv, uint32_t ldq, uint32_t ns,
                                                     uint32_t ns_v, uint64_t sstride, const float *__restrict__ ss,
                                                     uint32_t ss_ng,
                                                     uint32_t ss_n, float eps, const float *__restrict__ bq,
                                                     const float *__restrict__ bk, const float *__restrict__ bv,
                                                     float *__restrict__ kc, float *__restrict__ vc,
                                                     const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                     uint32_t q_dim, uint32_t kv_dim, uint32_t hd, uint32_t pos0,
                                                     uint32_t slot0)
{
    const uint32_t t = blockIdx.y, i0 = 2 * (blockIdx.x * blockDim.x + threadIdx.x), half = hd / 2;
    const uint32_t pos = pos0 + t, slot = slot0 + t;
    float *q = qkv + (size_t)t * ldq, *k = q + q_dim, *v = k + kv_dim;
    // the GEMM took the norm's numerator: its 1 / rms here, before the biases
    const float r = pf_inv_rms(ss, ss_ng, t, ss_n, eps);
    if (i0 < q_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float x0 = sum_slices(q + i0, ns, sstride) * r + bq[i0];
        const float x1 = sum_slices(q + i0 + 1, ns, sstride) * r + bq[i0 + 1];
        q[i0] = x0 * c - x1 * s;
        q[i0 + 1] = x0 * s + x1 * c;
    }
    if (i0 < kv_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float x0 = sum_slices(k + i0, ns, sstride) * r + bk[i0];
        const float x1 = sum_slices(k + i0 + 1, ns, sstride) * r + bk[i0 + 1];
        float *kr = kc + (size_t)slot * kv_dim, *vr = vc + (size_t)slot * kv_dim;
        kr[i0] = x0 * c - x1 * s;
        kr[i0 + 1] = x0 * s + x1 * c;
        vr[i0] = sum_slices(v + i0, ns_v, sstride) * r + bv[i0];
        vr[i0 + 1] = sum_slices(v + i0 + 1, ns_v, sstride) * r + bv[i0 + 1];
    }
}

// Attention of query head blockIdx.x for tokens t0 .. t0 + 15 (t0 = 16
// blockIdx.y) of the chunk, token t over cache slots 0 .. slot0 + t
// (attention.rs:93-121, math.rs:63-70 / 104-118), on the f32 matrix cores
// (v_mfma_f32_16x16x4f32: f32 products and sums).  Positions go in tiles of
// 64 rows of K and V staged in LDS; wave w takes tile positions 16 w .. 16 w
// + 15: S = Q K^T for its 16 positions (hd / 4 MFMAs, Q in registers), then,
// after the tile's running maximum per token is agreed through LDS,
// P = exp(S - M) for them, and O += P V for output columns 64 w' .. (its hd /
// 64 column blocks of 16) over the tile's 64 positions (16 MFMAs per block).
// Each token keeps a running (max, sum) and its output is rescaled when the
// maximum grows, so the result is the softmax over all positions.
// 16x16x4 f32 layout (gfx950): lane l holds A[l % 16][l / 16],
// B[l / 16][l % 16] and D[4 (l / 16) + i][l % 16], i = 0..3.
constexpr uint32_t kPfAttRows = 16, kPfAttTile = 64;
__host__ __device__ constexpr size_t pf_att_lds(uint32_t hd)
{
    // Q [16][hd + 4], K [64][hd + 4], V [64][hd + 16], P [16][64 + 4], the
    // waves' per-token maxima and sums [2][4][16]
    return ((size_t)kPfAttRows * (hd + 4u) + (size_t)kPfAttTile * (hd + 4u) + (size_t)kPfAttTile * (hd + 16u) +
            (size_t)kPfAttRows * (kPfAttTile + 4u) + 2u * 4u * kPfAttRows) * sizeof(float);
}
template <uint32_t HD>
__global__ void __launch_bounds__(256) pf_attention_k(const float *__restrict__ qkv, uint32_t ldq,
                                                      const float *__restrict__ kc, const float *__restrict__ vc,
                                                      float *__restrict__ out, uint32_t kv_dim, uint32_t n_rep,
                                                      float scale, uint32_t slot0, uint32_t ntok)
{
    constexpr uint32_t TP = kPfAttTile, LQ = HD + 4u, LK = HD + 4u, LV = HD + 16u, LP = TP + 4u;
    constexpr uint32_t KS = HD / 4u, NB = HD / 64u;                  // k-steps of S; O column blocks per wave
    static_assert(HD == 64 || HD == 128 || HD == 256, "head_dim 64, 128 or 256");
    typedef float v4f __attribute__((ext_vector_type(4)));
    extern __shared__ float4 att_lds4[];
    float *qs = (float *)att_lds4, *ks = qs + kPfAttRows * LQ, *vs = ks + TP * LK, *ps = vs + TP * LV;
    float *wmax = ps + kPfAttRows * LP, *wsum = wmax + 4u * kPfAttRows;
    const uint32_t h = blockIdx.x, t0 = blockIdx.y * kPfAttRows, kvh = (h / n_rep) * HD;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, w = tid >> 6, c = lane & 15u, g = lane >> 4;
    const uint32_t nrow = min(kPfAttRows, ntok - t0), npos = slot0 + t0 + nrow;     // positions any row sees
    // the 16 tokens' q (rows past the chunk: the last token's, never stored)
    for (uint32_t i = tid; i < kPfAttRows * (HD / 4u); i += 256u) {
        const uint32_t rr = i / (HD / 4u), d4 = i % (HD / 4u);
        const float *q = qkv + (size_t)(t0 + min(rr, nrow - 1u)) * ldq + (size_t)h * HD;
        *(float4 *)(qs + rr * LQ + 4u * d4) = *(const float4 *)(q + 4u * d4);
    }
    __syncthreads();
    // A of S: q[token c][4 k + g], k = 0 .. HD/4 - 1
    float qa[KS];
#pragma unroll
    for (uint32_t k = 0; k < KS; k++) qa[k] = qs[c * LQ + 4u * k + g];
    // this lane's D rows: tokens 4 g + i; their running max and sum
    float m[4], l[4];
    v4f o[NB];
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) { m[i] = -INFINITY; l[i] = 0.f; }
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) o[b] = v4f{0.f, 0.f, 0.f, 0.f};
    for (uint32_t base = 0; base < npos; base += TP) {
        const uint32_t nv = min(TP, npos - base);
        __syncthreads();                                                   // the previous tile's readers are done
        for (uint32_t i = tid; i < TP * (HD / 4u); i += 256u) {
            const uint32_t p = i / (HD / 4u), d4 = i % (HD / 4u);
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (p < nv) {
                const size_t gi = (size_t)(base + p) * kv_dim + kvh + 4u * d4;
                kv = *(const float4 *)(kc + gi);
                vv = *(const float4 *)(vc + gi);
            }
            *(float4 *)(ks + p * LK + 4u * d4) = kv;                       // rows past the tile: zeros
            *(float4 *)(vs + p * LV + 4u * d4) = vv;
        }
        __syncthreads();
        // S for tokens 0..15 x positions 16 w .. 16 w + 15 of the tile
        v4f s = v4f{0.f, 0.f, 0.f, 0.f};
        const float *kr = ks + (16u * w + c) * LK + g;
#pragma unroll
        for (uint32_t k = 0; k < KS; k++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[k], kr[4u * k], s, 0, 0, 0);
        // masked (past the tile, or after the token's own slot): -inf; then
        // the wave's maximum per token over its 16 positions
        const uint32_t pos = base + 16u * w + c;
        float sv[4], tm[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t t = t0 + 4u * g + i;
            sv[i] = (16u * w + c < nv && pos <= slot0 + t) ? s[i] * scale : -INFINITY;
            tm[i] = sv[i];
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) tm[i] = fmaxf(tm[i], __shfl_xor(tm[i], off, 64));
        }
        if (c == 0)
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) wmax[w * kPfAttRows + 4u * g + i] = tm[i];
        __syncthreads();
        float al[4], ls[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = 4u * g + i;
            const float mt = fmaxf(fmaxf(wmax[r], wmax[kPfAttRows + r]),
                                   fmaxf(wmax[2u * kPfAttRows + r], wmax[3u * kPfAttRows + r]));
            const float mn = fmaxf(m[i], mt);
            // every token has position 0 in the first tile: mn is finite from there on
            al[i] = m[i] == -INFINITY ? 0.f : expf(m[i] - mn);
            m[i] = mn;
            const float p = sv[i] == -INFINITY ? 0.f : expf(sv[i] - mn);
            ps[r * LP + 16u * w + c] = p;
            ls[i] = p;
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) ls[i] += __shfl_xor(ls[i], off, 64);
        }
        if (c == 0)
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) wsum[w * kPfAttRows + 4u * g + i] = ls[i];
        __syncthreads();                                                   // the tile's P and sums
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = 4u * g + i;
            l[i] = l[i] * al[i] + ((wsum[r] + wsum[kPfAttRows + r]) + (wsum[2u * kPfAttRows + r] +
                                                                      wsum[3u * kPfAttRows + r]));
        }
        // O[token][column] for this wave's column blocks: rescale, then P V
#pragma unroll
        for (uint32_t b = 0; b < NB; b++) {
            v4f acc = v4f{o[b][0] * al[0], o[b][1] * al[1], o[b][2] * al[2], o[b][3] * al[3]};
            const uint32_t col = (w * NB + b) * 16u + c;
#pragma unroll
            for (uint32_t k = 0; k < TP / 4u; k++)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ps[c * LP + 4u * k + g], vs[(4u * k + g) * LV + col], acc,
                                                           0, 0, 0);
            o[b] = acc;
        }
    }
    // token 4 g + i, column (w NB + b) 16 + c
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        const uint32_t r = 4u * g + i;
        if (r < nrow) {
            const float inv = 1.0f / l[i];
            float *dst = out + ((size_t)(t0 + r) * gridDim.x + h) * HD;          // out[t][q_dim]
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) dst[(w * NB + b) * 16u + c] = o[b][i] * inv;
        }
    }
}

}  // namespace qgp
namespace qg {

bool prefill_type_supported(uint32_t type)
{
    return type == T_Q4_K || type == T_Q5_K || type == T_Q6_K || type == T_Q8_0;
}

// sub-blocks per slice: ceil(nseg / slices) rounded up to whole chunks
static uint32_t pf_slice_len(uint32_t nseg, uint32_t slices)
{
    const uint32_t sps = (nseg + slices - 1) / slices;
    return (sps + qgp::kPfKC - 1) / qgp::kPfKC * qgp::kPfKC;
}

// Slices of a K split for `tiles` workgroup row tiles over nseg sub-blocks
// (nseg % kPfKC == 0), of whole chunks; returned so that ceil(nseg / sps) ==
// S for the slice length sps = pf_slice_len(nseg, S) (no empty slice).  Up
// to QG_PF_FILL tiles: at most QG_PF_FILL workgroups (one per CU: a second
// workgroup on a CU runs the GEMM at less than half the speed of the first)
// and kPfMaxSlices slices; more tiles: at most QG_PF_WG_TARGET workgroups and
// kPfSliceMax slices.
uint32_t pf_split(uint32_t tiles, uint32_t nseg)
{
    if (tiles == 0 || nseg < qgp::kPfKC) return 1;
    uint32_t s;
    if (tiles <= QG_PF_FILL) {
        s = QG_PF_FILL / tiles;
        if (s > qgp::kPfMaxSlices) s = qgp::kPfMaxSlices;
    } else {
        s = QG_PF_WG_TARGET / tiles;
        if (s > qgp::kPfSliceMax) s = qgp::kPfSliceMax;
    }
    if (s > nseg / qgp::kPfKC) s = nseg / qgp::kPfKC;
    if (s < 1u) s = 1u;
    const uint32_t sps = pf_slice_len(nseg, s);
    return (nseg + sps - 1) / sps;
}

uint32_t pf_tiles(size_t rows) { return (uint32_t)((rows + qgp::kPfRows - 1) / qgp::kPfRows); }

template <uint32_t T>
static void pf_gemm_launch(const qgp::PfJobs &jobs, bool rp, uint32_t tiles, uint32_t nseg, uint32_t slices,
                           const uint16_t *xp, const float *rec, uint32_t ntok, uint32_t cols, uint32_t ldy,
                           size_t sstride, hipStream_t st)
{
    const uint32_t sps = pf_slice_len(nseg, slices);
    const dim3 grid(tiles, slices), block(64 * qgp::kPfWaves);
    // the layout: repacked with one or several rows per group, or GGUF with
    // rows of whole blocks (Q8_0 blocks are single sub-blocks) or straddling
    if (rp) {
        if (jobs.j0.g == 1)
            hipLaunchKernelGGL((qgp::pf_gemm_k<T, 2>), grid, block, qgp::kPfLds, st, jobs, nseg, sps, xp, rec, ntok,
                               cols, ldy, (uint64_t)sstride);
        else
            hipLaunchKernelGGL((qgp::pf_gemm_k<T, 3>), grid, block, qgp::kPfLds, st, jobs, nseg, sps, xp, rec, ntok,
                               cols, ldy, (uint64_t)sstride);
    } else if (T == T_Q8_0 || nseg % 8u == 0) {
        hipLaunchKernelGGL((qgp::pf_gemm_k<T, 1>), grid, block, qgp::kPfLds, st, jobs, nseg, sps, xp, rec, ntok, cols,
                           ldy, (uint64_t)sstride);
    } else if constexpr (T != T_Q8_0) {
        hipLaunchKernelGGL((qgp::pf_gemm_k<T, 0>), grid, block, qgp::kPfLds, st, jobs, nseg, sps, xp, rec, ntok, cols,
                           ldy, (uint64_t)sstride);
    }
}

int launch_pf_gemm(const PfMat *mats, int n_mats, size_t cols, const uint16_t *xp, const float *rec, uint32_t ntok,
                   uint32_t ldy, uint32_t slices, size_t sstride, ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    if (n_mats < 1 || n_mats > 3 || cols % 128 != 0 || cols == 0 || cols > 0xFFFFFFFFull || ntok > kPfMaxTokens)
        return -1;
    const uint32_t nseg = (uint32_t)(cols / 32);
    if (slices < 1 || slices > nseg || slices > qgp::kPfMaxSlices) return -1;
    for (int i = 0; i < n_mats; i++) {
        const PfMat &m = mats[i];
        // 16-byte aligned weights (the K-quant block heads are read as one
        // uint4); a repacked matrix: whole row groups
        if (!prefill_type_supported(m.type) || m.rows == 0 || m.rows > 0xFFFFFFFFull || ((uintptr_t)m.w & 15u) != 0)
            return -1;
        if (m.rp && (m.g == 0 || m.g > 8 || m.rows % m.g != 0 || m.ni == 0 || m.gb == 0)) return -1;
    }
    // one launch per run of matrices of the same type and layout
    for (int i = 0; i < n_mats;) {
        qgp::PfJob j[3] = {};
        uint32_t tiles = 0;
        int n = 0;
        const uint32_t type = mats[i].type;
        const bool rp = mats[i].rp;
        const uint32_t g = mats[i].g;
        for (; i < n_mats && mats[i].type == type && mats[i].rp == rp && (!rp || mats[i].g == g); i++, n++) {
            const PfMat &m = mats[i];
            j[n] = qgp::PfJob{m.w, m.y, m.type, (uint32_t)m.rows, pf_tiles(m.rows), rp ? m.g : 1u, rp ? m.ni : 0u,
                              rp ? (uint64_t)m.gb : 0u};
            tiles += j[n].tiles;
        }
        const qgp::PfJobs jobs{j[0], j[1], j[2], (uint32_t)n};
        hipStream_t st = (hipStream_t)stream;
        const uint32_t c = (uint32_t)cols;
        switch (type) {
        case T_Q4_K: pf_gemm_launch<T_Q4_K>(jobs, rp, tiles, nseg, slices, xp, rec, ntok, c, ldy, sstride, st); break;
        case T_Q5_K: pf_gemm_launch<T_Q5_K>(jobs, rp, tiles, nseg, slices, xp, rec, ntok, c, ldy, sstride, st); break;
        case T_Q6_K: pf_gemm_launch<T_Q6_K>(jobs, rp, tiles, nseg, slices, xp, rec, ntok, c, ldy, sstride, st); break;
        case T_Q8_0: pf_gemm_launch<T_Q8_0>(jobs, rp, tiles, nseg, slices, xp, rec, ntok, c, ldy, sstride, st); break;
        default: return -1;
        }
        if (hipGetLastError() != hipSuccess) return -2;
    }
    return 0;
}

int launch_pf_planes(const float *a, uint32_t na, const float *b, uint32_t nb, size_t sstride, float *sum_out,
                     const float *nw, size_t n, size_t lda, int mode, const float *pre, size_t pre_n, float eps,
                     float *ss_out, uint16_t *xp, float *rec, uint32_t ntok, ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    // 16-byte aligned rows and slices (float4 reads); whole chunks
    if (n % 128 != 0 || n == 0 || n > 0xFFFFFFFFull || ntok > kPfMaxTokens || na < 1 || na > qgp::kPfMaxSlices ||
        (b && (nb < 1 || nb > qgp::kPfMaxSlices)) || (mode == 2 && !b) || (mode == 1 && (!nw || !ss_out)) ||
        (pre && (pre_n == 0 || pre_n > 0xFFFFFFFFull)) || lda % 4 != 0 || sstride % 4 != 0 || ((uintptr_t)a & 15u) ||
        ((uintptr_t)b & 15u) || ((uintptr_t)sum_out & 15u))
        return -1;
    const dim3 grid(qgp::pf_planes_blk((uint32_t)n), ntok), block(qgp::kPfPlanesT);
    hipLaunchKernelGGL(qgp::pf_split_k, grid, block, 0, (hipStream_t)stream, a, na, b, nb, (uint64_t)sstride, sum_out,
                       nw, (uint32_t)n, (uint32_t)lda, (uint32_t)mode, pre, (uint32_t)((pre_n + 255) / 256),
                       (uint32_t)pre_n, eps, ss_out, xp, rec);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_pf_sum(const float *x, uint32_t ns, size_t sstride, size_t n, float *out, ihipStream_t *stream)
{
    if (n == 0) return 0;
    if (ns < 1 || ns > qgp::kPfMaxSlices || n > 0xFFFFFFFFull) return -1;
    hipLaunchKernelGGL(qgp::pf_sum_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, ns,
                       (uint64_t)sstride, (uint32_t)n, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_pf_qkv_post(float *qkv, uint32_t ldq, uint32_t ns, uint32_t ns_v, size_t sstride, const float *ss,
                       size_t ss_n, float eps,
                       const float *bq, const float *bk, const float *bv, float *kc, float *vc, const float *cos_t,
                       const float *sin_t, uint32_t q_dim, uint32_t kv_dim, uint32_t hd, uint32_t pos0, uint32_t slot0,
                       uint32_t ntok, ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    if (ns < 1 || ns > qgp::kPfMaxSlices || ns_v < 1 || ns_v > qgp::kPfMaxSlices || ntok > kPfMaxTokens ||
        hd % 2 != 0 || !ss || ss_n == 0 ||
        ss_n > 0xFFFFFFFFull)
        return -1;
    const uint32_t pairs = (q_dim > kv_dim ? q_dim : kv_dim) / 2;
    hipLaunchKernelGGL(qgp::pf_qkv_post_k, dim3((pairs + 255) / 256, ntok), dim3(256), 0, (hipStream_t)stream, qkv,
                       ldq, ns, ns_v, (uint64_t)sstride, ss, (uint32_t)((ss_n + 255) / 256), (uint32_t)ss_n, eps, bq, bk, bv,
                       kc, vc, cos_t, sin_t, q_dim, kv_dim, hd, pos0, slot0);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_pf_attention(const float *qkv, uint32_t ldq, const float *kc, const float *vc, float *out, uint32_t n_heads,
                        uint32_t hd, uint32_t kv_dim, uint32_t n_rep, float scale, uint32_t slot0, uint32_t ntok,
                        ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    // 16-byte aligned rows (float4 reads of q, K, V and the output)
    if (ntok > kPfMaxTokens || n_rep == 0 || ldq % 4 != 0 || kv_dim % 4 != 0 || ((uintptr_t)qkv & 15u) ||
        ((uintptr_t)kc & 15u) || ((uintptr_t)vc & 15u) || ((uintptr_t)out & 15u))
        return -1;
    // every head's q inside a token's row of qkv, every kv head inside kv_dim
    if (n_heads % n_rep != 0 || (uint64_t)n_heads * hd > ldq || (uint64_t)(n_heads / n_rep) * hd > kv_dim) return -1;
    const dim3 grid(n_heads, (ntok + qgp::kPfAttRows - 1) / qgp::kPfAttRows), block(256);
    hipStream_t st = (hipStream_t)stream;
    switch (hd) {
    case 64:
        hipLaunchKernelGGL(qgp::pf_attention_k<64>, grid, block, qgp::pf_att_lds(64), st, qkv, ldq, kc, vc, out, kv_dim,
                           n_rep, scale, slot0, ntok);
        break;
    case 128:
        hipLaunchKernelGGL(qgp::pf_attention_k<128>, grid, block, qgp::pf_att_lds(128), st, qkv, ldq, kc, vc, out,
                           kv_dim, n_rep, scale, slot0, ntok);
        break;
    case 256:
        hipLaunchKernelGGL(qgp::pf_attention_k<256>, grid, block, qgp::pf_att_lds(256), st, qkv, ldq, kc, vc, out,
                           kv_dim, n_rep, scale, slot0, ntok);
        break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace qg
