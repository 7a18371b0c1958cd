// qg_prefill.hip -- batched prefill: the prompt's tokens through one layer at
// a time (include/qgmodel.h, qg_model_prefill), the multi-token form of the
// decode step of qg_model.hip.
//
// The reference feeds the prompt one token at a time (model.rs:361-365,
// Transformer::forward per token).  Here every projection of a chunk of up
// to kPfMaxTokens tokens is one GEMM on the matrix cores:
//
//   * pf_planes_k: each token's input vector (RMSNorm of the residual stream,
//     the attention output, or silu(g) * u) split into three bf16 pieces
//     x = hi + mid + lo (each the rounding of what the previous ones leave,
//     so the three carry x to f32 precision), written as xp[c][t][i], plus
//     per 32-element segment the sums of x over its halves;
//   * pf_gemm_k: y[t][r] = sum over the row's 32-element sub-blocks of
//     mul * (sum q x) + add * (sum x), with sum q x from three chained
//     v_mfma_f32_16x16x32_bf16 (A: 16 tokens x 32 elements of one piece, B:
//     32 codes x 16 rows as bf16 -- every code of the supported types is an
//     integer of at most 8 bits, exact in bf16; the products are exact in
//     f32, accumulated in f32), the weight scales applied per sub-block in
//     f32;
//   * pf_qkv_post_k, pf_attention_k: bias, RoPE and KV append of every token
//     (attention.rs:66-90), causal attention of every token over the cache up
//     to its own slot (attention.rs:93-121), as the decode path.
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16, checked on gfx950): lane l
// holds A[l % 16][8 (l/16) .. +8), B[8 (l/16) .. +8)[l % 16] and
// D[4 (l/16) + i][l % 16], i = 0..3.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "qg_common.h"

namespace qgp {

using qg::T_Q4_K;
using qg::T_Q5_K;
using qg::T_Q6_K;
using qg::T_Q8_0;

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
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

// quant.rs:606-615: scale and min of sub-block j (0..7) from the 12-byte pack
// held in the dwords q0, q1, q2, without branches on j (a lane-varying value
// when rows straddle blocks)
__device__ __forceinline__ void k4sm(uint32_t j, uint32_t q0, uint32_t q1, uint32_t q2, float &sc, float &m)
{
    const uint32_t s = 8u * (j & 3u);
    const uint32_t A = (q0 >> s) & 0xFFu, B = (q1 >> s) & 0xFFu, C = (q2 >> s) & 0xFFu;   // q[j%4], q[j%4+4], q[j%4+8]
    const bool lo = j < 4u;
    sc = (float)(lo ? (A & 63u) : ((C & 0xFu) | ((A >> 6) << 4)));
    m = (float)(lo ? (B & 63u) : ((C >> 4) | ((B >> 6) << 4)));
}

// bf16 of 1 + q / 2^b for the four b-bit codes in the bytes of c (q < 2^b,
// b <= 7): the exponent of 1 and q as the top b bits of the 7-bit mantissa,
// exact.  Two dwords of two bf16 each.
template <int B>
__device__ __forceinline__ void biased_bf16(uint32_t c, uint32_t &r0, uint32_t &r1)
{
    const uint32_t t = (c << (7 - B)) | 0x80808080u;                   // low byte of each bf16
    r0 = __builtin_amdgcn_perm(0x3F3F3F3Fu, t, 0x04010400u);           // [t0, 3F, t1, 3F]
    r1 = __builtin_amdgcn_perm(0x3F3F3F3Fu, t, 0x04030402u);           // [t2, 3F, t3, 3F]
}

// 8 signed byte codes as bf16 (exact: f32 conversion, top half)
__device__ __forceinline__ uint4 signed_bf16(uint32_t c0, uint32_t c1)
{
    uint32_t r[4];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t c = h ? c1 : c0;
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; i++) f[i] = (float)(int8_t)((c >> (8 * i)) & 0xFFu);
        r[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u);
        r[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u);
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// B operands of the K-quant codes: the MFMA over 32 x with B = 1 + q / 2^b
// gives D' = sum x + (sum q x) / 2^b, so sum q x = 2^b (D' - sum x) and a
// sub-block's mul * (sum q x) + add * (sum x) = mul' D' + add' (sum x) with
// mul' = 2^b mul, add' = add - mul'.  (Masked codes -- the other half of a
// Q6_K sub-block -- are B = 0.)
template <int B>
__device__ __forceinline__ uint4 kquant_b(uint32_t c0, uint32_t c1, bool keep)
{
    uint4 r;
    biased_bf16<B>(c0, r.x, r.y);
    biased_bf16<B>(c1, r.z, r.w);
    return keep ? r : make_uint4(0u, 0u, 0u, 0u);
}

// Per-type access to one 32-element sub-block (sub-block j of the block at
// blk; rows hold whole sub-blocks since cols % 32 == 0), in two steps so that
// the loads can be issued a chunk ahead:
//   load(blk, j, kq): the raw dwords the lane needs (every byte read lies in
//     the matrix or its tail pad);
//   decode(raw, j, kq, b, mul, add): b[h] = the B operand (codes 8 kq ..
//     8 kq + 7 as bf16) of set h, and the sub-block's contribution is sum
//     over sets of mul_h * D_h + add_h * (sum x over the set), D_h the MFMA
//     result;
//   NSET = 1 when one scale covers all 32 codes, 2 for Q6_K's 16-code
//   sub-blocks (h = 0 codes 0..15, h = 1 codes 16..31); SUMS: add is used.
template <uint32_t T> struct PfW;

// Q4_K (quant.rs:210-228): 8 sub-blocks per 144-byte block; sub-block j is
// the low (j even) or high (j odd) nibbles of qs[32 (j/2) .. +32); the value
// is d * sc * q - dmin * m.
template <> struct PfW<T_Q4_K> {
    static constexpr int NSET = 1;
    static constexpr bool SUMS = true;
    struct Raw {
        uint4 head;
        uint2 v;
    };
    static constexpr uint32_t BB = 144;
    __device__ static Raw load(const uint8_t *b, uint32_t j, uint32_t kq)
    {
        return Raw{*(const uint4 *)b, *(const uint2 *)(b + 16u + 32u * (j >> 1) + 8u * kq)};
    }
    __device__ static void decode(const Raw &r, uint32_t j, uint32_t, uint4 (&bq)[2], float (&mul)[2],
                                  float (&add)[2])
    {
        const uint32_t sh = (j & 1u) * 4u;
        bq[0] = kquant_b<4>((r.v.x >> sh) & 0x0F0F0F0Fu, (r.v.y >> sh) & 0x0F0F0F0Fu, true);
        float sc, m;
        k4sm(j, r.head.y, r.head.z, r.head.w, sc, m);
        mul[0] = 16.0f * (h2f(r.head.x) * sc);
        add[0] = -(h2f(r.head.x >> 16) * m) - mul[0];
    }
    // the repacked row group G (the library's repack_k layout: the nb = ni/2
    // block heads, then piece k' (16 bytes) of item it at 16 nb + (k' ni + it)
    // 16; item it = the quant bytes 64 (it & 1) .. +64 of block it / 2): the
    // same registers as load
    using RawR = Raw;
    __device__ static RawR load_rp(const uint8_t *G, uint32_t b, uint32_t j, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = 2u * b + (j >> 2), kp = 2u * ((j >> 1) & 1u) + (kq >> 1);
        return Raw{*(const uint4 *)(G + 16u * b), *(const uint2 *)(G + 8u * ni + (kp * ni + it) * 16u + 8u * (kq & 1u))};
    }
    __device__ static void decode_rp(const RawR &r, uint32_t j, uint32_t kq, uint4 (&bq)[2], float (&mul)[2],
                                     float (&add)[2])
    {
        decode(r, j, kq, bq, mul, add);
    }
};

// Q5_K (quant.rs:231-262): as Q4_K with a fifth bit, bit j of qh[l].
template <> struct PfW<T_Q5_K> {
    static constexpr int NSET = 1;
    static constexpr bool SUMS = true;
    struct Raw {
        uint4 head;
        uint2 v, h;
    };
    static constexpr uint32_t BB = 176;
    __device__ static Raw load(const uint8_t *b, uint32_t j, uint32_t kq)
    {
        return Raw{*(const uint4 *)b, *(const uint2 *)(b + 48u + 32u * (j >> 1) + 8u * kq),
                   *(const uint2 *)(b + 16u + 8u * kq)};
    }
    __device__ static void decode(const Raw &r, uint32_t j, uint32_t, uint4 (&bq)[2], float (&mul)[2],
                                  float (&add)[2])
    {
        const uint32_t sh = (j & 1u) * 4u;
        const uint32_t c0 = ((r.v.x >> sh) & 0x0F0F0F0Fu) | (((r.h.x >> j) & 0x01010101u) << 4);
        const uint32_t c1 = ((r.v.y >> sh) & 0x0F0F0F0Fu) | (((r.h.y >> j) & 0x01010101u) << 4);
        bq[0] = kquant_b<5>(c0, c1, true);
        float sc, m;
        k4sm(j, r.head.y, r.head.z, r.head.w, sc, m);
        mul[0] = 32.0f * (h2f(r.head.x) * sc);
        add[0] = -(h2f(r.head.x >> 16) * m) - mul[0];
    }
    // the repacked row group G (repack_k: the nb = ni/4 block heads, piece k'
    // of item it's 32 quant bytes at 16 nb + (k' ni + it) 16, then 8 bytes per
    // item at 16 nb + 32 ni + 8 it: bits 8 bb + 2 t' + q of word w are bit
    // 2 (it & 3) + q of qh[16 w + 4 t' + bb]; item it = block it / 4, sub-blocks
    // 2 (it & 3) and 2 (it & 3) + 1)
    struct RawR {
        uint4 head;
        uint2 v;
        uint32_t w;
    };
    __device__ static RawR load_rp(const uint8_t *G, uint32_t b, uint32_t j, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = 4u * b + (j >> 1), H = 4u * ni;             // 16 nb
        return RawR{*(const uint4 *)(G + 16u * b),
                    *(const uint2 *)(G + H + ((kq >> 1) * ni + it) * 16u + 8u * (kq & 1u)),
                    *(const uint32_t *)(G + H + 32u * ni + 8u * it + 4u * (kq >> 1))};
    }
    __device__ static void decode_rp(const RawR &r, uint32_t j, uint32_t kq, uint4 (&bq)[2], float (&mul)[2],
                                     float (&add)[2])
    {
        // code 8 kq + e: qh byte 16 w + 4 t' + bb with w = kq / 2, t' =
        // 2 (kq & 1) + e / 4, bb = e % 4, so its bit j sits at 8 (e % 4) + s
        // (+ 2 for e >= 4), s = 4 (kq & 1) + (j & 1)
        const uint32_t sh = (j & 1u) * 4u, s = 4u * (kq & 1u) + (j & 1u);
        const uint32_t c0 = ((r.v.x >> sh) & 0x0F0F0F0Fu) | (((r.w >> s) & 0x01010101u) << 4);
        const uint32_t c1 = ((r.v.y >> sh) & 0x0F0F0F0Fu) | (((r.w >> (s + 2u)) & 0x01010101u) << 4);
        bq[0] = kquant_b<5>(c0, c1, true);
        float sc, m;
        k4sm(j, r.head.y, r.head.z, r.head.w, sc, m);
        mul[0] = 32.0f * (h2f(r.head.x) * sc);
        add[0] = -(h2f(r.head.x >> 16) * m) - mul[0];
    }
};

// Q6_K (quant.rs:265-292): 210-byte blocks (2-byte aligned), halves n of 128
// elements; within a half, sub-block k4 (32 elements, l = 0..31) takes the
// low (k4 < 2) or high nibbles of ql[64 n + 32 (k4 & 1) + l], bits 2 k4 of
// qh[32 n + l], and scale sc[8 n + l/16 + 2 k4]; the value is
// d * sc * (q - 32).  Reads stay inside the block but for the dword holding
// d, which can end 2 bytes past the last block (inside the buffer's tail pad).
template <> struct PfW<T_Q6_K> {
    static constexpr int NSET = 2;
    static constexpr bool SUMS = true;
    struct Raw {
        uint32_t ql[3], qh[3], s, d, sb;
    };
    static constexpr uint32_t BB = 210;
    __device__ static Raw load(const uint8_t *b, uint32_t j, uint32_t kq)
    {
        const uint32_t n = j >> 2, k4 = j & 3u;
        const uint32_t *pl = adown(b + 64u * n + 32u * (k4 & 1u) + 8u * kq);
        const uint32_t *ph = adown(b + 128u + 32u * n + 8u * kq);
        Raw r;
        r.ql[0] = pl[0];
        r.ql[1] = pl[1];
        r.ql[2] = pl[2];
        r.qh[0] = ph[0];
        r.qh[1] = ph[1];
        r.qh[2] = ph[2];
        r.s = *adown(b + 192u + 8u * n + 2u * k4);
        r.d = *adown(b + 208u);
        r.sb = (uint32_t)((uintptr_t)b & 3u);
        return r;
    }
    __device__ static void decode(const Raw &r, uint32_t j, uint32_t kq, uint4 (&bq)[2], float (&mul)[2],
                                  float (&add)[2])
    {
        // w is 4-byte aligned: the block starts at byte sb = 0 or 2 of a dword;
        // ql, qh and d at offsets 0 mod 4 from it, the scale pair at 2 k4
        const uint32_t sb = r.sb, k4 = j & 3u, ss = (sb + 2u * k4) & 3u;
        const uint32_t sl = (k4 >> 1) * 4u, shh = 2u * k4;
        const uint32_t L0 = abyte(r.ql[1], r.ql[0], sb), L1 = abyte(r.ql[2], r.ql[1], sb);
        const uint32_t H0 = abyte(r.qh[1], r.qh[0], sb), H1 = abyte(r.qh[2], r.qh[1], sb);
        const uint32_t c0 = ((L0 >> sl) & 0x0F0F0F0Fu) | (((H0 >> shh) & 0x03030303u) << 4);
        const uint32_t c1 = ((L1 >> sl) & 0x0F0F0F0Fu) | (((H1 >> shh) & 0x03030303u) << 4);
        const bool lo = kq < 2u;                                      // codes 0..15 of the sub-block
        bq[0] = kquant_b<6>(c0, c1, lo);
        bq[1] = kquant_b<6>(c0, c1, !lo);
        const uint32_t s = r.s >> (8 * ss), dd = r.d >> (8 * sb);   // sc[8n + 2k4], sc[8n + 2k4 + 1]; d
        const float d = h2f(dd);
        const float m0 = d * (float)(int8_t)(s & 0xFFu), m1 = d * (float)(int8_t)((s >> 8) & 0xFFu);
        mul[0] = 64.0f * m0;
        mul[1] = 64.0f * m1;
        add[0] = -32.0f * m0 - mul[0];
        add[1] = -32.0f * m1 - mul[1];
    }
    // the repacked row group G (repack_k: item it = block it/4, half
    // n = (it/2) & 1, i = it & 1 -- l in 16 i .. 16 i + 15 of the half;
    // ql[64n+16i..+16] at 16 it, ql[64n+32+16i..+16] at 16 (ni + it),
    // qh[32n+16i..+16] at 16 (2 ni + it), sc[8n+i+2k] at 48 ni + 4 it + k, d
    // at 52 ni + 2 b)
    struct RawR {
        uint2 ql, qh, sc;
        uint32_t d;
    };
    __device__ static RawR load_rp(const uint8_t *G, uint32_t b, uint32_t j, uint32_t kq, uint32_t ni)
    {
        const uint32_t n = j >> 2, k4 = j & 3u, it0 = 4u * b + 2u * n, it = it0 + (kq >> 1);
        return RawR{*(const uint2 *)(G + ((k4 & 1u) * ni + it) * 16u + 8u * (kq & 1u)),
                    *(const uint2 *)(G + (2u * ni + it) * 16u + 8u * (kq & 1u)),
                    *(const uint2 *)(G + 48u * ni + 4u * it0),          // scales of items it0, it0 + 1
                    (uint32_t)*(const uint16_t *)(G + 52u * ni + 2u * b)};
    }
    __device__ static void decode_rp(const RawR &r, uint32_t j, uint32_t kq, uint4 (&bq)[2], float (&mul)[2],
                                     float (&add)[2])
    {
        const uint32_t k4 = j & 3u, sl = (k4 >> 1) * 4u, shh = 2u * k4;
        const uint32_t c0 = ((r.ql.x >> sl) & 0x0F0F0F0Fu) | (((r.qh.x >> shh) & 0x03030303u) << 4);
        const uint32_t c1 = ((r.ql.y >> sl) & 0x0F0F0F0Fu) | (((r.qh.y >> shh) & 0x03030303u) << 4);
        const bool lo = kq < 2u;                                      // codes 0..15 of the sub-block
        bq[0] = kquant_b<6>(c0, c1, lo);
        bq[1] = kquant_b<6>(c0, c1, !lo);
        const float d = h2f(r.d);
        // sc[8n + 2k4] (l < 16: item it0) and sc[8n + 2k4 + 1] (item it0 + 1)
        const float m0 = d * (float)(int8_t)((r.sc.x >> (8u * k4)) & 0xFFu);
        const float m1 = d * (float)(int8_t)((r.sc.y >> (8u * k4)) & 0xFFu);
        mul[0] = 64.0f * m0;
        mul[1] = 64.0f * m1;
        add[0] = -32.0f * m0 - mul[0];
        add[1] = -32.0f * m1 - mul[1];
    }
};

// Q8_0 (quant.rs:106-113): one 34-byte block (2-byte aligned) per sub-block,
// int8 codes as bf16 (exact), value d * q.
template <> struct PfW<T_Q8_0> {
    static constexpr int NSET = 1;
    static constexpr bool SUMS = false;
    struct Raw {
        uint32_t q[3], d, sb;
    };
    static constexpr uint32_t BB = 34;
    __device__ static Raw load(const uint8_t *b, uint32_t, uint32_t kq)
    {
        const uint32_t *pq = adown(b + 2u + 8u * kq);
        return Raw{{pq[0], pq[1], pq[2]}, *adown(b), (uint32_t)((uintptr_t)b & 3u)};
    }
    __device__ static void decode(const Raw &r, uint32_t, uint32_t, uint4 (&bq)[2], float (&mul)[2],
                                  float (&add)[2])
    {
        // w is 4-byte aligned: block b starts at byte 0 or 2 of a dword, its
        // codes (b + 2 + 8 kq) at byte 2 or 0 of q[0]
        const uint32_t sb = r.sb, sq = (sb + 2u) & 3u;
        bq[0] = signed_bf16(abyte(r.q[1], r.q[0], sq), abyte(r.q[2], r.q[1], sq));
        mul[0] = h2f(r.d >> (8 * sb));
        add[0] = 0.0f;
    }
    // the repacked row group G (repack_k: item it = blocks 2 it, 2 it + 1;
    // piece k' (codes 16 k' .. +16) at (k' ni + it) 16, the two d halves at
    // 64 ni + 4 it)
    struct RawR {
        uint2 q;
        uint32_t d;
    };
    __device__ static RawR load_rp(const uint8_t *G, uint32_t b, uint32_t, uint32_t kq, uint32_t ni)
    {
        const uint32_t it = b >> 1, kp = 2u * (b & 1u) + (kq >> 1);
        return RawR{*(const uint2 *)(G + (kp * ni + it) * 16u + 8u * (kq & 1u)),
                    (uint32_t)*(const uint16_t *)(G + 64u * ni + 4u * it + 2u * (b & 1u))};
    }
    __device__ static void decode_rp(const RawR &r, uint32_t, uint32_t, uint4 (&bq)[2], float (&mul)[2],
                                     float (&add)[2])
    {
        bq[0] = signed_bf16(r.q.x, r.q.y);
        mul[0] = h2f(r.d);
        add[0] = 0.0f;
    }
};

#ifndef QG_PF_KC
#define QG_PF_KC 2
#endif
#ifndef QG_PF_R
#define QG_PF_R 2
#endif
#ifndef QG_PF_WAVES
#define QG_PF_WAVES 4
#endif
constexpr uint32_t kPfKC = QG_PF_KC;                         // sub-blocks per staged chunk
constexpr uint32_t kPfR = QG_PF_R;                           // 16-row tiles per wave
constexpr uint32_t kPfWaves = QG_PF_WAVES;                   // waves per workgroup
constexpr uint32_t kPfRows = 16u * kPfR * kPfWaves;          // rows per workgroup tile
constexpr uint32_t kPfBufX = kPfKC * 3u * 64u * 64u;         // bytes of x pieces per buffer
constexpr uint32_t kPfBuf = kPfBufX + kPfKC * 1024u;         // ... and of the sums
constexpr uint32_t kPfLds = 2u * kPfBuf;                     // two buffers

// 16 bytes per lane from global memory straight into LDS at byte m0 + 16 lane
// (global_load_lds_dwordx4, issued from asm: the compiler does not track it,
// the waits for it are explicit; lds_addr is an operand bound to M0, which
// the compiler writes itself)
__device__ __forceinline__ void pf_dma16(const void *gp, uint32_t lds_addr)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "{m0}"(lds_addr) : "memory");
}

// Issue the copies of chunk kc (nk sub-blocks) into the buffer at LDS byte
// address b0: x block u = (kk * 3 + c) * 4 + g (sub-block kk, piece c,
// tokens 16 g .. 16 g + 15; 1 KB, token t's 64 bytes as four 16-byte slots,
// slot s stored at position s ^ pf_swz(t) so that the A-operand reads of
// 8 or 16 consecutive tokens at one slot hit distinct banks), then per
// sub-block the 256 sums.  Tokens
// past the chunk repeat the last one (their outputs are never stored).
// slot position of token t's slots in its 64-byte LDS row: the 16-byte
// reads of tokens t..t+7 (t % 8 == 0) at one slot cover 8 distinct 16-byte
// bank groups mod 128 bytes, those of t..t+15 16 distinct groups mod 256
__device__ __forceinline__ uint32_t pf_swz(uint32_t t) { return ((t >> 1) ^ (t >> 3)) & 3u; }

__device__ __forceinline__ void pf_stage(const uint16_t *__restrict__ xp, const float *__restrict__ rec,
                                         uint32_t ntok, uint32_t n, uint32_t kc, uint32_t nk, uint32_t b0,
                                         uint32_t wave, uint32_t lane)
{
#pragma unroll
    for (uint32_t v = 0; v < (kPfKC * 12u + kPfWaves - 1u) / kPfWaves; v++) {
        const uint32_t u = v * kPfWaves + wave, kk = u / 12u, c = (u >> 2) % 3u, g = u & 3u;
        if (kk < nk) {                                               // wave-uniform (u past the chunk: kk >= kPfKC)
            const uint32_t t = min(16u * g + (lane >> 2), ntok - 1u);
            const uint32_t s = (lane & 3u) ^ pf_swz(lane >> 2);
            pf_dma16(xp + ((size_t)c * ntok + t) * n + 32u * (kc + kk) + 8u * s, b0 + u * 1024u);
        }
    }
    if (wave < nk) pf_dma16(rec + (size_t)(kc + wave) * 256u + 4u * lane, b0 + kPfBufX + wave * 1024u);
}

// One workgroup's share of a grouped GEMM: rows row0 .. row0 + 16 R (R
// tiles of 16 rows per wave; waves past the matrix still stage), K slice
// k0 .. k1, all the chunk's tokens.  x of token t: xp[c][t][i] (c = 0..2,
// piece stride ntok * n); per sub-block k the sums rec[(4 k + f) * 64 + t],
// f = 0: sum x, 1: sum x[0..16), 2: sum x[16..32).  Chunks of kPfKC
// sub-blocks are copied into two LDS buffers in turn, the next chunk's copy
// and weight loads in flight while this one is computed.  D[4 kq + i][c16]
// of an MFMA is token 16 tt + 4 kq + i of row r0 + c16.  LAY, the weight
// layout: 0 GGUF, rows straddling blocks; 1 GGUF, every row starts a block
// (nseg % 8 == 0, or single-sub-block blocks), so the sub-block index within
// the block is the same in every lane; 2 repacked (repack_k), one row per
// row group; 3 repacked, gg rows per group of gb bytes (ni items).
template <uint32_t T, int R, int LAY>
__device__ __forceinline__ void pf_gemm_rows(const uint8_t *__restrict__ w, uint32_t rows, uint32_t row0,
                                             uint32_t nseg, uint32_t k0, uint32_t k1,
                                             const uint16_t *__restrict__ xp, const float *__restrict__ rec,
                                             uint32_t ntok, uint32_t n, uint8_t *lds, float *__restrict__ y,
                                             uint32_t ldy, uint32_t gg, uint64_t gb, uint32_t ni)
{
    using P = PfW<T>;
    constexpr bool RPL = LAY >= 2, AL = LAY != 0;
    using Raw = std::conditional_t<RPL, typename P::RawR, typename P::Raw>;
    constexpr bool SB1 = T == T_Q8_0;                                 // one sub-block per block
    const uint32_t lane = threadIdx.x & 63u, kq = lane >> 4, c16 = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
    const bool active = row0 < rows;                                  // wave-uniform
    const uint32_t swz = kq ^ pf_swz(c16);                           // this lane's slot position
    // per row tile: GGUF, the flat index of the row's first sub-block and
    // (AL) its first block; repacked, the row's sub-block offset in its row
    // group and the group
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
            rb[i] = w + (SB1 ? fb[i] : fb[i] / 8u) * P::BB;
        }
    }
    // sub-block k of row tile i: its index in its block, and the block
    auto subj = [&](int i, uint32_t k) -> uint32_t {
        if constexpr (SB1) return 0u;
        else if constexpr (AL && LAY != 3) return k & 7u;
        else return ((uint32_t)fb[i] + k) & 7u;
    };
    auto block = [&](int i, uint32_t k) -> const uint8_t * {
        if constexpr (SB1) return rb[i] + (size_t)k * P::BB;
        else if constexpr (AL) return rb[i] + (size_t)(k >> 3) * P::BB;
        else return w + ((fb[i] + k) >> 3) * P::BB;
    };
    // weights of sub-block k (clamped into the slice: the loads past its end
    // are harmless repeats, unconditional so that none waits on a branch)
    auto wload = [&](int i, uint32_t k) -> Raw {
        const uint32_t kc = min(k, k1 - 1u);
        if constexpr (RPL) {
            const uint32_t f = (uint32_t)fb[i] + kc;                 // sub-block in the row group
            return P::load_rp(rb[i], SB1 ? f : f >> 3, f & 7u, kq, ni);
        } else {
            return P::load(block(i, kc), subj(i, kc), kq);
        }
    };
    v4f acc[R][4];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int tt = 0; tt < 4; tt++) acc[i][tt] = v4f{0.f, 0.f, 0.f, 0.f};
    Raw raw[kPfKC][R];
    pf_stage(xp, rec, ntok, n, k0, min(kPfKC, k1 - k0), lds0, wave, lane);
#pragma unroll
    for (uint32_t kk = 0; kk < kPfKC; kk++)
#pragma unroll
        for (int i = 0; i < R; i++) raw[kk][i] = wload(i, k0 + kk);
    uint32_t buf = 0;
    for (uint32_t kc = k0; kc < k1; kc += kPfKC, buf ^= 1u) {
        const uint32_t nk = min(kPfKC, k1 - kc);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");             // this wave's copies of chunk kc landed
        __syncthreads();                                              // everyone's; the other buffer is free
        if (kc + kPfKC < k1)
            pf_stage(xp, rec, ntok, n, kc + kPfKC, min(kPfKC, k1 - kc - kPfKC), lds0 + (buf ^ 1u) * kPfBuf, wave,
                     lane);
        const uint8_t *xb = lds + buf * kPfBuf;
        const float *rs = (const float *)(xb + kPfBufX);
        float addv[R][kPfKC][2];
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (uint32_t kk = 0; kk < kPfKC; kk++) addv[i][kk][0] = addv[i][kk][1] = 0.f;
#pragma unroll
        for (uint32_t kk = 0; kk < kPfKC; kk++) {
            if (kk >= nk) break;
            // decode this sub-block's weights, then reuse their registers for
            // the next chunk's
            uint4 bq[R][2];
            float mul[R][2];
#pragma unroll
            for (int i = 0; i < R; i++) {
                if constexpr (RPL) P::decode_rp(raw[kk][i], subj(i, kc + kk), kq, bq[i], mul[i], addv[i][kk]);
                else P::decode(raw[kk][i], subj(i, kc + kk), kq, bq[i], mul[i], addv[i][kk]);
            }
#pragma unroll
            for (int i = 0; i < R; i++) raw[kk][i] = wload(i, kc + kPfKC + kk);
            if (!active) continue;
#pragma unroll
            for (uint32_t tt = 0; tt < 4; tt++) {
                const uint8_t *xa = xb + ((((kk * 3u) * 64u + 16u * tt + c16) * 4u + swz) << 4);
                const bf8 a0 = *(const bf8 *)xa;
                const bf8 a1 = *(const bf8 *)(xa + 64u * 64u);
                const bf8 a2 = *(const bf8 *)(xa + 128u * 64u);
#pragma unroll
                for (int h = 0; h < P::NSET; h++)
#pragma unroll
                    for (int i = 0; i < R; i++) {
                        const bf8 b = __builtin_bit_cast(bf8, bq[i][h]);
                        const v4f z = {0.f, 0.f, 0.f, 0.f};
                        v4f d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, z, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b, d, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[i][tt][e] = __builtin_fmaf(mul[i][h], d[e], acc[i][tt][e]);
                    }
            }
        }
        if constexpr (P::SUMS) {
            if (!active) continue;
            // the chunk's add * (sum x) terms as one f32 MFMA (K = 4) per row
            // tile and token tile: K slot kq is sub-block qk, set qh of the
            // chunk (A: the sums of the tile's 16 tokens, B: the row's add)
            const uint32_t qk = P::NSET == 1 ? kq : kq >> 1, qh = P::NSET == 1 ? 0u : kq & 1u;
            const bool qv = qk < nk;
            float bv[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                float s = 0.f;
#pragma unroll
                for (uint32_t kk = 0; kk < kPfKC; kk++)
#pragma unroll
                    for (uint32_t h = 0; h < (uint32_t)P::NSET; h++) s = (qk == kk && qh == h) ? addv[i][kk][h] : s;
                bv[i] = qv ? s : 0.f;
            }
            const float *sa = rs + min(qk, kPfKC - 1u) * 256u + (P::NSET == 1 ? 0u : 64u * (1u + qh)) + c16;
#pragma unroll
            for (uint32_t tt = 0; tt < 4; tt++) {
                const float av = qv ? sa[16u * tt] : 0.f;
#pragma unroll
                for (int i = 0; i < R; i++) acc[i][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[i], acc[i][tt], 0, 0, 0);
            }
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
                if (t < ntok) y[(size_t)t * ldy + r] = acc[i][tt][e];
            }
        }
    }
}

// One matrix of a grouped GEMM launch: its rows, workgroup tiles of
// 64 kPfR rows, and where row 0 of token 0 of slice 0 of its output goes.
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
// sub-blocks; slice s of a job writes its partial products to
// y + s * sstride (the consumer sums the slices in order s = 0, 1, ...).
// 4 waves of 16 kPfR rows per workgroup.
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
    const uint32_t k0 = blockIdx.y * sps, k1 = min(nseg, k0 + sps);
    pf_gemm_rows<T, kPfR, LAY>(J.w, J.rows, row0, nseg, k0, k1, xp, rec, ntok, n, (uint8_t *)pf_lds4,
                               J.y + (size_t)blockIdx.y * sstride, ldy, J.g, J.gb, J.ni);
}

// ---------------------------------------------------------------- planes
//
// The input vector of token blockIdx.y (mode 0: a; mode 1: rmsnorm(a + b) * nw
// with a + b stored to sum_out when given; mode 2: silu(a) * b) as three
// bf16 pieces and per-segment sums.  a and b may be the K-split slices of a
// GEMM (na, nb <= kPfMaxSlices slices sstride floats apart, summed in slice
// order).  Each thread converts 8-element pieces (a quarter of a 32-element
// segment; the four threads of a segment combine their sums through lane
// shuffles).  Mode 1 runs one workgroup per token (the norm needs the whole
// row); sum_out must not alias a or b.
constexpr int kPfPlanesBlock = 256;
constexpr uint32_t kPfMaxSlices = 16;

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

// bf16 of x rounded to nearest even (finite x), as the top half of a dword
__device__ __forceinline__ uint32_t bf16_rn(float x)
{
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
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

__global__ void __launch_bounds__(1024) pf_planes_k(const float *__restrict__ a, uint32_t na,
                                                    const float *__restrict__ b, uint32_t nb, uint64_t sstride,
                                                    float *__restrict__ sum_out, const float *__restrict__ nw,
                                                    float eps, uint32_t n, uint32_t lda, uint32_t mode,
                                                    uint16_t *__restrict__ xp, float *__restrict__ rec,
                                                    uint32_t ntok)
{
    __shared__ float red[16];
    const uint32_t t = blockIdx.y, npc = n / 8u;
    const float *at = a + (size_t)t * lda, *bt = b ? b + (size_t)t * lda : nullptr;
    float inv = 1.0f;
    if (mode == 1) {
        float ss = 0.f;
        for (uint32_t j = threadIdx.x; j < npc; j += blockDim.x) {
            float v[8];
            pf_input8(at, na, bt, nb, sstride, mode, 8u * j, v);
            if (sum_out) {
                float *so = sum_out + (size_t)t * lda + 8u * j;
                *(float4 *)so = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(so + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) ss += v[e] * v[e];
        }
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
        for (uint32_t i = 0; i < blockDim.x / 64u; i++) tot += red[i];
        inv = 1.0f / sqrtf(tot / (float)n + eps);
    }
    const size_t piece = (size_t)ntok * n;
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < npc; j += gridDim.x * blockDim.x) {
        const uint32_t e0 = 8u * j;
        float v[8];
        if (mode == 1 && sum_out) {                                   // written above by this thread
            const float *so = sum_out + (size_t)t * lda + e0;
            const float4 p0 = *(const float4 *)so, p1 = *(const float4 *)(so + 4);
            v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w; v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
        } else {
            pf_input8(at, na, bt, nb, sstride, mode, e0, v);
        }
        if (mode == 1)
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = v[e] * inv * nw[e0 + e];   // math.rs:253-255
        // per float4 (x0 + x1) + (x2 + x3); per quarter the two; per half the two quarters
        const float qsum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        const float hsum = qsum + __shfl_xor(qsum, 1, 64);           // this quarter's half
        const float other = __shfl_xor(hsum, 2, 64);
        const uint32_t qi = j & 3u;
        const float s0 = qi < 2u ? hsum : other, s1 = qi < 2u ? other : hsum;
        uint32_t w[3][4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t pc[3][2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float x = v[e + h];
                const bool fin = __builtin_isfinite(x);
                const uint32_t hi = fin ? bf16_rn(x) : (__float_as_uint(x) & 0xFFFF0000u) | (x != x ? 0x00400000u : 0u);
                const float r1 = fin ? x - __uint_as_float(hi) : 0.f;
                const uint32_t mid = bf16_rn(r1);
                const uint32_t lo = bf16_rn(r1 - __uint_as_float(mid));
                pc[0][h] = hi;
                pc[1][h] = mid;
                pc[2][h] = lo;
            }
#pragma unroll
            for (int c = 0; c < 3; c++) w[c][e >> 1] = (pc[c][0] >> 16) | pc[c][1];
        }
        uint16_t *p0 = xp + (size_t)t * n + e0;
#pragma unroll
        for (int c = 0; c < 3; c++) *(uint4 *)(p0 + c * piece) = make_uint4(w[c][0], w[c][1], w[c][2], w[c][3]);
        if (qi == 0u) {
            float *rg = rec + (size_t)(j >> 2) * 256u + t;
            rg[0] = s0 + s1;
            rg[64] = s0;
            rg[128] = s1;
        }
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
                                                     uint64_t sstride, const float *__restrict__ bq,
                                                     const float *__restrict__ bk, const float *__restrict__ bv,
                                                     float *__restrict__ kc, float *__restrict__ vc,
                                                     const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                     uint32_t q_dim, uint32_t kv_dim, uint32_t hd, uint32_t pos0,
                                                     uint32_t slot0)
{
    const uint32_t t = blockIdx.y, i0 = 2 * (blockIdx.x * blockDim.x + threadIdx.x), half = hd / 2;
    const uint32_t pos = pos0 + t, slot = slot0 + t;
    float *q = qkv + (size_t)t * ldq, *k = q + q_dim, *v = k + kv_dim;
    if (i0 < q_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float x0 = sum_slices(q + i0, ns, sstride) + bq[i0], x1 = sum_slices(q + i0 + 1, ns, sstride) + bq[i0 + 1];
        q[i0] = x0 * c - x1 * s;
        q[i0 + 1] = x0 * s + x1 * c;
    }
    if (i0 < kv_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float x0 = sum_slices(k + i0, ns, sstride) + bk[i0], x1 = sum_slices(k + i0 + 1, ns, sstride) + bk[i0 + 1];
        float *kr = kc + (size_t)slot * kv_dim, *vr = vc + (size_t)slot * kv_dim;
        kr[i0] = x0 * c - x1 * s;
        kr[i0 + 1] = x0 * s + x1 * c;
        vr[i0] = sum_slices(v + i0, ns, sstride) + bv[i0];
        vr[i0 + 1] = sum_slices(v + i0 + 1, ns, sstride) + bv[i0 + 1];
    }
}

// Attention of query head blockIdx.x of token blockIdx.y over cache slots
// 0 .. slot0 + t (attention.rs:93-121, math.rs:63-70 / 104-118); LDS: hd
// floats of q, then the scores.
__global__ void __launch_bounds__(256) pf_attention_k(const float *__restrict__ qkv, uint32_t ldq,
                                                      const float *__restrict__ kc, const float *__restrict__ vc,
                                                      float *__restrict__ out, uint32_t hd, uint32_t kv_dim,
                                                      uint32_t n_rep, float scale, uint32_t slot0)
{
    extern __shared__ float sm[];
    __shared__ float red[4];
    float *qs = sm, *sc = sm + hd;
    const uint32_t t = blockIdx.y, h = blockIdx.x, kvh = (h / n_rep) * hd, seq = slot0 + t + 1;
    const float *q = qkv + (size_t)t * ldq + (size_t)h * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = q[d];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float *kr = kc + (size_t)j * kv_dim + kvh;
        float s = 0.f;
        for (uint32_t d = 0; d < hd; d++) s += qs[d] * kr[d];
        s = s * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sum;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) sc[j] *= inv;
    __syncthreads();
    float *o = out + ((size_t)t * gridDim.x + h) * hd;             // out[t][q_dim]
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
        for (uint32_t j = 0; j < seq; j++) acc += sc[j] * vc[(size_t)j * kv_dim + kvh + d];
        o[d] = acc;
    }
}

}  // namespace qgp

namespace qg {

bool prefill_type_supported(uint32_t type)
{
    return type == T_Q4_K || type == T_Q5_K || type == T_Q6_K || type == T_Q8_0;
}

// Slices of a K split for `tiles` workgroup row tiles over nseg sub-blocks:
// about 1024 workgroups in all, at most 16 slices of at least 4 sub-blocks;
// returned so that ceil(nseg / ceil(nseg / S)) == S (no empty slice).
uint32_t pf_split(uint32_t tiles, uint32_t nseg)
{
    if (tiles == 0 || nseg == 0) return 1;
    uint32_t s = (512u + tiles - 1) / tiles;
    if (s > 16u) s = 16u;
    if (s > nseg / 4u) s = nseg / 4u;
    if (s < 1u) s = 1u;
    const uint32_t sps = (nseg + s - 1) / s;
    return (nseg + sps - 1) / sps;
}

uint32_t pf_tiles(size_t rows) { return (uint32_t)((rows + qgp::kPfRows - 1) / qgp::kPfRows); }

template <uint32_t T>
static void pf_gemm_launch(const qgp::PfJobs &jobs, bool rp, uint32_t tiles, uint32_t nseg, uint32_t slices,
                           const uint16_t *xp, const float *rec, uint32_t ntok, uint32_t cols, uint32_t ldy,
                           size_t sstride, hipStream_t st)
{
    const uint32_t sps = (nseg + slices - 1) / slices;
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
    if (n_mats < 1 || n_mats > 3 || cols % 32 != 0 || cols == 0 || cols > 0xFFFFFFFFull || ntok > kPfMaxTokens)
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
                     const float *nw, float eps, size_t n, size_t lda, int mode, uint16_t *xp, float *rec,
                     uint32_t ntok, ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    // 16-byte aligned rows and slices (float4 reads)
    if (n % 32 != 0 || n == 0 || n > 0xFFFFFFFFull || ntok > kPfMaxTokens || na < 1 || na > qgp::kPfMaxSlices ||
        (b && (nb < 1 || nb > qgp::kPfMaxSlices)) || (mode == 2 && !b) || lda % 4 != 0 || sstride % 4 != 0 ||
        ((uintptr_t)a & 15u) || ((uintptr_t)b & 15u) || ((uintptr_t)sum_out & 15u))
        return -1;
    const uint32_t pieces = (uint32_t)(n / 8);
    // mode 1: one workgroup per token (up to 1024 threads); else 256-thread
    // workgroups over the pieces
    uint32_t block = qgp::kPfPlanesBlock, gx = (pieces + block - 1) / block;
    if (mode == 1) {
        block = pieces < 1024u ? (pieces + 63u) / 64u * 64u : 1024u;
        gx = 1;
    }
    hipLaunchKernelGGL(qgp::pf_planes_k, dim3(gx, ntok), dim3(block), 0, (hipStream_t)stream, a, na, b, nb,
                       (uint64_t)sstride, sum_out, nw, eps, (uint32_t)n, (uint32_t)lda, (uint32_t)mode, xp, rec,
                       ntok);
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

int launch_pf_qkv_post(float *qkv, uint32_t ldq, uint32_t ns, size_t sstride, const float *bq, const float *bk,
                       const float *bv, float *kc, float *vc, const float *cos_t, const float *sin_t, uint32_t q_dim,
                       uint32_t kv_dim, uint32_t hd, uint32_t pos0, uint32_t slot0, uint32_t ntok,
                       ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    if (ns < 1 || ns > qgp::kPfMaxSlices || ntok > kPfMaxTokens || hd % 2 != 0) return -1;
    const uint32_t pairs = (q_dim > kv_dim ? q_dim : kv_dim) / 2;
    hipLaunchKernelGGL(qgp::pf_qkv_post_k, dim3((pairs + 255) / 256, ntok), dim3(256), 0, (hipStream_t)stream, qkv,
                       ldq, ns, (uint64_t)sstride, bq, bk, bv, kc, vc, cos_t, sin_t, q_dim, kv_dim, hd, pos0, slot0);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_pf_attention(const float *qkv, uint32_t ldq, const float *kc, const float *vc, float *out, uint32_t n_heads,
                        uint32_t hd, uint32_t kv_dim, uint32_t n_rep, float scale, uint32_t slot0, uint32_t ntok,
                        size_t lds, ihipStream_t *stream)
{
    if (ntok == 0) return 0;
    hipLaunchKernelGGL(qgp::pf_attention_k, dim3(n_heads, ntok), dim3(256), lds, (hipStream_t)stream, qkv, ldq, kc, vc,
                       out, hd, kv_dim, n_rep, scale, slot0);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace qg
