// qg_model.hip -- the decode step of yudono/rust-inference on device
// (include/qgmodel.h).
//
// Every tensor stays in HBM for the whole generation: the quantized weights
// (raw GGUF blocks, mat-vec'd by the library's GEMV), norms and biases, the
// f32 KV caches, the activations, the logits and the token history.  The
// per-token values (token id, position, cache slot) live in a device-side
// Step record that the kernels read when they run, so one forward pass is a
// fixed sequence of launches: it is captured once as a HIP graph and replayed
// per token.  In generate, the sampler appends its token to the history and
// advances the Step itself, so a decode step needs no host round trip.
//
// Kernels (all f32, -ffp-contract=off: every product and sum is rounded where
// the reference rounds it, except that reductions add in tree order and the
// attention softmax is split over position ranges):
//   RMSNorm          math.rs:237-257 (RmsNorm::forward), inside the next GEMV
//                    with the residual add of transformer.rs:31-46
//   attn_rope_split_k  attention.rs:66-121 for head_dim 64/128/256: bias
//                    add, RoPE on q and k (rope.rs:88-96, pairs 2i/2i+1), KV
//   attn_combine_k   append (kv_cache.rs:52-73), then attention over one range
//                    of positions for the query heads of one kv head; then the
//                    ranges' partial softmax sums are merged (math.rs:104-118
//                    rescaled)
//   qkv_post_k       the bias add, RoPE and KV append alone, and
//   attention_k      attention in one workgroup per head (other head_dim)
//   SiLU * up        mlp.rs:31-43, silu as math.rs:137-146, in the epilogue
//                    of the [gate; up] GEMV (gate and up rows paired), else
//                    inside the down GEMV's prologue or a separate kernel
//   sample_part_k    sampler.rs:109-127 then math.rs:328-339 over one range
//   sample_final_k   of the logits per workgroup; then the first maximum
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "qg_common.h"
#include "qg_internal.h"
#include "qgmodel.h"

namespace qgm {

constexpr uint32_t kRecentMax = 64;       // model.rs:370-374 passes the last 64 tokens
constexpr uint32_t kSampleWG = 256;       // partial-argmax workgroups
constexpr uint32_t kMaxGroup = 8;         // query heads per attention workgroup
constexpr uint32_t kMaxSplit = 64;        // position ranges per head
constexpr uint32_t kMinLen = 8;           // positions per range (the last may hold fewer)

// Positions per range for seq cached positions; ranges = ceil(seq / len).
__host__ __device__ __forceinline__ uint32_t range_len(uint32_t seq, uint32_t nsplit)
{
    const uint32_t l = (seq + nsplit - 1) / nsplit;
    return l > kMinLen ? l : kMinLen;
}

// Per-token state read by the kernels: the token fed to the next forward
// pass, its position (RoPE) and its cache slot (number of cached positions).
struct Step {
    uint32_t token, pos, slot, pad;
};

// Sum / max over the 64 lanes of a full wave, returned to every lane.
// DPP steps (gfx9 controls: quad_perm 0xB1 / 0x4E, row_half_mirror 0x141,
// row_mirror 0x140, row_bcast15 0x142 into rows 1 and 3, row_bcast31 0x143
// into rows 2 and 3) leave the total in lane 63; rows outside a step's row
// mask are left as they are.
template <int CTRL, int ROW_MASK = 0xF> __device__ __forceinline__ float dppf(float v, float old)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 0xF, false));
}

__device__ __forceinline__ float lane63(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v)
{
    v += dppf<0xB1>(v, 0.f);
    v += dppf<0x4E>(v, 0.f);
    v += dppf<0x141>(v, 0.f);
    v += dppf<0x140>(v, 0.f);
    v += dppf<0x142, 0xA>(v, 0.f);
    v += dppf<0x143, 0xC>(v, 0.f);
    return lane63(v);
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dppf<0xB1>(v, v));
    v = fmaxf(v, dppf<0x4E>(v, v));
    v = fmaxf(v, dppf<0x141>(v, v));
    v = fmaxf(v, dppf<0x140>(v, v));
    v = fmaxf(v, dppf<0x142, 0xA>(v, v));
    v = fmaxf(v, dppf<0x143, 0xC>(v, v));
    return lane63(v);
}

// Sum / max over a workgroup of whole waves (every thread gets the result).
__device__ float block_sum(float v, float *red)
{
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

__device__ float block_max(float v, float *red)
{
    v = wave_max(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

// One thread per (2i, 2i+1) pair of q (q_dim/2 pairs) and of k/v (kv_dim/2).
__global__ void __launch_bounds__(256) qkv_post_k(float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, const float *__restrict__ bq,
                                                  const float *__restrict__ bk, const float *__restrict__ bv,
                                                  float *__restrict__ kc, float *__restrict__ vc,
                                                  const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                  uint32_t q_dim, uint32_t kv_dim, uint32_t hd,
                                                  const Step *__restrict__ st)
{
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x, half = hd / 2;
    const uint32_t pos = st->pos, slot = st->slot;
    const uint32_t i0 = 2 * t;
    if (i0 < q_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[pos * half + j], s = sin_t[pos * half + j];
        const float x0 = q[i0] + bq[i0], x1 = q[i0 + 1] + bq[i0 + 1];
        q[i0] = x0 * c - x1 * s;
        q[i0 + 1] = x0 * s + x1 * c;
    }
    if (i0 < kv_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[pos * half + j], s = sin_t[pos * half + j];
        const float x0 = k[i0] + bk[i0], x1 = k[i0 + 1] + bk[i0 + 1];
        float *kr = kc + (size_t)slot * kv_dim, *vr = vc + (size_t)slot * kv_dim;
        kr[i0] = x0 * c - x1 * s;
        kr[i0 + 1] = x0 * s + x1 * c;
        vr[i0] = v[i0] + bv[i0];
        vr[i0 + 1] = v[i0 + 1] + bv[i0 + 1];
    }
}

// Arguments of the split attention kernel.
struct AttnArgs {
    const float *q, *k, *v;          // this token's projections, before bias and RoPE
    const float *bq, *bk, *bv;
    float *kc, *vc;                  // the layer's cache, [max_seq_len][kv_dim]
    const float *cos_t, *sin_t;      // [max_seq_len][head_dim / 2]
    float *part, *ml;                // per (head, range): partial output, (max, sum)
    const Step *st;
    uint32_t kv_dim, n_rep, grp, nsplit;
    uint32_t cap;                    // rows of the cache (max_seq_len)
    float scale;
    // attn_rope_head_k<E, 2>: floats between the ranges' outputs in part (q_dim)
    // and between their (max, sum) rows in ml (2 n_heads)
    uint32_t part_stride, ml_stride;
};

// Element d of a head after RoPE (rope.rs: the pair (2i, 2i+1) turned by
// pos * theta_i); `self` is element d, `other` its partner d ^ 1, cs / sn the
// position's rows of the tables.  The same expressions as qkv_post_k.
__device__ __forceinline__ float rope1(float self, float other, uint32_t d, float c, float s)
{
    // even d: self c - other s; odd d: other s + self c (= self c + other s)
    const float p0 = self * c, p1 = other * s;
    return p0 + ((d & 1u) ? p1 : -p1);
}

// Attention of the token at st->pos over positions [j0, j1) of the
// seq = slot + 1 cached ones, for the `grp` query heads h0 .. h0 + grp - 1
// that share one kv head (head_dim = 64 * E), with the projections'
// post-processing folded in: q, k, v biases (attention.rs:66-76), RoPE of q
// and k (attention.rs:78-87) and the cache append at `slot`
// (attention.rs:89-90, kv_cache.rs:52-73).  The range that holds `slot` uses
// this token's k and v from registers, and its first head group of each kv
// head stores them to the cache, so no other workgroup reads the slot being
// written.
//
// (Merging the ranges in the last workgroup to finish, behind a device-scope
// counter, measured slower than the separate merge kernel: the fences that
// make the partial sums visible across the XCDs' L2 caches cost more than the
// launch.)
//
// Workgroup (head group, range): 4 waves, each lane owns dimensions
// lane + 64 e (every K and V row is one coalesced read shared by the group's
// heads).  A wave takes positions j0 + wave + 4 p in chunks of kPW, all K and
// V rows of a chunk loaded before any use, with a running (max, sum, output)
// per head (the softmax of attention.rs:101-119 over the wave's positions);
// the four waves are merged in LDS.  Writes the unnormalised partial output
// sum_j exp(s_j - m) v_j and (m, l = sum_j exp(s_j - m)) of the range;
// workgroups whose range starts past seq exit.
// Positions per wave per chunk: the chunk's code is unrolled over heads and
// positions, and a larger chunk made the kernel slower (straight-line code
// fetched cold by every workgroup) while short ranges fill only one chunk.
constexpr uint32_t kPW = 2;
template <int E>
__global__ void __launch_bounds__(256) attn_rope_split_k(AttnArgs a)
{
    constexpr uint32_t HD = 64 * E;
    __shared__ float sacc[4][kMaxGroup][HD];
    __shared__ float sml[4][kMaxGroup][2];
    // wave index as a uniform value: the position loop's bounds depend on it,
    // and a per-lane value would turn every branch on them into exec masking
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t grp = a.grp, split = blockIdx.x % a.nsplit, h0 = (blockIdx.x / a.nsplit) * grp;
    const uint32_t kvo = (h0 / a.n_rep) * HD;
    // Every load below is unconditional (clamped indices, selects after the
    // loads): a load behind a branch waits for everything issued before it.
    // The projections do not depend on the step record, so they are in flight
    // while it arrives.
    float qv[kMaxGroup][E], kn[E], vn[E];
#pragma unroll
    for (uint32_t r = 0; r < kMaxGroup; r++)
#pragma unroll
        for (int e = 0; e < E; e++) {
            const uint32_t i = (h0 + (r < grp ? r : 0u)) * HD + lane + 64 * e;
            qv[r][e] = a.q[i] + a.bq[i];
        }
#pragma unroll
    for (int e = 0; e < E; e++) {
        kn[e] = a.k[kvo + lane + 64 * e] + a.bk[kvo + lane + 64 * e];
        vn[e] = a.v[kvo + lane + 64 * e] + a.bv[kvo + lane + 64 * e];
    }
    const uint32_t pos = a.st->pos, slot = a.st->slot, seq = slot + 1;
    const uint32_t len = range_len(seq, a.nsplit);
    const uint32_t j0 = split * len, j1 = min(seq, j0 + len);
    // K and V rows of this wave's positions j0 + wave + 4 p, kPW at a time,
    // clamped into the cache rows that exist (a workgroup past seq loads and
    // exits); the next chunk is in flight while one is used
    float kk[kPW][E], vv[kPW][E], nk[kPW][E], nv[kPW][E];
    auto load = [&](uint32_t b, float (&ko)[kPW][E], float (&vo)[kPW][E]) {
#pragma unroll
        for (uint32_t p = 0; p < kPW; p++) {
            const uint32_t j = min(b + 4 * p, slot);
            const float *kr = a.kc + (size_t)j * a.kv_dim + kvo, *vr = a.vc + (size_t)j * a.kv_dim + kvo;
#pragma unroll
            for (int e = 0; e < E; e++) {
                ko[p][e] = kr[lane + 64 * e];
                vo[p][e] = vr[lane + 64 * e];
            }
        }
    };
    uint32_t base = j0 + wave;
    load(base, kk, vv);
    // cos / sin of this lane's pairs (the table rows of `pos`)
    float cv[E], sv[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        cv[e] = a.cos_t[(size_t)pos * (HD / 2) + ((lane + 64 * e) >> 1)];
        sv[e] = a.sin_t[(size_t)pos * (HD / 2) + ((lane + 64 * e) >> 1)];
    }
#pragma unroll
    for (uint32_t r = 0; r < kMaxGroup; r++)
#pragma unroll
        for (int e = 0; e < E; e++) {
            const float o = __shfl_xor(qv[r][e], 1, 64);
            qv[r][e] = r < grp ? rope1(qv[r][e], o, lane + 64 * e, cv[e], sv[e]) : 0.f;
        }
#pragma unroll
    for (int e = 0; e < E; e++) kn[e] = rope1(kn[e], __shfl_xor(kn[e], 1, 64), lane + 64 * e, cv[e], sv[e]);
    if (j0 >= seq) return;
    const bool has_new = j1 == seq;
    if (has_new && h0 % a.n_rep == 0 && wave == 0) {
        float *kr = a.kc + (size_t)slot * a.kv_dim + kvo, *vr = a.vc + (size_t)slot * a.kv_dim + kvo;
#pragma unroll
        for (int e = 0; e < E; e++) {
            kr[lane + 64 * e] = kn[e];
            vr[lane + 64 * e] = vn[e];
        }
    }
    float m[kMaxGroup], l[kMaxGroup], acc[kMaxGroup][E];
#pragma unroll
    for (uint32_t r = 0; r < kMaxGroup; r++) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) acc[r][e] = 0.f;
    }
    for (; base < j1; base += 4 * kPW) {
        const uint32_t np = min((j1 - base + 3) / 4, kPW);   // this wave's positions in the chunk
        if (base + 4 * kPW < j1) load(base + 4 * kPW, nk, nv);
        // the slot being appended comes from registers (its cache row is written above)
#pragma unroll
        for (uint32_t p = 0; p < kPW; p++)
            if (base + 4 * p == slot)
#pragma unroll
                for (int e = 0; e < E; e++) { kk[p][e] = kn[e]; vv[p][e] = vn[e]; }
#pragma unroll
        for (uint32_t r = 0; r < kMaxGroup; r++) {
            if (r >= grp) break;
            float sc[kPW], cm = -INFINITY;
#pragma unroll
            for (uint32_t p = 0; p < kPW; p++) {
                if (p >= np) break;
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < E; e++) t += qv[r][e] * kk[p][e];
                sc[p] = wave_sum(t) * a.scale;
                cm = fmaxf(cm, sc[p]);
            }
            const float mn = fmaxf(m[r], cm);
            const float al = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
            float ls = 0.f, o[E];
#pragma unroll
            for (int e = 0; e < E; e++) o[e] = 0.f;
#pragma unroll
            for (uint32_t p = 0; p < kPW; p++) {
                if (p >= np) break;
                const float ex = expf(sc[p] - mn);
                ls += ex;
#pragma unroll
                for (int e = 0; e < E; e++) o[e] += ex * vv[p][e];
            }
            l[r] = l[r] * al + ls;
#pragma unroll
            for (int e = 0; e < E; e++) acc[r][e] = acc[r][e] * al + o[e];
            m[r] = mn;
        }
#pragma unroll
        for (uint32_t p = 0; p < kPW; p++)
#pragma unroll
            for (int e = 0; e < E; e++) { kk[p][e] = nk[p][e]; vv[p][e] = nv[p][e]; }
    }
#pragma unroll
    for (uint32_t r = 0; r < kMaxGroup; r++) {
        if (r >= grp) break;
#pragma unroll
        for (int e = 0; e < E; e++) sacc[wave][r][lane + 64 * e] = acc[r][e];
        if (lane == 0) { sml[wave][r][0] = m[r]; sml[wave][r][1] = l[r]; }
    }
    __syncthreads();
    // merge the waves: weights exp(m_w - M) (0 for a wave without positions)
    for (uint32_t i = threadIdx.x; i < grp * HD; i += blockDim.x) {
        const uint32_t r = i / HD, d = i % HD;
        float mx = sml[0][r][0];
#pragma unroll
        for (int w = 1; w < 4; w++) mx = fmaxf(mx, sml[w][r][0]);
        float sum = 0.f, lsum = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = sml[w][r][0];
            const float f = mw == -INFINITY ? 0.f : expf(mw - mx);
            sum += f * sacc[w][r][d];
            lsum += f * sml[w][r][1];
        }
        const size_t o = (size_t)(h0 + r) * a.nsplit + split;
        a.part[o * HD + d] = sum;
        if (d == 0) {
            a.ml[2 * o] = mx;
            a.ml[2 * o + 1] = lsum;
        }
    }
}

// out[h] = sum_s w_s part_s with w_s = exp(m_s - max m) / sum_s exp(m_s - max m) l_s:
// the softmax-weighted sum of v over all positions.  One workgroup per head;
// wave 0 derives the weights of the ranges in use.
__global__ void __launch_bounds__(256) attn_combine_k(const float *__restrict__ part, const float *__restrict__ ml,
                                                      float *__restrict__ out, const Step *__restrict__ st,
                                                      uint32_t hd, uint32_t nsplit)
{
    __shared__ float wt[kMaxSplit];
    const uint32_t h = blockIdx.x, seq = st->slot + 1;
    const uint32_t len = range_len(seq, nsplit), nr = (seq + len - 1) / len;
    const float *m = ml + (size_t)h * nsplit * 2;
    if (threadIdx.x < 64) {
        const uint32_t s = threadIdx.x;
        const float ms = s < nr ? m[2 * s] : -INFINITY, ls = s < nr ? m[2 * s + 1] : 0.f;
        const float mx = wave_max(ms);
        const float w = s < nr ? expf(ms - mx) : 0.f;
        const float l = wave_sum(w * ls);
        wt[s] = w / l;
    }
    __syncthreads();
    const float *p = part + (size_t)h * nsplit * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
        for (uint32_t s = 0; s < nr; s++) acc += wt[s] * p[(size_t)s * hd + d];
        out[h * hd + d] = acc;
    }
}

// Short contexts: the whole attention of query head blockIdx.x in one
// workgroup, with the projections' post-processing of attn_rope_split_k
// (biases, RoPE of q and k, the cache append at `slot` by the first query
// head of each kv head, this token's k and v from registers at `slot`).
// kHeadWaves waves take positions wave + kHeadWaves p in chunks of 8 (4 for
// head_dim 256: one chunk, or a few, per wave up to kShortSeq positions, all
// its K and V rows loaded before any use) with a running (max, sum, output)
// each, merged in LDS into the normalised output row (math.rs:104-118 over
// all positions).  One launch, no partial sums: at a few hundred cached
// positions the split kernel's second launch and its reads of the partials
// cost more than the positions per wave here.
//
// NR = 2: two workgroups per head, workgroup (h, r) taking the positions
// j = r (mod 2) -- twice the CUs, each reading half the K and V rows, which is
// what bounds the kernel -- and writing its range's unnormalised output and
// (max, sum of exponentials) instead, range-major: part[r * q_dim + h * hd + d],
// ml[2 (r * n_heads + h) + {0, 1}].  The consumer (the wo GEMV's input
// prologue, launch_gemv_attn) merges the two ranges.  Chunks of 4 positions
// per wave there: a workgroup then loads the rows of about the positions it
// has, 64 at a time, instead of 128 (decode +0.4 %).
constexpr uint32_t kHeadWaves = 16;
// cached positions up to which the forward pass uses attn_rope_head_k
constexpr uint32_t kShortSeq = 512;
template <int E, int NR = 1>
__global__ void __launch_bounds__(64 * kHeadWaves) attn_rope_head_k(AttnArgs a, float *__restrict__ out)
{
    static_assert(NR == 1 || NR == 2, "one or two position ranges");
    // positions per wave per chunk
    constexpr uint32_t HD = 64 * E, NW = kHeadWaves, PW = E <= 2 && NR == 1 ? 8u : 4u;
    constexpr uint32_t ST = NR * NW;                 // position stride between a wave's positions
    __shared__ float sacc[NW][HD];
    __shared__ float sml[NW][2];
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t h = blockIdx.x / NR, rg = blockIdx.x % NR, kvo = (h / a.n_rep) * HD;
    // unconditional loads; the projections are in flight while the step record arrives
    float qv[E], kn[E], vn[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t i = h * HD + lane + 64 * e;
        qv[e] = a.q[i] + a.bq[i];
        kn[e] = a.k[kvo + lane + 64 * e] + a.bk[kvo + lane + 64 * e];
        vn[e] = a.v[kvo + lane + 64 * e] + a.bv[kvo + lane + 64 * e];
    }
    float kk[PW][E], vv[PW][E], nk[PW][E], nv[PW][E];
    auto load = [&](uint32_t b, uint32_t last, float (&ko)[PW][E], float (&vo)[PW][E]) {
#pragma unroll
        for (uint32_t p = 0; p < PW; p++) {
            const uint32_t j = min(b + ST * p, last);
            const float *kr = a.kc + (size_t)j * a.kv_dim + kvo, *vr = a.vc + (size_t)j * a.kv_dim + kvo;
#pragma unroll
            for (int e = 0; e < E; e++) {
                ko[p][e] = kr[lane + 64 * e];
                vo[p][e] = vr[lane + 64 * e];
            }
        }
    };
    // the first chunk's rows, before the step record arrives (clamped to the
    // cache: rows past slot are never used -- the chunk's loop stops at the
    // wave's last position -- and the one at slot is replaced by this
    // token's k and v)
    uint32_t base = rg + NR * wave;
    load(base, a.cap - 1u, kk, vv);
    const uint32_t pos = a.st->pos, slot = a.st->slot, seq = slot + 1;
    float cv[E], sv[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        cv[e] = a.cos_t[(size_t)pos * (HD / 2) + ((lane + 64 * e) >> 1)];
        sv[e] = a.sin_t[(size_t)pos * (HD / 2) + ((lane + 64 * e) >> 1)];
    }
#pragma unroll
    for (int e = 0; e < E; e++) {
        qv[e] = rope1(qv[e], __shfl_xor(qv[e], 1, 64), lane + 64 * e, cv[e], sv[e]);
        kn[e] = rope1(kn[e], __shfl_xor(kn[e], 1, 64), lane + 64 * e, cv[e], sv[e]);
    }
    if (h % a.n_rep == 0 && rg == 0 && wave == 0) {
        float *kr = a.kc + (size_t)slot * a.kv_dim + kvo, *vr = a.vc + (size_t)slot * a.kv_dim + kvo;
#pragma unroll
        for (int e = 0; e < E; e++) {
            kr[lane + 64 * e] = kn[e];
            vr[lane + 64 * e] = vn[e];
        }
    }
    float m = -INFINITY, l = 0.f, acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;
    for (; base < seq; base += ST * PW) {
        const uint32_t np = min((seq - base + ST - 1) / ST, PW);   // this wave's positions in the chunk
        if (base + ST * PW < seq) load(base + ST * PW, slot, nk, nv);
#pragma unroll
        for (uint32_t p = 0; p < PW; p++)
            if (base + ST * p == slot)
#pragma unroll
                for (int e = 0; e < E; e++) { kk[p][e] = kn[e]; vv[p][e] = vn[e]; }
        float sc[PW], cm = -INFINITY;
#pragma unroll
        for (uint32_t p = 0; p < PW; p++) {
            if (p >= np) break;
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < E; e++) t += qv[e] * kk[p][e];
            sc[p] = wave_sum(t) * a.scale;
            cm = fmaxf(cm, sc[p]);
        }
        const float mn = fmaxf(m, cm);
        const float al = m == -INFINITY ? 0.f : expf(m - mn);
        float ls = 0.f, o[E];
#pragma unroll
        for (int e = 0; e < E; e++) o[e] = 0.f;
#pragma unroll
        for (uint32_t p = 0; p < PW; p++) {
            if (p >= np) break;
            const float ex = expf(sc[p] - mn);
            ls += ex;
#pragma unroll
            for (int e = 0; e < E; e++) o[e] += ex * vv[p][e];
        }
        l = l * al + ls;
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] = acc[e] * al + o[e];
        m = mn;
#pragma unroll
        for (uint32_t p = 0; p < PW; p++)
#pragma unroll
            for (int e = 0; e < E; e++) { kk[p][e] = nk[p][e]; vv[p][e] = nv[p][e]; }
    }
#pragma unroll
    for (int e = 0; e < E; e++) sacc[wave][lane + 64 * e] = acc[e];
    if (lane == 0) { sml[wave][0] = m; sml[wave][1] = l; }
    __syncthreads();
    // merge the waves: weights exp(m_w - M) (0 for a wave without positions),
    // derived once by the first kHeadWaves lanes, over their sum (NR = 2:
    // unnormalised, the sum goes out with M)
    __shared__ float swt[NW];
    if (threadIdx.x < NW) {
        const uint32_t w = threadIdx.x;
        float mx = sml[0][0];
#pragma unroll
        for (uint32_t v = 1; v < NW; v++) mx = fmaxf(mx, sml[v][0]);
        const float mw = sml[w][0];
        const float f = mw == -INFINITY ? 0.f : expf(mw - mx);
        float lsum = f * sml[w][1];
#pragma unroll
        for (uint32_t o = 1; o < NW; o <<= 1) lsum += __shfl_xor(lsum, o, 64);
        if constexpr (NR == 1) {
            swt[w] = f / lsum;
        } else {
            swt[w] = f;
            if (w == 0) {
                const size_t o = (size_t)rg * (a.ml_stride / 2) + h;
                a.ml[2 * o] = mx;
                a.ml[2 * o + 1] = lsum;
            }
        }
    }
    __syncthreads();
    float *dst = NR == 1 ? out + h * HD : a.part + (size_t)rg * a.part_stride + h * HD;
    for (uint32_t d = threadIdx.x; d < HD; d += blockDim.x) {
        float sum = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) sum += swt[w] * sacc[w][d];
        dst[d] = sum;
    }
}

// One workgroup per query head for any even head_dim; LDS: hd floats of q,
// max_seq_len floats of scores.
__global__ void __launch_bounds__(256) attention_k(const float *__restrict__ q, const float *__restrict__ kc,
                                                   const float *__restrict__ vc, float *__restrict__ out,
                                                   const Step *__restrict__ st, uint32_t hd, uint32_t kv_dim,
                                                   uint32_t n_rep, float scale)
{
    extern __shared__ float sm[];
    __shared__ float red[4];
    float *qs = sm, *sc = sm + hd;
    const uint32_t seq = st->slot + 1;
    const uint32_t h = blockIdx.x, kvh = (h / n_rep) * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = q[h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float *kr = kc + (size_t)j * kv_dim + kvh;
        float s = 0.f;
        for (uint32_t d = 0; d < hd; d++) s += qs[d] * kr[d];             // math.rs:63-70
        s = s * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float sum = 0.f;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) sc[j] *= inv;
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
        for (uint32_t j = 0; j < seq; j++) acc += sc[j] * vc[(size_t)j * kv_dim + kvh + d];
        out[h * hd + d] = acc;
    }
}

// Greedy sampler.  The recent tokens are either an explicit list (recent,
// n_recent) or, in generate, the last min(window, 64) entries of the token
// history hist[0 .. slot + 1).
struct SampleArgs {
    float *logits;
    uint32_t n;
    const uint32_t *recent;
    uint32_t n_recent;
    uint32_t *hist;              // generate: history (NULL: explicit list)
    uint32_t window;
    float penalty;
    Step *st;
    float *pv;                   // per-workgroup maximum and its index
    uint32_t *pi;
    uint32_t *token;             // the sampled token
};

// (value, index) max with the smaller index on ties, over one wave
__device__ __forceinline__ void argmax_wave(float &best, uint32_t &idx)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(idx, o, 64);
        if (oi != 0xFFFFFFFFu && (idx == 0xFFFFFFFFu || ov > best || (ov == best && oi < idx))) {
            best = ov; idx = oi;
        }
    }
}

// (value, index) of the first maximum over [lo, hi) after the repetition
// penalty of the tokens in this range (sampler.rs:109-127: in list order, each
// occurrence again).  Occurrences of different tokens do not interact, so lane
// r of wave 0 applies all k occurrences of token r where r is its first
// occurrence, in the order the sequential loop applies them.  NaN never wins.
__global__ void __launch_bounds__(256) sample_part_k(SampleArgs a)
{
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t per = (a.n + gridDim.x - 1) / gridDim.x;
    const uint32_t lo = blockIdx.x * per, hi = min(a.n, lo + per);
    if (threadIdx.x < 64 && a.penalty != 1.0f) {                   // sampler.rs:76-78
        const uint32_t *rc = a.recent;
        uint32_t nr = a.n_recent;
        if (a.hist) {
            const uint32_t cnt = a.st->slot + 1, w = min(min(a.window, kRecentMax), cnt);
            rc = a.hist + (cnt - w);
            nr = w;
        }
        const uint32_t r = threadIdx.x;
        const uint32_t t = r < nr ? rc[r] : 0xFFFFFFFFu;
        uint32_t k = 0;
        bool first = true;
        for (uint32_t j = 0; j < nr; j++) {
            const uint32_t u = __shfl(t, (int)j, 64);
            k += u == t;
            first = first && !(u == t && j < r);
        }
        if (r < nr && first && t >= lo && t < hi) {
            float l = a.logits[t];
            for (uint32_t i = 0; i < k; i++) l = l > 0.0f ? l / a.penalty : l * a.penalty;
            a.logits[t] = l;
        }
    }
    __syncthreads();
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        const float v = a.logits[i];
        if (v > best || (idx == 0xFFFFFFFFu && v == best)) { best = v; idx = i; }
    }
    argmax_wave(best, idx);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = -INFINITY;
        uint32_t id = 0xFFFFFFFFu;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) {
            if (bi[i] == 0xFFFFFFFFu) continue;
            if (id == 0xFFFFFFFFu || bv[i] > b || (bv[i] == b && bi[i] < id)) { b = bv[i]; id = bi[i]; }
        }
        a.pv[blockIdx.x] = b;
        a.pi[blockIdx.x] = id;
    }
}

// The first maximum over the ranges (math.rs:328-339: a NaN at index 0
// returns 0, as the reference's strict ">" scan does).  In generate the token
// is appended to the history and becomes the next step's token.  One wave:
// lane l scans ranges l, l + 64, ... in order; ranges hold increasing indices,
// so ties go to the smaller index.  (A single launch whose last workgroup
// takes this maximum needs device-scope fences to publish the ranges across
// the XCDs' L2 caches; measured slower than the second launch.)
__global__ void __launch_bounds__(64) sample_final_k(SampleArgs a, uint32_t nparts)
{
    float b = -INFINITY;
    uint32_t id = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < nparts; i += 64) {
        const float v = a.pv[i];
        const uint32_t j = a.pi[i];
        if (j != 0xFFFFFFFFu && (id == 0xFFFFFFFFu || v > b)) { b = v; id = j; }
    }
    argmax_wave(b, id);
    if (threadIdx.x != 0) return;
    const float l0 = a.logits[0];
    const uint32_t tok = (l0 != l0 || id == 0xFFFFFFFFu) ? 0u : id;
    *a.token = tok;
    if (a.hist) {
        Step *s = a.st;
        const uint32_t n = s->slot + 1;
        a.hist[n] = tok;
        s->slot = n;
        s->pos += 1;
        s->token = tok;
    }
}

// Prefill: the next step feeds the next history token.
__global__ void advance_k(Step *st, const uint32_t *hist)
{
    if (threadIdx.x == 0) {
        st->slot += 1;
        st->pos += 1;
        st->token = hist[st->slot];
    }
}

}  // namespace qgm

// ----------------------------------------------------------------- engine

namespace {
constexpr int kSlots = 7;                 // WQ .. DOWN
constexpr uint32_t kRing = 256;           // pinned Step records for host-fed forwards
}

struct qg_model {
    qg_ctx *ctx = nullptr;
    qg_model_config cfg{};
    uint32_t hd = 0, q_dim = 0, kv_dim = 0, n_rep = 0;
    uint32_t att_grp = 0, att_nsplit = 0;   // split attention (head_dim 64, 128, 256)
    size_t att_lds = 0;                     // LDS of the one-workgroup-per-head kernel
    qg_mat *tok = nullptr, *lm = nullptr;
    // a slot holds a matrix the model owns (set_matrix), one it shares
    // (share_matrix: counted in qg_mat::shares), or -- lm only -- an alias of
    // tok (a tied output, neither owned nor shared)
    bool tok_owned = false, lm_owned = false, tok_shared = false, lm_shared = false;
    std::vector<qg_mat *> w[kSlots];
    std::vector<bool> owned[kSlots];
    float *final_norm = nullptr;
    std::vector<float *> vec[6];          // per layer: attn_norm, ffn_norm, bq, bk, bv (slot 0 unused)
    float *kc = nullptr, *vc = nullptr;   // [n_layers][max_seq_len][kv_dim]
    size_t seq = 0;
    float *cos_t = nullptr, *sin_t = nullptr;
    float *h0 = nullptr, *h1 = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *ao = nullptr, *ao2 = nullptr, *g = nullptr, *u = nullptr, *hb = nullptr, *fo = nullptr;
    float *logits = nullptr;
    float *zeros = nullptr;               // the residual addend of the first layer
    float *att_part = nullptr, *att_ml = nullptr;
    // per layer: [Q;K;V] (n = 3) or [Q;K] (n = 2) stacked into one matrix
    // when the parts share a type, and [gate;up]; the outputs q,k,v and g,u
    // are contiguous, so one mat-vec fills them.  Built before the first
    // forward pass after any matrix change.
    std::vector<qg_mat *> f_qkv, f_gu;
    std::vector<uint8_t> f_qkv_n;
    bool fused_ready = false;
    float *s_pv = nullptr;
    uint32_t *s_pi = nullptr;
    uint32_t *d_recent = nullptr, *d_token = nullptr, *d_hist = nullptr;
    qgm::Step *d_step = nullptr;
    uint32_t *h_recent = nullptr, *h_token = nullptr;   // pinned
    qgm::Step *h_steps = nullptr;                       // pinned ring
    uint32_t ring = 0;
    bool use_graphs = true;
    // batched prefill (qg_prefill.hip): per chunk of up to kPfMaxTokens tokens,
    // the residual stream (two buffers, read one / write the other), q|k|v,
    // attention output, wo output, [gate|up] and down outputs of every token
    // (the GEMM outputs with room for their K-split slices: pf_s* slices of
    // kPfMaxTokens rows each), the last token's summed down output, the x
    // planes / records of the GEMMs and the prompt's token ids; allocated on
    // first use
    bool pf_batched = true;
    float *pf_h[2] = {nullptr, nullptr}, *pf_qkv = nullptr, *pf_ao = nullptr, *pf_ao2 = nullptr,
          *pf_g = nullptr, *pf_fo = nullptr, *pf_last = nullptr;
    uint16_t *pf_xp = nullptr;
    float *pf_rec = nullptr, *pf_ss = nullptr;
    uint32_t *pf_tok = nullptr;
    uint32_t pf_s_qkv = 1, pf_s_o = 1, pf_s_gu = 1, pf_s_down = 1;
    // the QKV output's K splits: [Q; K; V] in one launch (one type), or
    // [Q; K] and V in two (V another type: its few row tiles take more slices)
    uint32_t pf_s_qkv1 = 1, pf_s_qk = 1, pf_s_v = 1;
    // captured graphs per attention mode: [0] the split attention
    // (attn_rope_split_k + attn_combine_k), [1] whole heads in one workgroup
    // each (attn_rope_head_k), [2] two position ranges per head merged in the
    // wo GEMV's input (attn_rope_head_k<E, 2> + launch_gemv_attn); att_mode
    // selects what enqueue_forward launches
    hipGraphExec_t g_fwd[3] = {nullptr, nullptr, nullptr};   // forward pass
    hipGraphExec_t g_dec[3] = {nullptr, nullptr, nullptr};   // sample + advance + forward (generate)
    int att_mode = 0;
    int att_path = 0;                     // qg_model_set_attention_path
    float g_dec_penalty = 0.f;
    uint32_t g_dec_window = 0;
    std::vector<void *> allocs;
    size_t alloc_bytes = 0;               // device bytes of allocs
};

namespace {

int mfail(qg_model *m, int st, const char *what, hipError_t e = hipSuccess)
{
    return qg_fail(m ? m->ctx : nullptr, st, what, e);
}

#define QGM_HIP(m, call)                                                      \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) return mfail((m), QG_ERR_HIP, #call, e_);       \
    } while (0)

template <class T> int dalloc(qg_model *m, T **p, size_t n)
{
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, (n ? n : 1) * sizeof(T));
    if (e != hipSuccess) return mfail(m, QG_ERR_OUT_OF_MEMORY, "hipMalloc", e);
    e = hipMemset(d, 0, (n ? n : 1) * sizeof(T));
    if (e != hipSuccess) { (void)hipFree(d); return mfail(m, QG_ERR_HIP, "hipMemset", e); }
    m->allocs.push_back(d);
    m->alloc_bytes += (n ? n : 1) * sizeof(T);
    *p = (T *)d;
    return QG_OK;
}

void drop_graphs(qg_model *m)
{
    for (int i = 0; i < 3; i++) {
        if (m->g_fwd[i]) (void)hipGraphExecDestroy(m->g_fwd[i]);
        if (m->g_dec[i]) (void)hipGraphExecDestroy(m->g_dec[i]);
        m->g_fwd[i] = m->g_dec[i] = nullptr;
    }
}

// Frees the stacked matrices.  Parts that are views into them (qg_stack_views)
// first get their own copies back (restore), unless the model is being freed
// with them.  A stack whose parts could not all get their copies back (an
// allocation failed) stays: its remaining views still point into it, and
// prepare() keeps it rather than stacking those parts again.
int drop_fused(qg_model *m, bool restore = true)
{
    int rc = QG_OK;
    for (size_t l = 0; l < m->f_qkv.size(); l++) {
        if (m->f_qkv[l]) {
            int r = QG_OK;
            for (int i = 0; i < m->f_qkv_n[l] && restore; i++) {
                const int ri = qg_mat_unview(m->ctx, m->w[QG_M_WQ - 2 + i][l]);
                r = r ? r : ri;
            }
            if (r == QG_OK) {
                qg_mat_free(m->ctx, m->f_qkv[l]);
                m->f_qkv[l] = nullptr;
                m->f_qkv_n[l] = 0;
            }
            rc = rc ? rc : r;
        }
        if (m->f_gu[l]) {
            int r = QG_OK;
            for (int s : {QG_M_GATE - 2, QG_M_UP - 2})
                if (restore) {
                    const int ri = qg_mat_unview(m->ctx, m->w[s][l]);
                    r = r ? r : ri;
                }
            if (r == QG_OK) {
                qg_mat_free(m->ctx, m->f_gu[l]);
                m->f_gu[l] = nullptr;
            }
            rc = rc ? rc : r;
        }
    }
    m->fused_ready = false;
    return rc;
}

// One stacked matrix of parts (owned[i]: the model owns part i): the parts
// become views into it when the model owns them all and their layout allows
// (no second copy), else a stacked copy beside them.
int stack_parts(qg_model *m, qg_mat *const *parts, const bool *owned, int n, qg_mat **out)
{
    bool all = true;
    for (int i = 0; i < n; i++) all = all && owned[i];
    if (all) {
        const int rc = qg_stack_views(m->ctx, parts, n, out);
        if (rc != QG_ERR_SHAPE) return rc;
    }
    return qg_stack_mats(m->ctx, parts, n, out);
}

// parts stack into one matrix: same type and cols, all but the last a whole
// number of blocks
bool stackable(qg_mat *const *p, int n)
{
    for (int i = 0; i < n; i++) {
        if (p[i]->type != p[0]->type || p[i]->cols != p[0]->cols) return false;
        if (i + 1 < n && (p[i]->rows * p[i]->cols) % qg::block_elems(p[i]->type) != 0) return false;
    }
    return true;
}

int prepare(qg_model *m)
{
    // the embedding rows are read in the GGUF layout (dequantize_row); a
    // token_embd the model owns that is not also the lm_head needs no
    // repacked copy
    if (m->tok) {
        int rc;
        if ((rc = qg_mat_keep_gguf(m->ctx, m->tok))) return rc;
        if (m->tok_owned && m->lm != m->tok && m->tok->d_rp && (rc = qg_mat_drop_repacked(m->ctx, m->tok))) return rc;
    }
    if (m->fused_ready) return QG_OK;
    for (uint32_t l = 0; l < m->cfg.n_layers; l++) {
        qg_mat *qkv[3] = {m->w[QG_M_WQ - 2][l], m->w[QG_M_WK - 2][l], m->w[QG_M_WV - 2][l]};
        const int n = stackable(qkv, 3) ? 3 : stackable(qkv, 2) ? 2 : 0;
        const bool oq[3] = {m->owned[QG_M_WQ - 2][l], m->owned[QG_M_WK - 2][l], m->owned[QG_M_WV - 2][l]};
        int rc;
        // a stack kept by a drop_fused that could not restore every part
        // still holds exactly these parts' bytes
        if (!m->f_qkv[l]) {
            if (n && (rc = stack_parts(m, qkv, oq, n, &m->f_qkv[l]))) return rc;
            m->f_qkv_n[l] = (uint8_t)n;
        }
        qg_mat *gu[2] = {m->w[QG_M_GATE - 2][l], m->w[QG_M_UP - 2][l]};
        const bool og[2] = {m->owned[QG_M_GATE - 2][l], m->owned[QG_M_UP - 2][l]};
        if (!m->f_gu[l] && stackable(gu, 2) && (rc = stack_parts(m, gu, og, 2, &m->f_gu[l]))) return rc;
    }
    m->fused_ready = true;
    return QG_OK;
}

// lm is an alias of tok (a tied output): it holds no reference of its own
bool lm_alias(const qg_model *m) { return m->lm && m->lm == m->tok && !m->lm_owned && !m->lm_shared; }

void free_model(qg_model *m)
{
    m->ctx->models.erase(m);
    drop_graphs(m);
    (void)drop_fused(m, false);
    for (int s = 0; s < kSlots; s++)
        for (size_t l = 0; l < m->w[s].size(); l++)
            qg_mat_release(m->ctx, m->w[s][l], m->owned[s][l]);
    const bool alias = lm_alias(m);
    qg_mat_release(m->ctx, m->tok, m->tok_owned);
    if (!alias) qg_mat_release(m->ctx, m->lm, m->lm_owned);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->h_recent) (void)hipHostFree(m->h_recent);
    if (m->h_token) (void)hipHostFree(m->h_token);
    if (m->h_steps) (void)hipHostFree(m->h_steps);
    delete m;
}

// expected (rows, cols) of a slot
void slot_shape(const qg_model *m, uint32_t which, size_t *rows, size_t *cols)
{
    const size_t E = m->cfg.embed_dim, H = m->cfg.hidden_dim, V = m->cfg.vocab_size;
    switch (which) {
    case QG_M_TOKEN_EMBD: case QG_M_LM_HEAD: *rows = V; *cols = E; break;
    case QG_M_WQ: *rows = m->q_dim; *cols = E; break;
    case QG_M_WK: case QG_M_WV: *rows = m->kv_dim; *cols = E; break;
    case QG_M_WO: *rows = E; *cols = m->q_dim; break;
    case QG_M_GATE: case QG_M_UP: *rows = H; *cols = E; break;
    case QG_M_DOWN: *rows = E; *cols = H; break;
    default: *rows = *cols = 0;
    }
}

// Puts `mat` into slot (which, layer), owned by the model or shared (counted
// in mat->shares), releasing what the slot held.  A tied lm_head that aliases
// the token_embd being replaced takes over that matrix, as the reference's
// lm_head is a clone made at load time (model.rs:224-226).
void put_slot(qg_model *m, uint32_t which, uint32_t layer, qg_mat *mat, bool shared)
{
    if (shared) mat->shares++;
    if (which == QG_M_TOKEN_EMBD || which == QG_M_LM_HEAD) {
        if (which == QG_M_TOKEN_EMBD && lm_alias(m) && m->tok != mat) {
            m->lm_owned = m->tok_owned;
            m->lm_shared = m->tok_shared;
            m->tok = nullptr;
            m->tok_owned = m->tok_shared = false;
        }
        const bool lm = which == QG_M_LM_HEAD;
        qg_mat *&dst = lm ? m->lm : m->tok;
        bool &own = lm ? m->lm_owned : m->tok_owned, &shr = lm ? m->lm_shared : m->tok_shared;
        if (dst && !(lm && lm_alias(m))) {
            if (shr) { if (dst->shares > 0) dst->shares--; }
            else if (own) qg_mat_free(m->ctx, dst);
        }
        dst = mat;
        own = !shared;
        shr = shared;
        return;
    }
    const int s = (int)which - QG_M_WQ;
    qg_mat_release(m->ctx, m->w[s][layer], m->owned[s][layer]);
    m->w[s][layer] = mat;
    m->owned[s][layer] = !shared;
}

int gemv(qg_model *m, const qg_mat *a, const float *x, float *y)
{
    if (qg::launch_gemv(a->type, a->plan, qg_gemv_bytes(a), a->nbytes, a->rows, a->cols, x, y,
                        (ihipStream_t *)m->ctx->stream) != 0)
        return mfail(m, QG_ERR_HIP, "GEMV launch", hipGetLastError());
    return QG_OK;
}

// y = A · (rmsnorm(xa + xb) * nw); sum_out (may be NULL) receives xa + xb.
// The GEMV's own prologue does the norm when the matrix runs on the stream
// kernel; otherwise a separate RMSNorm kernel writes m->xn first.
int gemv_norm(qg_model *m, const qg_mat *A, const float *xa, const float *xb, const float *nw,
              float *sum_out, float *y)
{
    return qg_norm_matvec(m->ctx, A, xa, xb, nw, m->cfg.norm_eps, sum_out, y, m->xn, m->ctx->stream);
}

int launched(qg_model *m, const char *what)
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? QG_OK : mfail(m, QG_ERR_HIP, what, e);
}

bool complete(const qg_model *m)
{
    if (!m->tok || !m->lm || !m->final_norm) return false;
    for (int s = 0; s < kSlots; s++)
        for (qg_mat *p : m->w[s])
            if (!p) return false;
    return true;
}

// A row of a matrix whose rows are whole blocks starts on a block boundary,
// so the reference's straddle placement (quant.rs:152-174) writes every
// element of the row and leaves no gap to be zero.
bool whole_rows(const qg_mat *t)
{
    return t->cols % qg::block_elems(t->type) == 0;
}

// Transformer::forward (transformer.rs:63-98) for the token, position and
// slot in m->d_step; enqueues kernels only (also used under graph capture).
int enqueue_forward(qg_model *m)
{
    const qg_model_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    ihipStream_t *sti = (ihipStream_t *)st;
    const uint32_t E = c.embed_dim;
    int rc;
    // embedding row into a zeroed buffer (transformer.rs:74-75, quant.rs:152-174);
    // with whole blocks per row every element is written, so no fill
    if ((!whole_rows(m->tok) && qg::launch_fill(m->h0, E, 0.0f, sti)) ||
        qg::launch_dequantize_row_dev(m->tok->type, m->tok->d, m->tok->rows, m->tok->cols, &m->d_step->token,
                                      m->h0, sti))
        return mfail(m, QG_ERR_HIP, "embedding", hipGetLastError());
    const size_t kv_layer = (size_t)c.max_seq_len * m->kv_dim;
    const float scale = 1.0f / sqrtf((float)m->hd);                      // attention.rs:99
    const uint32_t pairs = (m->q_dim > m->kv_dim ? m->q_dim : m->kv_dim) / 2;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        // the residual stream entering the layer is h0 (layer 0: the
        // embedding) or h1 + fo, which the Q GEMV also stores to h0
        const float *na = l == 0 ? m->h0 : m->h1, *nb = l == 0 ? m->zeros : m->fo;
        const float *anorm = m->vec[QG_V_ATTN_NORM][l];
        float *res = l == 0 ? nullptr : m->h0;
        const int nq = m->f_qkv_n[l];
        if (nq == 3) {
            if ((rc = gemv_norm(m, m->f_qkv[l], na, nb, anorm, res, m->q))) return rc;
        } else if (nq == 2) {
            // [Q;K] and V (another type) in one launch where the pair is
            // supported (a graph branch on a second stream measured slower
            // than one launch after the other)
            if ((rc = qg_norm_pair_matvec(m->ctx, m->f_qkv[l], m->w[QG_M_WV - 2][l], na, nb, anorm, c.norm_eps, res,
                                          m->q, m->v, m->xn, st)))
                return rc;
        } else if ((rc = gemv_norm(m, m->w[QG_M_WQ - 2][l], na, nb, anorm, res, m->q)) ||
                   (rc = gemv_norm(m, m->w[QG_M_WK - 2][l], na, nb, anorm, nullptr, m->k)) ||
                   (rc = gemv_norm(m, m->w[QG_M_WV - 2][l], na, nb, anorm, nullptr, m->v))) {
            return rc;
        }
        float *kc = m->kc + l * kv_layer, *vc = m->vc + l * kv_layer;
        if (m->att_grp) {
            qgm::AttnArgs aa{};
            aa.q = m->q; aa.k = m->k; aa.v = m->v;
            aa.bq = m->vec[QG_V_BQ][l]; aa.bk = m->vec[QG_V_BK][l]; aa.bv = m->vec[QG_V_BV][l];
            aa.kc = kc; aa.vc = vc; aa.cos_t = m->cos_t; aa.sin_t = m->sin_t;
            aa.part = m->att_part; aa.ml = m->att_ml; aa.st = m->d_step;
            aa.kv_dim = m->kv_dim; aa.n_rep = m->n_rep; aa.grp = m->att_grp; aa.nsplit = m->att_nsplit;
            aa.cap = c.max_seq_len;
            aa.scale = scale;
            if (m->att_mode == 2) {
                // two workgroups per head (even / odd positions); the wo GEMV
                // below merges their outputs
                aa.part_stride = m->q_dim;
                aa.ml_stride = 2 * c.n_heads;
                const dim3 grid(2 * c.n_heads), block(64 * qgm::kHeadWaves);
                if (m->hd == 64)
                    hipLaunchKernelGGL((qgm::attn_rope_head_k<1, 2>), grid, block, 0, st, aa, m->ao);
                else if (m->hd == 128)
                    hipLaunchKernelGGL((qgm::attn_rope_head_k<2, 2>), grid, block, 0, st, aa, m->ao);
                else
                    hipLaunchKernelGGL((qgm::attn_rope_head_k<4, 2>), grid, block, 0, st, aa, m->ao);
            } else if (m->att_mode == 1) {
                // one launch: whole heads, normalised output (short contexts)
                const dim3 grid(c.n_heads), block(64 * qgm::kHeadWaves);
                if (m->hd == 64)
                    hipLaunchKernelGGL(qgm::attn_rope_head_k<1>, grid, block, 0, st, aa, m->ao);
                else if (m->hd == 128)
                    hipLaunchKernelGGL(qgm::attn_rope_head_k<2>, grid, block, 0, st, aa, m->ao);
                else
                    hipLaunchKernelGGL(qgm::attn_rope_head_k<4>, grid, block, 0, st, aa, m->ao);
            } else {
                const dim3 grid(c.n_heads / m->att_grp * m->att_nsplit);
                if (m->hd == 64)
                    hipLaunchKernelGGL(qgm::attn_rope_split_k<1>, grid, dim3(256), 0, st, aa);
                else if (m->hd == 128)
                    hipLaunchKernelGGL(qgm::attn_rope_split_k<2>, grid, dim3(256), 0, st, aa);
                else
                    hipLaunchKernelGGL(qgm::attn_rope_split_k<4>, grid, dim3(256), 0, st, aa);
                hipLaunchKernelGGL(qgm::attn_combine_k, dim3(c.n_heads), dim3(256), 0, st, m->att_part, m->att_ml,
                                   m->ao, m->d_step, m->hd, m->att_nsplit);
            }
        } else {
            hipLaunchKernelGGL(qgm::qkv_post_k, dim3((pairs + 255) / 256), dim3(256), 0, st, m->q, m->k, m->v,
                               m->vec[QG_V_BQ][l], m->vec[QG_V_BK][l], m->vec[QG_V_BV][l], kc, vc, m->cos_t,
                               m->sin_t, m->q_dim, m->kv_dim, m->hd, m->d_step);
            hipLaunchKernelGGL(qgm::attention_k, dim3(c.n_heads), dim3(256), m->att_lds, st, m->q, kc, vc, m->ao,
                               m->d_step, m->hd, m->kv_dim, m->n_rep, scale);
        }
        if ((rc = launched(m, "attention"))) return rc;
        if (m->att_grp && m->att_mode == 2) {
            const qg_mat *wo = m->w[QG_M_WO - 2][l];
            if (qg::launch_gemv_attn(wo->plan, qg_gemv_bytes(wo), wo->nbytes, wo->rows, wo->cols, m->att_part,
                                     m->att_ml, c.n_heads, m->hd, m->ao2, (ihipStream_t *)st) != 0)
                return mfail(m, QG_ERR_HIP, "GEMV launch (attention merge)", hipGetLastError());
        } else if ((rc = gemv(m, m->w[QG_M_WO - 2][l], m->ao, m->ao2))) {
            return rc;
        }
        // h1 = h0 + attention output (stored by the gate GEMV); MLP input = ffn_norm(h1)
        const float *fnorm = m->vec[QG_V_FFN_NORM][l];
        if (m->f_gu[l]) {
            // silu(gate) * up (mlp.rs:31-43) paired in the [gate; up] kernel
            // (or its outputs in g, u and a product kernel), then down
            if ((rc = qg_norm_glu_matvec(m->ctx, m->f_gu[l], m->h0, m->ao2, fnorm, c.norm_eps, m->h1, m->hb, m->g,
                                         m->xn, st)) ||
                (rc = gemv(m, m->w[QG_M_DOWN - 2][l], m->hb, m->fo)))
                return rc;
            continue;
        }
        if ((rc = gemv_norm(m, m->w[QG_M_GATE - 2][l], m->h0, m->ao2, fnorm, m->h1, m->g)) ||
            (rc = gemv_norm(m, m->w[QG_M_UP - 2][l], m->h0, m->ao2, fnorm, nullptr, m->u)))
            return rc;
        // down(silu(g) * u) (mlp.rs:36-45): the product inside the down GEMV's prologue
        if ((rc = qg_silu_matvec(m->ctx, m->w[QG_M_DOWN - 2][l], m->g, m->u, m->fo, m->hb, st))) return rc;
    }
    // final norm of h1 + fo (transformer.rs:87-97) inside the lm_head GEMV
    return gemv_norm(m, m->lm, m->h1, m->fo, m->final_norm, nullptr, m->logits);
}

qgm::SampleArgs sample_args(qg_model *m, uint32_t n_recent, float penalty, bool generate, uint32_t window)
{
    qgm::SampleArgs a{};
    a.logits = m->logits;
    a.n = m->cfg.vocab_size;
    a.recent = m->d_recent;
    a.n_recent = n_recent;
    a.hist = generate ? m->d_hist : nullptr;
    a.window = window;
    a.penalty = penalty;
    a.st = m->d_step;
    a.pv = m->s_pv;
    a.pi = m->s_pi;
    a.token = m->d_token;
    return a;
}

int enqueue_sample(qg_model *m, const qgm::SampleArgs &a)
{
    hipStream_t st = m->ctx->stream;
    hipLaunchKernelGGL(qgm::sample_part_k, dim3(qgm::kSampleWG), dim3(256), 0, st, a);
    hipLaunchKernelGGL(qgm::sample_final_k, dim3(1), dim3(64), 0, st, a, qgm::kSampleWG);
    return launched(m, "sample");
}

// generate's decode step: sample from the last logits, append and advance,
// then the forward pass of the sampled token
int enqueue_decode(qg_model *m)
{
    int rc = enqueue_sample(m, sample_args(m, 0, m->g_dec_penalty, true, m->g_dec_window));
    return rc ? rc : enqueue_forward(m);
}

int capture(qg_model *m, int (*fn)(qg_model *), hipGraphExec_t *out)
{
    hipStream_t st = m->ctx->stream;
    QGM_HIP(m, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const int rc = fn(m);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return mfail(m, QG_ERR_HIP, "hipStreamEndCapture", e);
    const hipError_t e2 = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e2 != hipSuccess) { *out = nullptr; return mfail(m, QG_ERR_HIP, "hipGraphInstantiate", e2); }
    return QG_OK;
}

// Whether every layer's wo can take the two-range attention output
// (launch_gemv_attn: a stream-kernel plan of a fixed-point type with one row
// per group) and the partial-output buffers hold two ranges.
bool two_range_ok(const qg_model *m)
{
    if (!m->att_grp || m->att_nsplit < 2 || m->hd % 16 != 0) return false;
    for (uint32_t l = 0; l < m->cfg.n_layers; l++) {
        const qg_mat *wo = m->w[QG_M_WO - 2][l];
        if (!wo || wo->plan.kind != 1 || !wo->plan.fn_attn) return false;
    }
    return true;
}

// the attention mode of the forward pass that writes cache slot `slot`: up to
// kShortSeq cached positions whole heads, as two position ranges per head
// where every wo takes them (mode 2) or in one workgroup per head (mode 1);
// beyond, split over position ranges (mode 0).  att_path: 0 by length, 1
// always one workgroup per head, 2 always split, 3 always two ranges where
// the wo matrices allow it (else one workgroup per head).
void pick_attention(qg_model *m, uint32_t slot)
{
    const bool shrt = m->att_path == 1 || m->att_path == 3 || (m->att_path == 0 && slot + 1 <= qgm::kShortSeq);
    if (!m->att_grp || !shrt) m->att_mode = 0;
    else m->att_mode = m->att_path != 1 && two_range_ok(m) ? 2 : 1;
}

int run_forward(qg_model *m, uint32_t slot)
{
    int rc;
    if ((rc = prepare(m))) return rc;
    pick_attention(m, slot);
    if (!m->use_graphs) return enqueue_forward(m);
    hipGraphExec_t &g = m->g_fwd[m->att_mode];
    if (!g && (rc = capture(m, enqueue_forward, &g))) return rc;
    QGM_HIP(m, hipGraphLaunch(g, m->ctx->stream));
    return QG_OK;
}

// slot: the cache slot of the forward pass after the sampled token
int run_decode(qg_model *m, float penalty, uint32_t window, uint32_t slot)
{
    if (m->g_dec_penalty != penalty || m->g_dec_window != window)
        for (hipGraphExec_t &g : m->g_dec)
            if (g) {
                (void)hipGraphExecDestroy(g);
                g = nullptr;
            }
    m->g_dec_penalty = penalty;
    m->g_dec_window = window;
    int rc;
    if ((rc = prepare(m))) return rc;
    pick_attention(m, slot);
    if (!m->use_graphs) return enqueue_decode(m);
    hipGraphExec_t &g = m->g_dec[m->att_mode];
    if (!g && (rc = capture(m, enqueue_decode, &g))) return rc;
    QGM_HIP(m, hipGraphLaunch(g, m->ctx->stream));
    return QG_OK;
}

// host-fed Step record (pinned ring; the stream is drained before a slot is reused)
int put_step(qg_model *m, uint32_t token, uint32_t pos, uint32_t slot)
{
    if (m->ring == kRing) {
        QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
        m->ring = 0;
    }
    qgm::Step *s = m->h_steps + m->ring++;
    *s = qgm::Step{token, pos, slot, 0};
    QGM_HIP(m, hipMemcpyAsync(m->d_step, s, sizeof(qgm::Step), hipMemcpyHostToDevice, m->ctx->stream));
    return QG_OK;
}

// ---------------------------------------------------------- batched prefill

// Every layer matrix on the MFMA path: supported type, cols % 128 == 0; and
// the prefill attention's scores fit its LDS.
bool pf_supported(const qg_model *m)
{
    if (!m->pf_batched) return false;
    if (m->hd != 64 && m->hd != 128 && m->hd != 256) return false;        // pf_attention_k's head sizes
    for (int s = 0; s < kSlots; s++)
        for (const qg_mat *p : m->w[s])
            if (!p || !qg::prefill_type_supported(p->type) || p->cols % 128 != 0) return false;
    return true;
}

int pf_alloc(qg_model *m)
{
    if (m->pf_h[0]) return QG_OK;
    const size_t T = qg::kPfMaxTokens, E = m->cfg.embed_dim, H = m->cfg.hidden_dim;
    const size_t ldq = m->q_dim + 2 * (size_t)m->kv_dim;
    size_t kmax = E > H ? E : H;
    if (m->q_dim > kmax) kmax = m->q_dim;
    // the K splits of the four GEMM groups (the same shapes in every layer)
    const uint32_t tq = qg::pf_tiles(m->q_dim), tk = qg::pf_tiles(m->kv_dim), ne = (uint32_t)(E / 32);
    m->pf_s_qkv1 = qg::pf_split(tq + 2 * tk, ne);
    m->pf_s_qk = qg::pf_split(tq + tk, ne);
    m->pf_s_v = qg::pf_split(tk, ne);
    m->pf_s_qkv = std::max({m->pf_s_qkv1, m->pf_s_qk, m->pf_s_v});          // slabs of the buffer
    m->pf_s_o = qg::pf_split(qg::pf_tiles(E), (uint32_t)(m->q_dim / 32));
    m->pf_s_gu = qg::pf_split(2 * qg::pf_tiles(H), (uint32_t)(E / 32));
    m->pf_s_down = qg::pf_split(qg::pf_tiles(E), (uint32_t)(H / 32));
    int rc;
    if ((rc = dalloc(m, &m->pf_h[0], T * E)) || (rc = dalloc(m, &m->pf_h[1], T * E)) ||
        (rc = dalloc(m, &m->pf_qkv, m->pf_s_qkv * T * ldq)) || (rc = dalloc(m, &m->pf_ao, T * m->q_dim)) ||
        (rc = dalloc(m, &m->pf_ao2, m->pf_s_o * T * E)) || (rc = dalloc(m, &m->pf_g, m->pf_s_gu * T * 2 * H)) ||
        (rc = dalloc(m, &m->pf_fo, m->pf_s_down * T * E)) || (rc = dalloc(m, &m->pf_last, E)) ||
        (rc = dalloc(m, &m->pf_xp, 2 * T * kmax)) ||
        (rc = dalloc(m, &m->pf_rec, T * (kmax / 32 + (kmax + 255) / 256))) ||
        (rc = dalloc(m, &m->pf_ss, T * ((E + 255) / 256))) ||
        (rc = dalloc(m, &m->pf_tok, (size_t)m->cfg.max_seq_len)))
        return rc;
    return QG_OK;
}

// y[t][0..rows) (row stride ldy, slices of T * ldy floats) = mat . x_t for the
// chunk's tokens and 1..3 matrices over the same x, given as the f16 pieces
// of the last pf_planes call over `cols` elements
int pf_gemm(qg_model *m, const qg::PfMat *mats, int n, size_t cols, uint32_t ntok, uint32_t ldy, uint32_t slices)
{
    const int r = qg::launch_pf_gemm(mats, n, cols, m->pf_xp, m->pf_rec, ntok, ldy, slices,
                                     (size_t)qg::kPfMaxTokens * ldy, (ihipStream_t *)m->ctx->stream);
    return r ? mfail(m, QG_ERR_HIP, "prefill GEMM launch", hipGetLastError()) : QG_OK;
}

// a layer matrix for the prefill GEMM: its GGUF-layout bytes, or its
// repacked copy (an uploaded matrix keeps only that)
qg::PfMat pf_mat(const qg_mat *mat, float *y)
{
    if (mat->d) return qg::PfMat{mat->type, mat->d, mat->rows, y, false, 0, 0, 0};
    return qg::PfMat{mat->type, mat->d_rp, mat->rows, y, true, mat->plan.g, mat->plan.ni, (size_t)mat->plan.group_bytes};
}

// f16 pieces of x = f(a, b) for the chunk's tokens (scaled per 256-element
// group); a and b of na / nb slices kPfMaxTokens * lda floats apart.  Mode 1
// (the RMSNorm's numerator) leaves its sums of squares in m->pf_ss, which the
// consumer of the GEMM's output (pf_qkv_post_k, the mode-2 call: `pre`)
// turns into 1 / rms.
int pf_planes(qg_model *m, const float *a, uint32_t na, const float *b, uint32_t nb, float *sum_out, const float *nw,
              size_t n, size_t lda, int mode, bool pre, uint32_t ntok)
{
    const size_t E = m->cfg.embed_dim;
    const int r = qg::launch_pf_planes(a, na, b, nb, (size_t)qg::kPfMaxTokens * lda, sum_out, nw, n, lda, mode,
                                       pre ? m->pf_ss : nullptr, E, m->cfg.norm_eps, m->pf_ss, m->pf_xp, m->pf_rec,
                                       ntok, (ihipStream_t *)m->ctx->stream);
    return r ? mfail(m, QG_ERR_HIP, "prefill planes launch", hipGetLastError()) : QG_OK;
}

// Transformer::forward (transformer.rs:63-98) for tokens d_tok[0..ntok) (on
// device) at positions / cache slots s0 .. s0 + ntok - 1, every layer's
// projections as GEMMs over the chunk; leaves the last token's logits in
// m->logits.
int pf_chunk(qg_model *m, const uint32_t *d_tok, uint32_t ntok, uint32_t s0)
{
    const qg_model_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    ihipStream_t *sti = (ihipStream_t *)st;
    const uint32_t E = c.embed_dim, H = c.hidden_dim, ldq = m->q_dim + 2 * m->kv_dim;
    const size_t T = qg::kPfMaxTokens;
    int rc;
    // embedding rows into zeroed rows (transformer.rs:74-75, quant.rs:152-174)
    float *h = m->pf_h[0], *h2 = m->pf_h[1];
    if ((!whole_rows(m->tok) && qg::launch_fill(h, (size_t)ntok * E, 0.0f, sti)) ||
        qg::launch_dequantize_rows_dev(m->tok->type, m->tok->d, m->tok->rows, m->tok->cols, d_tok, ntok, h, E, sti))
        return mfail(m, QG_ERR_HIP, "embedding", hipGetLastError());
    const size_t kv_layer = (size_t)c.max_seq_len * m->kv_dim;
    const float scale = 1.0f / sqrtf((float)m->hd);                      // attention.rs:99
    for (uint32_t l = 0; l < c.n_layers; l++) {
        // the residual stream entering the layer: the embeddings, or h + fo of
        // the previous layer (written to the other buffer), then attn_norm
        if (l) {
            if ((rc = pf_planes(m, h, 1, m->pf_fo, m->pf_s_down, h2, m->vec[QG_V_ATTN_NORM][l], E, E, 1, false,
                                ntok)))
                return rc;
            std::swap(h, h2);
        } else if ((rc = pf_planes(m, h, 1, nullptr, 0, nullptr, m->vec[QG_V_ATTN_NORM][l], E, E, 1, false,
                                   ntok))) {
            return rc;
        }
        const qg::PfMat qkv[3] = {pf_mat(m->w[QG_M_WQ - 2][l], m->pf_qkv),
                                  pf_mat(m->w[QG_M_WK - 2][l], m->pf_qkv + m->q_dim),
                                  pf_mat(m->w[QG_M_WV - 2][l], m->pf_qkv + m->q_dim + m->kv_dim)};
        // V in a launch of its own (another type or layout than K) takes its own slices
        const bool v_apart = qkv[2].type != qkv[1].type || qkv[2].rp != qkv[1].rp || (qkv[2].rp && qkv[2].g != qkv[1].g);
        const uint32_t s_qk = v_apart ? m->pf_s_qk : m->pf_s_qkv1, s_v = v_apart ? m->pf_s_v : m->pf_s_qkv1;
        if (v_apart) {
            if ((rc = pf_gemm(m, qkv, 2, E, ntok, ldq, s_qk)) || (rc = pf_gemm(m, qkv + 2, 1, E, ntok, ldq, s_v)))
                return rc;
        } else if ((rc = pf_gemm(m, qkv, 3, E, ntok, ldq, s_qk))) {
            return rc;
        }
        float *kc = m->kc + l * kv_layer, *vc = m->vc + l * kv_layer;
        if (qg::launch_pf_qkv_post(m->pf_qkv, ldq, s_qk, s_v, T * ldq, m->pf_ss, E, c.norm_eps,
                                   m->vec[QG_V_BQ][l], m->vec[QG_V_BK][l], m->vec[QG_V_BV][l], kc, vc, m->cos_t,
                                   m->sin_t, m->q_dim, m->kv_dim, m->hd, s0, s0, ntok, sti) ||
            qg::launch_pf_attention(m->pf_qkv, ldq, kc, vc, m->pf_ao, c.n_heads, m->hd, m->kv_dim, m->n_rep, scale, s0,
                                    ntok, sti))
            return mfail(m, QG_ERR_HIP, "prefill attention", hipGetLastError());
        const qg::PfMat wo = pf_mat(m->w[QG_M_WO - 2][l], m->pf_ao2);
        if ((rc = pf_planes(m, m->pf_ao, 1, nullptr, 0, nullptr, nullptr, m->q_dim, m->q_dim, 0, false, ntok)) ||
            (rc = pf_gemm(m, &wo, 1, m->q_dim, ntok, E, m->pf_s_o)))
            return rc;
        // h = h + attention output; MLP input = ffn_norm(h) (transformer.rs:31-46)
        if ((rc = pf_planes(m, h, 1, m->pf_ao2, m->pf_s_o, h2, m->vec[QG_V_FFN_NORM][l], E, E, 1, false, ntok)))
            return rc;
        std::swap(h, h2);
        const qg::PfMat gu[2] = {pf_mat(m->w[QG_M_GATE - 2][l], m->pf_g), pf_mat(m->w[QG_M_UP - 2][l], m->pf_g + H)};
        if ((rc = pf_gemm(m, gu, 2, E, ntok, 2 * H, m->pf_s_gu))) return rc;
        // down(silu(gate) * up) (mlp.rs:36-45)
        const qg::PfMat down = pf_mat(m->w[QG_M_DOWN - 2][l], m->pf_fo);
        if ((rc = pf_planes(m, m->pf_g, m->pf_s_gu, m->pf_g + H, m->pf_s_gu, nullptr, nullptr, H, 2 * (size_t)H, 2,
                            true, ntok)) ||
            (rc = pf_gemm(m, &down, 1, H, ntok, E, m->pf_s_down)))
            return rc;
    }
    // the last token's final norm of h + fo inside the lm_head GEMV (transformer.rs:87-97)
    const size_t last = (size_t)(ntok - 1) * E;
    if (qg::launch_pf_sum(m->pf_fo + last, m->pf_s_down, T * E, E, m->pf_last, sti))
        return mfail(m, QG_ERR_HIP, "prefill sum", hipGetLastError());
    return gemv_norm(m, m->lm, h + last, m->pf_last, m->final_norm, nullptr, m->logits);
}

// n tokens at cache slots / positions m->seq ..; leaves the last logits on
// device and advances m->seq
int prefill(qg_model *m, const uint32_t *tok, size_t n)
{
    int rc;
    if (n == 0) return QG_OK;
    if (pf_supported(m)) {
        if ((rc = prepare(m)) || (rc = pf_alloc(m))) return rc;
        // the token ids to device once (n <= max_seq_len - seq, checked by the caller)
        QGM_HIP(m, hipMemcpyAsync(m->pf_tok, tok, n * sizeof(uint32_t), hipMemcpyHostToDevice, m->ctx->stream));
        QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
        for (size_t i = 0; i < n; i += qg::kPfMaxTokens) {
            const uint32_t nt = (uint32_t)(n - i < qg::kPfMaxTokens ? n - i : qg::kPfMaxTokens);
            if ((rc = pf_chunk(m, m->pf_tok + i, nt, (uint32_t)(m->seq + i)))) return rc;
        }
        m->seq += n;
        return QG_OK;
    }
    for (size_t i = 0; i < n; i++) {
        if ((rc = put_step(m, tok[i], (uint32_t)m->seq, (uint32_t)m->seq)) || (rc = run_forward(m, (uint32_t)m->seq)))
            return rc;
        m->seq += 1;
    }
    return QG_OK;
}

}  // namespace

extern "C" {

int qg_model_create(qg_ctx *ctx, const qg_model_config *cfg, qg_model **out)
{
    if (!ctx || !cfg || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    const qg_model_config c = *cfg;
    if (c.embed_dim == 0 || c.n_layers == 0 || c.n_heads == 0 || c.hidden_dim == 0 ||
        c.vocab_size == 0 || c.max_seq_len == 0 || c.embed_dim % c.n_heads != 0)
        return qg_fail(ctx, QG_ERR_SHAPE, "model config");
    const uint32_t n_kv = c.n_kv_heads ? c.n_kv_heads : c.n_heads;   // model.rs:100
    const uint32_t hd = c.embed_dim / c.n_heads;
    if (hd % 2 != 0 || c.n_heads % n_kv != 0) return qg_fail(ctx, QG_ERR_SHAPE, "model config");
    qg_model *m = new (std::nothrow) qg_model;
    if (!m) return qg_fail(ctx, QG_ERR_OUT_OF_MEMORY, "host allocation");
    m->ctx = ctx;
    m->cfg = c;
    m->cfg.n_kv_heads = n_kv;
    m->hd = hd;
    m->q_dim = c.n_heads * hd;
    m->kv_dim = n_kv * hd;
    m->n_rep = c.n_heads / n_kv;
    // attention layout: workgroups of grp query heads (a divisor of n_rep, at
    // most 8) times up to 64 position ranges of at least 8 positions, about
    // 256 workgroups in all at long sequences; any max_seq_len
    constexpr size_t kLdsMax = 65536;
    if (hd == 64 || hd == 128 || hd == 256) {
        uint32_t grp = 1;
        for (uint32_t d = 1; d <= qgm::kMaxGroup; d++)
            if (m->n_rep % d == 0) grp = d;
        const uint32_t groups = c.n_heads / grp;
        uint32_t ns = (256 + groups - 1) / groups;
        ns = ns < 1 ? 1 : ns > qgm::kMaxSplit ? qgm::kMaxSplit : ns;
        m->att_grp = grp;
        m->att_nsplit = ns;
    } else {
        m->att_lds = ((size_t)hd + c.max_seq_len) * sizeof(float);
        if (m->att_lds > kLdsMax) {
            delete m;
            return qg_fail(ctx, QG_ERR_SHAPE, "max_seq_len too large for this head_dim");
        }
    }
    const size_t L = c.n_layers, E = c.embed_dim, H = c.hidden_dim;
    for (int s = 0; s < kSlots; s++) { m->w[s].assign(L, nullptr); m->owned[s].assign(L, false); }
    int rc;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) { free_model(m); return qg_fail(ctx, QG_ERR_HIP, "hipSetDevice", e); }
    const size_t kvn = L * (size_t)c.max_seq_len * m->kv_dim;
    const size_t npart = m->att_grp ? (size_t)c.n_heads * m->att_nsplit : 1;
    if ((rc = dalloc(m, &m->final_norm, E)) || (rc = dalloc(m, &m->kc, kvn)) ||
        (rc = dalloc(m, &m->vc, kvn)) || (rc = dalloc(m, &m->h0, E)) || (rc = dalloc(m, &m->h1, E)) ||
        (rc = dalloc(m, &m->xn, E > H ? E : H)) || (rc = dalloc(m, &m->q, m->q_dim + 2 * (size_t)m->kv_dim)) ||
        (rc = dalloc(m, &m->ao, m->q_dim)) || (rc = dalloc(m, &m->ao2, E)) ||
        (rc = dalloc(m, &m->g, 2 * H)) || (rc = dalloc(m, &m->hb, H)) ||
        (rc = dalloc(m, &m->fo, E)) || (rc = dalloc(m, &m->logits, c.vocab_size)) ||
        (rc = dalloc(m, &m->zeros, E > H ? E : H)) || (rc = dalloc(m, &m->att_part, npart * hd)) ||
        (rc = dalloc(m, &m->att_ml, npart * 2)) || (rc = dalloc(m, &m->s_pv, qgm::kSampleWG)) ||
        (rc = dalloc(m, &m->s_pi, qgm::kSampleWG)) || (rc = dalloc(m, &m->d_recent, qgm::kRecentMax)) ||
        (rc = dalloc(m, &m->d_token, 1)) || (rc = dalloc(m, &m->d_hist, (size_t)c.max_seq_len + 1)) ||
        (rc = dalloc(m, &m->d_step, 1))) {
        free_model(m);
        return rc;
    }
    m->k = m->q + m->q_dim;                 // q, k, v and g, u are contiguous
    m->v = m->k + m->kv_dim;
    m->u = m->g + H;
    m->f_qkv.assign(L, nullptr);
    m->f_gu.assign(L, nullptr);
    m->f_qkv_n.assign(L, 0);
    for (int s = 1; s < 6; s++) {
        m->vec[s].assign(L, nullptr);
        const size_t n = s <= 2 ? E : s == 3 ? m->q_dim : m->kv_dim;
        for (size_t l = 0; l < L; l++)
            if ((rc = dalloc(m, &m->vec[s][l], n))) { free_model(m); return rc; }
    }
    // RoPE tables (rope.rs:42-58): f32 powf / cos / sin, as the reference
    const size_t half = hd / 2, np = (size_t)c.max_seq_len * half;
    std::vector<float> ct(np), st(np);
    for (size_t pos = 0; pos < c.max_seq_len; pos++)
        for (size_t i = 0; i < half; i++) {
            const float exponent = (float)(2 * i) / (float)hd;
            const float theta = 1.0f / powf(c.rope_base, exponent);
            const float angle = (float)pos * theta;
            ct[pos * half + i] = cosf(angle);
            st[pos * half + i] = sinf(angle);
        }
    if ((rc = dalloc(m, &m->cos_t, np)) || (rc = dalloc(m, &m->sin_t, np))) { free_model(m); return rc; }
    if ((e = hipMemcpy(m->cos_t, ct.data(), np * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(m->sin_t, st.data(), np * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipHostMalloc((void **)&m->h_recent, qgm::kRecentMax * sizeof(uint32_t), hipHostMallocDefault)) !=
            hipSuccess ||
        (e = hipHostMalloc((void **)&m->h_token, sizeof(uint32_t), hipHostMallocDefault)) != hipSuccess ||
        (e = hipHostMalloc((void **)&m->h_steps, kRing * sizeof(qgm::Step), hipHostMallocDefault)) != hipSuccess) {
        free_model(m);
        return qg_fail(ctx, QG_ERR_HIP, "model set-up", e);
    }
    ctx->models.insert(m);
    *out = m;
    return QG_OK;
}

int qg_model_destroy(qg_model *m)
{
    if (!m) return QG_ERR_INVALID_ARG;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_model(m);
    return QG_OK;
}

int qg_model_set_matrix(qg_model *m, uint32_t which, uint32_t layer, const void *raw, size_t nbytes,
                        uint32_t ggml_type, size_t rows, size_t cols)
{
    if (!m || !raw) return QG_ERR_INVALID_ARG;
    size_t er, ec;
    slot_shape(m, which, &er, &ec);
    if (er == 0) return mfail(m, QG_ERR_INVALID_ARG, "matrix slot");
    if (rows != er || cols != ec) return mfail(m, QG_ERR_SHAPE, "matrix shape does not match the config");
    const bool per_layer = which >= QG_M_WQ;
    if (per_layer && layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
    qg_mat *mat = nullptr;
    int rc = qg_upload(m->ctx, raw, nbytes, ggml_type, rows, cols, &mat);
    if (rc) return rc;
    (void)hipStreamSynchronize(m->ctx->stream);
    drop_graphs(m);
    if ((rc = drop_fused(m))) {
        qg_mat_free(m->ctx, mat);
        return rc;
    }
    put_slot(m, which, layer, mat, false);
    return QG_OK;
}

int qg_model_share_matrix(qg_model *m, uint32_t which, uint32_t layer, const qg_mat *mat)
{
    if (!m || !mat) return QG_ERR_INVALID_ARG;
    // a live matrix of this model's context before any of its fields is read
    int rc = qg_check_mat(m->ctx, mat);
    if (rc) return rc;
    size_t er, ec;
    slot_shape(m, which, &er, &ec);
    if (er == 0) return mfail(m, QG_ERR_INVALID_ARG, "matrix slot");
    if (mat->rows != er || mat->cols != ec)
        return mfail(m, QG_ERR_SHAPE, "matrix shape does not match the config");
    const bool per_layer = which >= QG_M_WQ;
    if (per_layer && layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
    (void)hipStreamSynchronize(m->ctx->stream);
    drop_graphs(m);
    if ((rc = drop_fused(m))) return rc;
    put_slot(m, which, layer, const_cast<qg_mat *>(mat), true);
    return QG_OK;
}

int qg_model_set_vector(qg_model *m, uint32_t which, uint32_t layer, const float *v, size_t n)
{
    if (!m || !v) return QG_ERR_INVALID_ARG;
    float *dst;
    size_t want;
    if (which == QG_V_FINAL_NORM) { dst = m->final_norm; want = m->cfg.embed_dim; }
    else if (which <= QG_V_BV) {
        if (layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
        dst = m->vec[which][layer];
        want = which <= QG_V_FFN_NORM ? m->cfg.embed_dim : which == QG_V_BQ ? m->q_dim : m->kv_dim;
    } else {
        return mfail(m, QG_ERR_INVALID_ARG, "vector slot");
    }
    if (n != want) return mfail(m, QG_ERR_SHAPE, "vector length does not match the config");
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
    QGM_HIP(m, hipMemcpy(dst, v, n * sizeof(float), hipMemcpyHostToDevice));
    return QG_OK;
}

int qg_model_use_graphs(qg_model *m, int enable)
{
    if (!m) return QG_ERR_INVALID_ARG;
    m->use_graphs = enable != 0;
    return QG_OK;
}

int qg_model_reset(qg_model *m)
{
    if (!m) return QG_ERR_INVALID_ARG;
    m->seq = 0;
    return QG_OK;
}

int qg_model_seq_len(const qg_model *m, size_t *len)
{
    if (!m || !len) return QG_ERR_INVALID_ARG;
    *len = m->seq;
    return QG_OK;
}

int qg_model_forward(qg_model *m, uint32_t token, uint32_t pos, float *logits)
{
    if (!m) return QG_ERR_INVALID_ARG;
    if (!complete(m)) return mfail(m, QG_ERR_INVALID_ARG, "model matrices / final norm not all set");
    const qg_model_config &c = m->cfg;
    if (token >= c.vocab_size) return mfail(m, QG_ERR_SHAPE, "token id >= vocab_size");
    if (m->seq >= c.max_seq_len || pos >= c.max_seq_len)
        return mfail(m, QG_ERR_SHAPE, "KV cache full (max_seq_len)");   // kv_cache.rs:54-59
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    int rc;
    if ((rc = put_step(m, token, pos, (uint32_t)m->seq)) || (rc = run_forward(m, (uint32_t)m->seq))) return rc;
    m->seq += 1;
    if (logits) {
        QGM_HIP(m, hipMemcpyAsync(logits, m->logits, (size_t)c.vocab_size * sizeof(float),
                                  hipMemcpyDeviceToHost, m->ctx->stream));
        QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
    }
    return QG_OK;
}

int qg_model_prefill(qg_model *m, const uint32_t *tokens, size_t n, float *logits)
{
    if (!m || (n && !tokens)) return QG_ERR_INVALID_ARG;
    if (!complete(m)) return mfail(m, QG_ERR_INVALID_ARG, "model matrices / final norm not all set");
    const qg_model_config &c = m->cfg;
    if (n > c.max_seq_len || m->seq + n > c.max_seq_len)
        return mfail(m, QG_ERR_SHAPE, "KV cache full (max_seq_len)");   // kv_cache.rs:54-59
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= c.vocab_size) return mfail(m, QG_ERR_SHAPE, "token id >= vocab_size");
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    int rc;
    if ((rc = prefill(m, tokens, n))) return rc;
    if (logits && n) {
        QGM_HIP(m, hipMemcpyAsync(logits, m->logits, (size_t)c.vocab_size * sizeof(float), hipMemcpyDeviceToHost,
                                  m->ctx->stream));
        QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
    }
    return QG_OK;
}

int qg_model_use_batched_prefill(qg_model *m, int enable)
{
    if (!m) return QG_ERR_INVALID_ARG;
    m->pf_batched = enable != 0;
    return QG_OK;
}

int qg_model_resident_bytes(qg_model *m, size_t *weights, size_t *file_bytes, size_t *total)
{
    if (!m) return QG_ERR_INVALID_ARG;
    int rc;
    if (complete(m) && (rc = prepare(m))) return rc;
    std::set<const qg_mat *> mats;
    size_t w = 0, f = 0;
    auto add = [&](const qg_mat *p, bool slot) {
        if (!p) return;
        if (slot) f += p->nbytes;
        if (mats.insert(p).second) w += qg_mat_resident(p);
    };
    add(m->tok, true);
    if (!lm_alias(m)) add(m->lm, true);
    for (int s = 0; s < kSlots; s++)
        for (const qg_mat *p : m->w[s]) add(p, true);
    for (const qg_mat *p : m->f_qkv) add(p, false);
    for (const qg_mat *p : m->f_gu) add(p, false);
    if (weights) *weights = w;
    if (file_bytes) *file_bytes = f;
    if (total) *total = w + m->alloc_bytes;
    return QG_OK;
}

int qg_model_set_attention_path(qg_model *m, int path)
{
    if (!m || path < 0 || path > 3) return QG_ERR_INVALID_ARG;
    m->att_path = path;
    return QG_OK;
}

int qg_model_sample_greedy(qg_model *m, const uint32_t *recent, size_t n_recent, float penalty, size_t window,
                           uint32_t *token)
{
    if (!m || !token || (n_recent && !recent)) return QG_ERR_INVALID_ARG;
    // sampler.rs:109-116: the last `window` of the recent tokens
    size_t start = n_recent > window ? n_recent - window : 0;
    size_t n = n_recent - start;
    if (n > qgm::kRecentMax) { start += n - qgm::kRecentMax; n = qgm::kRecentMax; }
    hipStream_t st = m->ctx->stream;
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    if (n) {
        QGM_HIP(m, hipStreamSynchronize(st));                 // h_recent is reused
        std::memcpy(m->h_recent, recent + start, n * sizeof(uint32_t));
        QGM_HIP(m, hipMemcpyAsync(m->d_recent, m->h_recent, n * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    }
    // sampler.rs:76-78: no penalty pass without recent tokens or with penalty 1
    int rc = enqueue_sample(m, sample_args(m, (uint32_t)n, n ? penalty : 1.0f, false, 0));
    if (rc) return rc;
    QGM_HIP(m, hipMemcpyAsync(m->h_token, m->d_token, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    QGM_HIP(m, hipStreamSynchronize(st));
    *token = *m->h_token;
    return QG_OK;
}

int qg_model_generate(qg_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_new, float penalty,
                      size_t window, uint32_t *out_tokens, double *prefill_s, double *decode_s)
{
    if (!m || (n_prompt && !prompt) || (n_new && !out_tokens)) return QG_ERR_INVALID_ARG;
    if (n_prompt == 0 && n_new > 0) return mfail(m, QG_ERR_INVALID_ARG, "generation needs a prompt");
    if (!complete(m)) return mfail(m, QG_ERR_INVALID_ARG, "model matrices / final norm not all set");
    const qg_model_config &c = m->cfg;
    if (n_prompt + n_new > c.max_seq_len) return mfail(m, QG_ERR_SHAPE, "KV cache full (max_seq_len)");
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= c.vocab_size) return mfail(m, QG_ERR_SHAPE, "token id >= vocab_size");
    using clk = std::chrono::steady_clock;
    hipStream_t st = m->ctx->stream;
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    QGM_HIP(m, hipStreamSynchronize(st));
    m->seq = 0;                                                     // fresh caches (model.rs:341-346)
    if (n_prompt == 0) return QG_OK;
    QGM_HIP(m, hipMemcpy(m->d_hist, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice));
    // model.rs:370-374 passes the last 64 tokens; the sampler keeps `window` of them
    const uint32_t win = window > qgm::kRecentMax ? qgm::kRecentMax : (uint32_t)window;
    int rc;
    auto t0 = clk::now();
    if (pf_supported(m)) {
        // batched prefill, then the Step record the token-by-token loop ends with
        if ((rc = prefill(m, prompt, n_prompt)) ||
            (rc = put_step(m, prompt[n_prompt - 1], (uint32_t)(n_prompt - 1), (uint32_t)(n_prompt - 1))))
            return rc;
    } else {
        if ((rc = put_step(m, prompt[0], 0, 0))) return rc;
        for (size_t p = 0; p < n_prompt; p++) {
            if ((rc = run_forward(m, (uint32_t)p))) return rc;
            if (p + 1 < n_prompt) {
                hipLaunchKernelGGL(qgm::advance_k, dim3(1), dim3(64), 0, st, m->d_step, m->d_hist);
                if ((rc = launched(m, "advance"))) return rc;
            }
        }
    }
    QGM_HIP(m, hipStreamSynchronize(st));
    auto t1 = clk::now();
    for (size_t s = 0; s < n_new; s++)
        if ((rc = run_decode(m, penalty, win, (uint32_t)(n_prompt + s)))) return rc;
    QGM_HIP(m, hipStreamSynchronize(st));
    auto t2 = clk::now();
    m->seq = n_prompt + n_new;
    if (n_new)
        QGM_HIP(m, hipMemcpy(out_tokens, m->d_hist + n_prompt, n_new * sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
    if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
    return QG_OK;
}

}  // extern "C"

int qg_model_tie_lm_head(qg_model *m)
{
    if (!m || !m->tok) return QG_ERR_INVALID_ARG;
    (void)hipStreamSynchronize(m->ctx->stream);
    drop_graphs(m);
    if (!lm_alias(m)) qg_mat_release(m->ctx, m->lm, m->lm_owned);
    m->lm = m->tok;
    m->lm_owned = m->lm_shared = false;
    return QG_OK;
}

void qg_models_free_all(qg_ctx *ctx)
{
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    while (!ctx->models.empty()) free_model(*ctx->models.begin());
}
