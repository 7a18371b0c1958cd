// qg_probe.hip -- libqgprobe.so: measurement-only reads of a device buffer
// (include/qgprobe.h).  Nothing here computes anything; bench.py times these
// kernels to find the fastest plain read of the GEMV's byte count, the
// streaming ceiling its HBM rate is compared with.
#include <hip/hip_runtime.h>

#include "qgprobe.h"

namespace {

constexpr uint32_t kMagic = 0x9E3779B9u;

// Thread t of the grid reads 16-byte pieces t + k T (k < LOADS, T threads in
// the grid) per round, all LOADS loads in flight together; a grid smaller than
// the buffer strides over it round by round.
template <int LOADS>
__global__ void __launch_bounds__(1024) read_k(const uint4 *__restrict__ p, uint64_t n16, uint32_t *__restrict__ out)
{
    const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += LOADS * T) {
        uint4 v[LOADS];
#pragma unroll
        for (int k = 0; k < LOADS; k++) {
            const uint64_t j = i + k * T;
            v[k] = j < n16 ? p[j] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int k = 0; k < LOADS; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    if (acc == kMagic) out[0] = acc;
}

// gemv_wave's loads without its compute (see qgprobe.h): 16-byte pieces
// copied into LDS by global_load_lds_dwordx4 from inline asm (LDS byte address
// in M0, bound as an operand), waits on this wave's vmcnt only.
constexpr uint32_t kRows = 16, kSlot = 1088;
constexpr uint32_t kWaveLdsBytes = 8u * kRows * kSlot;

__device__ __forceinline__ void dma16(const void *gp, uint32_t lds_addr)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "{m0}"(lds_addr) : "memory");
}

__global__ void __launch_bounds__(512) read_wave_lds_k(const uint8_t *__restrict__ p, uint32_t rows,
                                                       uint32_t row_bytes, uint32_t *__restrict__ out)
{
    extern __shared__ uint4 lds4[];
    uint8_t *lds = (uint8_t *)lds4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t part = row_bytes / 8u, npc = part / 16u;
    const uint32_t off = w * part + 16u * (lane < npc ? lane : npc - 1u);
    const uint32_t reg = w * kRows * kSlot;
    auto issue = [&](uint32_t i) {
        const uint32_t r = min(blockIdx.x + i * gridDim.x, rows - 1u);
        dma16(p + (size_t)r * row_bytes + off, lds0 + reg + i * kSlot);
    };
#pragma unroll
    for (uint32_t i = 0; i < 4u; i++) issue(i);
#pragma unroll 1
    for (uint32_t s = 1; s < kRows / 4u; s++) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");        // step s - 1 landed
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) issue(4u * s + i);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint4 v = *(const uint4 *)(lds + reg + (kRows - 1u) * kSlot + 16u * (lane < npc ? lane : 0u));
    if ((v.x ^ v.y ^ v.z ^ v.w) == kMagic) out[0] = kMagic;
}

bool aligned_all(const void *const *bufs, size_t n)
{
    for (size_t i = 0; i < n; i++)
        if (!bufs[i] || ((uintptr_t)bufs[i] & 15u)) return false;
    return true;
}

}  // namespace

extern "C" int qgp_read(const void *const *bufs, size_t n_bufs, size_t nbytes, uint32_t *d_out, uint32_t threads,
                        uint32_t workgroups, uint32_t loads, size_t n_launches, void *stream)
{
    if (!bufs || n_bufs == 0 || !d_out || nbytes == 0 || nbytes % 16u || threads < 64u || threads > 1024u ||
        threads % 64u || !aligned_all(bufs, n_bufs))
        return -1;
    const void *fn = loads == 1 ? (const void *)read_k<1> : loads == 2 ? (const void *)read_k<2>
                   : loads == 4 ? (const void *)read_k<4> : loads == 8 ? (const void *)read_k<8> : nullptr;
    if (!fn) return -1;
    uint64_t n16 = nbytes / 16u;
    const uint64_t per = (uint64_t)threads * loads;
    const uint64_t grid = workgroups ? workgroups : (n16 + per - 1u) / per;
    if (grid > 0x7FFFFFFFull) return -1;
    for (size_t i = 0; i < n_launches; i++) {
        const uint4 *p = (const uint4 *)bufs[i % n_bufs];
        void *args[] = {&p, &n16, &d_out};
        if (hipLaunchKernel(fn, dim3((uint32_t)grid), dim3(threads), args, 0, (hipStream_t)stream) != hipSuccess)
            return -2;
    }
    return 0;
}

extern "C" int qgp_read_wave_lds(const void *const *bufs, size_t n_bufs, size_t rows, size_t row_bytes,
                                 uint32_t *d_out, size_t n_launches, void *stream)
{
    if (!bufs || n_bufs == 0 || !d_out || rows == 0 || rows > 0x7FFFFFFFull || row_bytes == 0 ||
        row_bytes % 128u || row_bytes > 8192u || !aligned_all(bufs, n_bufs))
        return -1;
    const uint32_t grid = (uint32_t)((rows + kRows - 1u) / kRows);
    uint32_t r32 = (uint32_t)rows, rb = (uint32_t)row_bytes;
    for (size_t i = 0; i < n_launches; i++) {
        const uint8_t *p = (const uint8_t *)bufs[i % n_bufs];
        void *args[] = {&p, &r32, &rb, &d_out};
        if (hipLaunchKernel((const void *)read_wave_lds_k, dim3(grid), dim3(512), args, kWaveLdsBytes,
                            (hipStream_t)stream) != hipSuccess)
            return -2;
    }
    return 0;
}
