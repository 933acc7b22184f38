// arc_exec148.hip -- the EXEC148 representation of a Q4_K tensor on gfx950:
// the repack (the reference's P1 path, shaders/b1_2_exec148_gpu_materialize.comp
// driven by src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:120-141) and its
// exact validation (the per-block half of validate_tensor,
// src/q4_down_exec148_materializer.h:21-22).
//
// EXEC148 block (148 bytes): bytes 0..3 the Q4_K block's d and dmin, bytes
// 4 + 2j, 5 + 2j the unpacked 6-bit (sc_j, mn_j), bytes 20 + p the codes of
// elements 2p (low nibble) and 2p + 1 (high nibble).
//
// Both kernels are HBM-bound byte work.  A workgroup handles 256 consecutive
// blocks, one per thread: each thread reads its 144-byte source block with
// nine 16-byte loads (the workgroup's loads cover its 36,864 source bytes
// contiguously), repacks it in registers and writes the 37 result dwords to
// LDS at a 37-dword stride (odd: conflict-free); the workgroup's 37,888
// result bytes then leave LDS in destination order with coalesced 16-byte
// accesses, written (repack) or compared with the destination (validation).
// The validation compares whole blocks: an EXEC148 block's canonical tuple
// (d and dmin bytes, the (sc, mn) bytes, every code nibble) holds every bit
// of the block, so equal tuples mean equal bytes.
#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

namespace arc {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kE148PerWg = 256;                     // blocks per workgroup
constexpr uint32_t kSrcPieces = kQ4Bytes / 16;           // 9 x 16 bytes per Q4_K block
constexpr uint32_t kDstWords = kE148Bytes / 4;           // 37 dwords per EXEC148 block

// Two code bytes per output byte: for output dword m of 64-element group g
// (bytes 32g + 4m .. +3), m < 4 pairs the low nibbles of source bytes
// 8m .. 8m+7 of the group, m >= 4 the high nibbles of bytes 8(m-4) .. +7.
// n = the source dword's nibbles of the plane, one per byte (0x0f0f0f0f
// lanes): byte i of the result pair is n_{2i} | n_{2i+1} << 4 (in bytes 0, 2).
__device__ __forceinline__ uint32_t pair_nibbles(uint32_t n) { return (n | (n >> 4)) & 0x00ff00ffu; }

// The EXEC148 block of the Q4_K block held in `in` (36 dwords) as 37 dwords.
__device__ __forceinline__ void repack_block(const uint32_t (&in)[36], uint32_t* out)
{
    out[0] = in[0];  // d, dmin
    const uint32_t s0 = in[1], s1 = in[2], s2 = in[3];  // scale bytes 4..15
    auto byte = [&](uint32_t i) { return ((i < 4 ? s0 : i < 8 ? s1 : s2) >> (8 * (i & 3))) & 0xffu; };
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
            const uint32_t j = 2 * w + h;
            uint32_t sc, mn;
            if (j < 4) {
                sc = byte(j) & 63u;
                mn = byte(j + 4) & 63u;
            } else {
                sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
                mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
            }
            v |= (sc | (mn << 8)) << (16 * h);
        }
        out[1 + w] = v;
    }
#pragma unroll
    for (uint32_t g = 0; g < 4; ++g)
#pragma unroll
        for (uint32_t m = 0; m < 8; ++m) {
            const uint32_t a = in[4 + 8 * g + 2 * (m & 3)], b = in[4 + 8 * g + 2 * (m & 3) + 1];
            const uint32_t sh = m < 4 ? 0u : 4u;
            const uint32_t pa = pair_nibbles((a >> sh) & 0x0f0f0f0fu), pb = pair_nibbles((b >> sh) & 0x0f0f0f0fu);
            out[5 + 8 * g + m] =
                (pa & 0xffu) | ((pa >> 8) & 0xff00u) | ((pb & 0xffu) << 16) | (((pb >> 16) & 0xffu) << 24);
        }
}

// Repacks this thread's block into out_lds (37-dword stride); returns the
// number of blocks of the workgroup.
__device__ __forceinline__ uint32_t repack_to_lds(const uint8_t* __restrict__ src, uint64_t nblocks, uint32_t* out_lds)
{
    const uint64_t b0 = uint64_t(blockIdx.x) * kE148PerWg;
    const uint32_t nb = uint32_t(min(uint64_t(kE148PerWg), nblocks - b0));
    if (threadIdx.x < nb) {
        const u32x4* g = reinterpret_cast<const u32x4*>(src + (b0 + threadIdx.x) * kQ4Bytes);
        uint32_t in[36];
#pragma unroll
        for (uint32_t p = 0; p < kSrcPieces; ++p) {
            const u32x4 v = g[p];
            in[4 * p] = v.x, in[4 * p + 1] = v.y, in[4 * p + 2] = v.z, in[4 * p + 3] = v.w;
        }
        repack_block(in, out_lds + threadIdx.x * kDstWords);
    }
    __syncthreads();
    return nb;
}

__global__ __launch_bounds__(256) void k_exec148_materialize(const uint8_t* __restrict__ src, uint64_t nblocks,
                                                             uint8_t* __restrict__ dst)
{
    __shared__ __align__(16) uint32_t out_lds[kE148PerWg * kDstWords];
    const uint32_t nb = repack_to_lds(src, nblocks, out_lds);
    // the workgroup's destination starts at a multiple of 256 * 148 bytes (16-byte aligned)
    uint32_t* g = reinterpret_cast<uint32_t*>(dst + uint64_t(blockIdx.x) * kE148PerWg * kE148Bytes);
    const uint32_t words = nb * kDstWords, quads = words / 4;
    for (uint32_t i = threadIdx.x; i < quads; i += kE148PerWg)
        reinterpret_cast<u32x4*>(g)[i] = reinterpret_cast<const u32x4*>(out_lds)[i];
    for (uint32_t i = quads * 4 + threadIdx.x; i < words; i += kE148PerWg) g[i] = out_lds[i];
}

// mismatched[0] += number of this workgroup's EXEC148 blocks that differ from
// the repack of their source block.
__global__ __launch_bounds__(256) void k_exec148_validate(const uint8_t* __restrict__ src,
                                                          const uint8_t* __restrict__ exec, uint64_t nblocks,
                                                          unsigned long long* __restrict__ mismatched)
{
    __shared__ __align__(16) uint32_t out_lds[kE148PerWg * kDstWords];
    __shared__ uint32_t bad[kE148PerWg];
    bad[threadIdx.x] = 0;
    const uint32_t nb = repack_to_lds(src, nblocks, out_lds);
    const uint32_t* g = reinterpret_cast<const uint32_t*>(exec + uint64_t(blockIdx.x) * kE148PerWg * kE148Bytes);
    const uint32_t words = nb * kDstWords, quads = words / 4;
    for (uint32_t i = threadIdx.x; i < quads; i += kE148PerWg) {
        const u32x4 x = reinterpret_cast<const u32x4*>(g)[i], y = reinterpret_cast<const u32x4*>(out_lds)[i];
        if (x.x != y.x) bad[(4 * i) / kDstWords] = 1;
        if (x.y != y.y) bad[(4 * i + 1) / kDstWords] = 1;
        if (x.z != y.z) bad[(4 * i + 2) / kDstWords] = 1;
        if (x.w != y.w) bad[(4 * i + 3) / kDstWords] = 1;
    }
    for (uint32_t i = quads * 4 + threadIdx.x; i < words; i += kE148PerWg)
        if (g[i] != out_lds[i]) bad[i / kDstWords] = 1;
    __syncthreads();
    const uint32_t n = uint32_t(__syncthreads_count(threadIdx.x < nb && bad[threadIdx.x] != 0));
    if (threadIdx.x == 0 && n) atomicAdd(mismatched, static_cast<unsigned long long>(n));
}

// The validation's mismatch counter: one per device, in static device memory,
// so a validation allocates nothing.  Calls hold g_count_mu from clearing it
// to reading it back (validation is synchronous), so they never share it.
static __device__ __align__(256) unsigned long long g_mismatch_count;

}  // namespace arc

using namespace arc;

namespace {

constexpr int kMaxCountDevices = 64;
std::mutex g_count_mu;
unsigned long long* g_count_ptr[kMaxCountDevices];

// Device address of g_mismatch_count on the current device (looked up once
// per device with it current).  Call with g_count_mu held.
int mismatch_counter(unsigned long long** out)
{
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "current device");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxCountDevices) return set_error(ARC_ERR_UNSUPPORTED, "device %d out of range", dev);
    if (!g_count_ptr[dev]) {
        void* ptr = nullptr;
        if ((rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_mismatch_count)), "validate counter address")))
            return rc;
        if (!ptr) return set_error(ARC_ERR_DEVICE, "no device address for the validate counter");
        g_count_ptr[dev] = static_cast<unsigned long long*>(ptr);
    }
    *out = g_count_ptr[dev];
    return ARC_OK;
}

int check_e148(const void* q4, uint32_t rows, uint32_t K, const void* exec, uint64_t& nblocks)
{
    if (!q4 || !exec) return set_error(ARC_ERR_INVALID_ARGUMENT, "null tensor pointer");
    if (rows == 0 || K == 0 || K % kQK)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad shape rows=%u K=%u (K must be a nonzero multiple of 256)", rows,
                         K);
    if (reinterpret_cast<uintptr_t>(q4) & 15u) return set_error(ARC_ERR_INVALID_ARGUMENT, "Q4_K tensor not 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(exec) & 15u)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "EXEC148 tensor not 16-byte aligned");
    nblocks = uint64_t(rows) * (K / kQK);
    if ((nblocks + kE148PerWg - 1) / kE148PerWg > 0x7fffffffull)
        return set_error(ARC_ERR_UNSUPPORTED, "tensor too large for one launch");
    return ARC_OK;
}

}  // namespace

extern "C" {

int arc_exec148_materialize(const void* q4, uint32_t rows, uint32_t K, void* exec, arc_stream_t stream)
{
    uint64_t nb = 0;
    const int rc = check_e148(q4, rows, K, exec, nb);
    if (rc) return rc;
    hipLaunchKernelGGL(k_exec148_materialize, dim3(uint32_t((nb + kE148PerWg - 1) / kE148PerWg)), dim3(kE148PerWg), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(q4), nb,
                       static_cast<uint8_t*>(exec));
    return check_hip(hipGetLastError(), "exec148 materialize");
}

int arc_exec148_validate_many(const void* const* q4, const void* const* exec, uint32_t count, uint32_t rows,
                              uint32_t K, uint64_t* mismatched, arc_stream_t stream)
{
    if (!q4 || !exec || !mismatched || count == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad validate arguments");
    uint64_t nb = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const int rc = check_e148(q4[i], rows, K, exec[i], nb);
        if (rc) return rc;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lock(g_count_mu);
    unsigned long long* cnt = nullptr;
    int rc = mismatch_counter(&cnt);
    if (rc) return rc;
    unsigned long long host = 0;
    rc = check_hip(hipMemcpyAsync(cnt, &host, sizeof(host), hipMemcpyHostToDevice, s), "exec148 validate clear");
    // one counter for every tensor, one synchronization at the end
    for (uint32_t i = 0; i < count && !rc; ++i) {
        hipLaunchKernelGGL(k_exec148_validate, dim3(uint32_t((nb + kE148PerWg - 1) / kE148PerWg)), dim3(kE148PerWg),
                           0, s, static_cast<const uint8_t*>(q4[i]), static_cast<const uint8_t*>(exec[i]), nb, cnt);
        rc = check_hip(hipGetLastError(), "exec148 validate");
    }
    if (!rc) rc = check_hip(hipMemcpyAsync(&host, cnt, sizeof(host), hipMemcpyDeviceToHost, s), "exec148 validate result");
    // on an error the wait still runs, so no launch outlives the lock
    const int sync = check_hip(hipStreamSynchronize(s), "exec148 validate sync");
    if (!rc) rc = sync;
    if (!rc) *mismatched = host;
    return rc;
}

int arc_exec148_validate(const void* q4, const void* exec, uint32_t rows, uint32_t K, uint64_t* mismatched,
                         arc_stream_t stream)
{
    return arc_exec148_validate_many(&q4, &exec, 1, rows, K, mismatched, stream);
}

}  // extern "C"
