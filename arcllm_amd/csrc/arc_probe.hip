// arc_probe.hip -- streaming-read probe: the practical HBM read ceiling of
// the device for a given buffer size, used by bench.py to put the GEMV
// numbers next to what a plain coalesced read achieves on the same box.
#include "../../include/arcllm_hip.h"

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace arc {
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

// Each lane reads 16-byte chunks in a grid-stride loop (one 1 KB coalesced
// access per wave instruction) and folds them with xor; one store per lane.
__global__ __launch_bounds__(256) void k_probe_read(const uint4* __restrict__ p, uint64_t n16,
                                                    uint32_t* __restrict__ out)
{
    uint64_t i = blockIdx.x * 256ull + threadIdx.x;
    const uint64_t stride = gridDim.x * 256ull;
    uint32_t acc = 0;
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[blockIdx.x * 256u + threadIdx.x] = acc;
}

// The same read with U independent 16-byte loads in flight per lane: each
// iteration issues the loads of U consecutive grid strides before folding
// any of them (indices past the end are clamped to the last chunk, read
// again and folded like the others).
template <int U>
__global__ __launch_bounds__(256) void k_probe_read_u(const uint4* __restrict__ p, uint64_t n16,
                                                      uint32_t* __restrict__ out)
{
    uint64_t i = blockIdx.x * 256ull + threadIdx.x;
    const uint64_t stride = gridDim.x * 256ull;
    uint32_t acc = 0;
    for (; i < n16; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + u * stride;
            v[u] = p[j < n16 ? j : n16 - 1];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    out[blockIdx.x * 256u + threadIdx.x] = acc;
}
// The one-load read with the non-temporal cache policy (`nt`): a plain
// stream reads each line once, so keeping it out of the caches' replacement
// order is free, and on MI355X it streams a few per cent faster.
__global__ __launch_bounds__(256) void k_probe_read_nt(const uint4* __restrict__ p, uint64_t n16,
                                                       uint32_t* __restrict__ out)
{
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v* q = reinterpret_cast<const u32x4v*>(p);
    uint64_t i = blockIdx.x * 256ull + threadIdx.x;
    const uint64_t stride = gridDim.x * 256ull;
    uint32_t acc = 0;
    for (; i < n16; i += stride) {
        const u32x4v v = __builtin_nontemporal_load(q + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[blockIdx.x * 256u + threadIdx.x] = acc;
}
}  // namespace arc

extern "C" int arc_probe_read_nt(const void* p, size_t bytes, uint32_t* out, uint32_t grid, arc_stream_t stream)
{
    if (!p || !out || bytes < 16 || grid == 0 || grid > 65536)
        return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "bad probe arguments");
    if (reinterpret_cast<uintptr_t>(p) & 15u) return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "probe buffer not 16-byte aligned");
    hipLaunchKernelGGL(arc::k_probe_read_nt, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(p), uint64_t(bytes / 16), out);
    return arc::check_hip(hipGetLastError(), "probe launch");
}

extern "C" int arc_probe_read(const void* p, size_t bytes, uint32_t* out, uint32_t grid, arc_stream_t stream)
{
    if (!p || !out || bytes < 16 || grid == 0 || grid > 65536)
        return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "bad probe arguments");
    if (reinterpret_cast<uintptr_t>(p) & 15u) return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "probe buffer not 16-byte aligned");
    hipLaunchKernelGGL(arc::k_probe_read, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(p), uint64_t(bytes / 16), out);
    return arc::check_hip(hipGetLastError(), "probe launch");
}

extern "C" int arc_probe_read_unrolled(const void* p, size_t bytes, uint32_t* out, uint32_t grid, int loads,
                                       arc_stream_t stream)
{
    if (!p || !out || bytes < 16 || grid == 0 || grid > 65536)
        return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "bad probe arguments");
    if (reinterpret_cast<uintptr_t>(p) & 15u) return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "probe buffer not 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint64_t n16 = uint64_t(bytes / 16);
    const uint4* q = static_cast<const uint4*>(p);
    switch (loads) {
    case 1: hipLaunchKernelGGL(arc::k_probe_read_u<1>, dim3(grid), dim3(256), 0, s, q, n16, out); break;
    case 2: hipLaunchKernelGGL(arc::k_probe_read_u<2>, dim3(grid), dim3(256), 0, s, q, n16, out); break;
    case 4: hipLaunchKernelGGL(arc::k_probe_read_u<4>, dim3(grid), dim3(256), 0, s, q, n16, out); break;
    case 8: hipLaunchKernelGGL(arc::k_probe_read_u<8>, dim3(grid), dim3(256), 0, s, q, n16, out); break;
    default: return arc::set_error(ARC_ERR_INVALID_ARGUMENT, "loads per iteration must be 1, 2, 4 or 8");
    }
    return arc::check_hip(hipGetLastError(), "probe launch");
}
