// arc_device.hpp -- gfx950 device helpers for the packed Q4_K/Q6_K kernels:
// super-block loads, x staging layout in LDS, in-register unpacking and
// wave64 cross-lane reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace arc {

constexpr int kWave = 64;
constexpr int kQK = 256;         // weights per super-block
constexpr int kQ4Bytes = 144;    // Q4_K super-block
constexpr int kQ6Bytes = 210;    // Q6_K super-block
constexpr int kQ6PBytes = 212;   // Q6_K super-block + 2 zero bytes
constexpr int kFmtQ4 = 12;
constexpr int kFmtQ6 = 14;
constexpr int kFmtQ6P = 214;     // Q6_K with each 210-byte block padded to 212 (dword-aligned blocks)
constexpr int kFmtE148 = 148;    // EXEC148: Q4_K repacked (unpacked scales, codes in element order)
constexpr int kE148Bytes = 148;

// Defined in arc_runtime.cpp.
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
// The library's one hipMalloc call site (counted, see arc_device_allocations).
int device_alloc(void** ptr, size_t bytes, const char* what);
// Device memory a planned arena must leave free for the runtime itself
// (code objects, graph kernel arguments, library workspaces).
constexpr uint64_t kResidencyHeadroom = 512ull << 20;
// ARC_OK when `bytes` more fit in the free device memory with the headroom
// to spare; otherwise ARC_ERR_OUT_OF_MEMORY naming `what`.
int residency_fits(uint64_t bytes, const char* what);

// Decode-step control block in device memory: the graph of one decode step
// reads the position and token from here, and the argmax writes them back.
struct DecodeCtl {
    uint32_t pos;        // position of the token being decoded
    uint32_t token;      // its id
    uint32_t step;       // tokens generated so far in this run
    uint32_t nonfinite;  // non-finite logits seen so far
    uint32_t waits_expired;  // cross-workgroup waits that gave up (an error of the step)
};
struct ArgBest {
    float val;
    uint32_t idx;
    uint32_t nonfinite;
    uint32_t pad;
};

// --------------------------------------------------------------- x staging
// Each super-block column of x is held in LDS as 4 lane slots of 68 floats:
// the 64 x values one lane of a 4-lane "quad" multiplies against (four
// groups of 16 consecutive elements), followed by the 4 group sums.  A quad
// of lanes covers one super-block; slot v belongs to lane v of the quad.
constexpr int kSlot = 68;
constexpr int kXBlk = 4 * kSlot;  // 272 floats per super-block column

// Element offset (within the super-block) of group t (0..3) of lane slot v.
//  Q4_K: lane v owns 16-byte nibble chunks v and v+4; chunk c holds
//        elements (c>>1)*64 + (c&1)*16 + i (low nibbles) and +32 (high).
//  Q6_K: lane v owns ql chunk v of both 128-element halves; it yields
//        quarter qa = v>>1 (low nibbles) and qa+2 (high nibbles), at
//        l = (v&1)*16 + i.
//  EXEC148: lane v owns elements 64v .. 64v+63 (codes in element order),
//        group t = elements 64v + 16t .. +15.
template <int FMT>
__device__ __host__ constexpr int x_group_offset(int v, int t)
{
    if (FMT == kFmtE148) return v * 64 + t * 16;
    if (FMT == kFmtQ4) {
        const int c = v + 4 * (t >> 1);
        return (c >> 1) * 64 + (t & 1) * 32 + (c & 1) * 16;
    } else {
        const int qa = v >> 1;
        const int q = (t & 1) ? qa + 2 : qa;
        return (t >> 1) * 128 + q * 32 + (v & 1) * 16;
    }
}

// ----------------------------------------------------------------- loads
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld16_aligned(const uint8_t* p)
{
    return *reinterpret_cast<const uint4*>(p);
}

// 16 bytes that start `sh` bytes (0 or 2) past the dword-aligned address a4,
// realigned in registers from one dwordx4 and the following dword.  `tail`
// returns that following dword shifted down by sh bytes.  a4 is derived from
// the block pointer by pointer arithmetic so the loads stay global_load.
__device__ __forceinline__ void ld16_shifted(const uint8_t* a4, uint32_t sh, uint32_t out[4], uint32_t& tail)
{
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(a4);
    const uint32_t t = *reinterpret_cast<const uint32_t*>(a4 + 16);
    out[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    out[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    out[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    out[3] = __builtin_amdgcn_alignbyte(t, v.w, sh);
    tail = t >> (8u * sh);
}

// Hides a value from instruction combining: after masking a word of 4-bit
// codes, this keeps the mask as one v_and so each byte converts with a
// single v_cvt_f32_ubyteN (instead of a v_bfe_u32 + v_cvt per element).
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xffffu)));
}

__device__ __forceinline__ float byte_f(uint32_t w, int i)
{
    return static_cast<float>((w >> (8 * i)) & 0xffu);
}

// ------------------------------------------------------------ reductions
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Row exchanges of gfx950 between two registers: v_permlane16_swap swaps
// the odd 16-lane rows of `a` with the even rows of `b`; v_permlane32_swap
// swaps the upper 32 lanes of `a` with the lower 32 of `b`.  Afterwards lane
// l holds a[l] and a[l ^ 16] (resp. ^ 32) where that bit of l is clear, and
// b[l ^ 16] and b[l] where it is set, so a + b is the pairwise sum of `a` in
// the first half of the lanes and of `b` in the other.  Inline asm: the
// compiler's builtins for these return the first result as both results.
// The s_nop pads cover the VALU-write -> permlane-read and permlane-write ->
// VALU-read hazards.
__device__ __forceinline__ void permlane16_swap(uint32_t& a, uint32_t& b)
{
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(uint32_t& a, uint32_t& b)
{
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// v[l] and v[l ^ 16] (XOR=16) or v[l] and v[l ^ 32] (XOR=32), in an order
// that depends on the lane; callers combine them commutatively.
template <int XOR>
__device__ __forceinline__ void xor_pair(float v, float& x, float& y)
{
    static_assert(XOR == 16 || XOR == 32, "row exchanges only");
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    if constexpr (XOR == 16) permlane16_swap(a, b);
    else permlane32_swap(a, b);
    x = __builtin_bit_cast(float, a);
    y = __builtin_bit_cast(float, b);
}
template <int XOR>
__device__ __forceinline__ float xor_sum(float v)
{
    float x, y;
    xor_pair<XOR>(v, x, y);
    return x + y;
}
template <int XOR>
__device__ __forceinline__ float xor_max(float v)
{
    float x, y;
    xor_pair<XOR>(v, x, y);
    return fmaxf(x, y);
}

// Sum over aligned groups of N consecutive lanes (N a power of two <= 64);
// every lane of the group receives the group total.  The combination order
// is fixed, so results are deterministic.
template <int N>
__device__ __forceinline__ float group_sum(float v)
{
    if constexpr (N >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (N >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (N >= 8) v += dpp_f<0x141>(v);   // row_half_mirror: other quad of 8
    if constexpr (N >= 16) v += dpp_f<0x140>(v);  // row_mirror: other 8 of 16
    if constexpr (N >= 32) v = xor_sum<16>(v);
    if constexpr (N >= 64) v = xor_sum<32>(v);
    return v;
}

// Sum over a workgroup of NT threads (fixed order: wave trees, then the
// waves in order); every thread receives the total.
template <int NT>
__device__ inline float block_sum(float v, float* red)
{
    v = group_sum<kWave>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / kWave; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = xor_max<16>(v);
    return xor_max<32>(v);
}

// ----------------------------------------------- cross-workgroup hand-off
// Results one workgroup hands to another inside the same launch go through
// memory with agent-scope relaxed atomics: stores write through the XCD's L2
// (sc1) and loads bypass it, so no L2 writeback or invalidate is needed (an
// agent-scope fence would write back the whole L2 of the XCD).  Nothing ever
// waits for another workgroup: the last one to arrive does the follow-up.
__device__ __forceinline__ void st_agent(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p)
{
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Two consecutive floats (8-byte aligned) in one load.
__device__ __forceinline__ float2 ld_agent2(const float* p)
{
    const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__builtin_bit_cast(float, uint32_t(v)), __builtin_bit_cast(float, uint32_t(v >> 32)));
}

// Called by every thread of the workgroup after its st_agent stores: waits
// until they have reached memory, counts the workgroup in at `counter`, and
// returns true in every thread of the one workgroup that arrives last out of
// `n`.  That workgroup also resets the counter to zero for the next launch.
// `flag` is a workgroup-shared word.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t n, uint32_t* flag)
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1u == n;
        if (last) st_agent(counter, 0u);
        *flag = last ? 1u : 0u;
    }
    __syncthreads();
    return *flag != 0u;
}

// A done counter one part of a launch raises and another part waits for is
// held in kDoneCopies copies kDoneStride words (256 bytes) apart: each
// waiting workgroup polls one copy, so no address takes more than a few
// workgroups' polls (hundreds of workgroups polling one address queue up
// behind each other, and behind the signal, for microseconds).
constexpr int kDoneCopies = 64;
constexpr int kDoneStride = 64;

// Called by every thread of the workgroup after its st_agent stores: waits
// until they have reached memory, then counts the workgroup in at each of
// `copies` (<= 64) copies of a counter, `stride` words apart (one part of a
// launch telling another that its results are readable; each waiter polls
// one copy, so no single address takes every poll).
__device__ __forceinline__ void signal_done(uint32_t* counter, uint32_t copies, uint32_t stride)
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x < copies)
        __hip_atomic_fetch_add(counter + threadIdx.x * stride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of the workgroup: waits until `counter` reaches n,
// one thread polling with a short sleep between polls, at most kWaitPolls
// polls (tens of milliseconds; a wait that long is an error the caller
// reports).  Returns false when it gave up.  Only launches whose waiting
// workgroups come after the ones they wait for in dispatch order, and fit on
// the device together with them, wait at all.
constexpr uint32_t kWaitPolls = 1u << 16;
__device__ __forceinline__ bool wait_count(const uint32_t* counter, uint32_t n, uint32_t* flag)
{
    if (threadIdx.x == 0) {
        uint32_t i = 0;
        while (ld_agent(counter) < n && ++i < kWaitPolls) __builtin_amdgcn_s_sleep(2);
        *flag = i < kWaitPolls ? 1u : 0u;
    }
    __syncthreads();
    return *flag != 0u;
}

}  // namespace arc
