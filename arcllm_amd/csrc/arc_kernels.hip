// arc_kernels.hip -- hand-written gfx950 kernels for the packed Q4_K/Q6_K
// decode hot path and their C-ABI launchers (include/arcllm_hip.h).
//
// GEMV structure (all formats and epilogues share it):
//  * A quad of 4 lanes covers one super-block of one row; lane v of the quad
//    loads 16-byte pieces of the block (Q4_K: header + nibble chunks v, v+4;
//    Q6_K: ql chunk v of both halves, the matching qh chunks, scales and d),
//    unpacks the codes in registers and multiplies 64 weights.
//  * BS quads of a row-group split the row's super-blocks round-robin, so a
//    row is reduced over 4*BS lanes with DPP (deterministic fixed tree).
//  * Each lane carries RPL rows (and both matrices of the fused gate/up), so
//    one LDS read of x feeds RPL*NMAT rows.
//  * x is staged once per workgroup into LDS, permuted so each lane reads 64
//    contiguous floats per block, with the four 16-element group sums that
//    fold the Q4_K min and the Q6_K -32 offset out of the inner loop:
//      Q4_K: sum_k (d sc q - dmin mn) x = d sum_g sc_g (q.x)_g - dmin sum_g mn_g (sum x)_g
//      Q6_K: sum_k d sc (u - 32) x      = d sum_g sc_g ((u.x)_g - 32 (sum x)_g)
//  * Workgroups are persistent: each wave strides over "wave tiles" of
//    RG*RPL rows, and walks the flattened (tile, super-block) sequence with
//    two register buffers, so the loads of the next super-block -- also
//    across tile boundaries -- are in flight while the current one is used.
#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

namespace arc {

// Defined in arc_runtime.cpp.
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

constexpr int kPanel = 80;  // max super-block columns of x staged per launch (87 KB LDS)
constexpr int kWaves = 4;   // waves per GEMV workgroup
constexpr int kThreads = kWaves * kWave;

// EPI_COLPART: split-K with one super-block column per split -- each quad's
// own sum is the partial of (column, row), written without a cross-quad
// reduction, so every column of a row is handled by one launch.
enum Epi { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_PARTIAL = 2, EPI_ARGMAX = 3, EPI_COLPART = 4 };
enum Flag : uint32_t { F_NORM = 1u, F_ACCUM = 2u, F_BIAS = 4u };

struct ArgBest {
    float val;
    uint32_t idx;
    uint32_t nonfinite;
    uint32_t pad;
};

struct GemvParams {
    const uint8_t* w0;
    const uint8_t* w1;
    uint64_t row_bytes;
    uint32_t rows;
    uint32_t nb;         // super-blocks per full row (RMSNorm length = nb*256)
    uint32_t split_bps;  // super-block columns per split (grid.y = splits)
    uint32_t kb_off;     // first column of this launch inside each split
    uint32_t panel;      // max columns handled by this launch (<= kPanel)
    uint32_t ntiles;     // wave tiles = ceil(rows / (RG*RPL))
    uint32_t flags;      // F_NORM | F_ACCUM | F_BIAS
    uint32_t nsplit;     // partial columns per row (split-K outputs)
    float eps;
    const float* x;
    const float* normw;
    const float* bias;
    float* y;
    ArgBest* best;
};

// ------------------------------------------------------------ block loads
struct Q4Blk {
    uint4 hdr, qa, qb;
};

__device__ __forceinline__ void q4_load(const uint8_t* blk, int v, Q4Blk& o)
{
    o.hdr = ld16_aligned(blk);
    o.qa = ld16_aligned(blk + 16 + v * 16);
    o.qb = ld16_aligned(blk + 80 + v * 16);
}

struct Q6Blk {
    uint32_t ql[2][4];
    uint32_t qh[2][4];
    uint32_t sc[4];
    uint32_t d;
};

// A Q6_K block starts 0 or 2 bytes past a dword boundary.  Every chunk offset
// used here is a multiple of 4, so each chunk is read as a dwordx4 plus one
// dword from the dword-aligned block base and shifted in registers.  The
// dwords read cover block bytes [o-2, o+18) for o <= 192: each one holds at
// least one byte of the block itself, so no read reaches a page the tensor
// does not touch.
__device__ __forceinline__ void q6_load(const uint8_t* blk, int v, Q6Blk& o)
{
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
    const uint8_t* b = blk - sh;
    uint32_t t;
    ld16_shifted(b + v * 16, sh, o.ql[0], t);
    ld16_shifted(b + 64 + v * 16, sh, o.ql[1], t);
    ld16_shifted(b + 128 + (v & 1) * 16, sh, o.qh[0], t);
    ld16_shifted(b + 160 + (v & 1) * 16, sh, o.qh[1], t);
    ld16_shifted(b + 192, sh, o.sc, t);
    o.d = t & 0xffffu;
}

template <int FMT>
struct BlkOf;
template <>
struct BlkOf<kFmtQ4> {
    using T = Q4Blk;
    static constexpr int bytes = kQ4Bytes;
};
template <>
struct BlkOf<kFmtQ6> {
    using T = Q6Blk;
    static constexpr int bytes = kQ6Bytes;
};

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// acc + h*x with h one fp16 half of `pair` (v_fma_mix_f32: fp16 operand,
// fp32 x and accumulator).  Codes are placed in the low bits of an fp16
// half, which makes them exact subnormals: bits q read as q * 2^-24.
__device__ __forceinline__ float fmix(uint32_t pair, bool hi, float x, float acc)
{
    const half2_t h = __builtin_bit_cast(half2_t, pair);
    return __builtin_fmaf(static_cast<float>(hi ? h.y : h.x), x, acc);
}

// acc += sum over the 4 bytes of `codes` (values < 1024 >> 4 = 64) of
// byte_i * 2^-24 * x_i: bytes 0,2 from the even halves, bytes 1,3 moved
// down with v_perm_b32.
__device__ __forceinline__ float mix4(uint32_t codes, const float4& x, float acc)
{
    const uint32_t ev = opaque(codes & 0x00ff00ffu);
    const uint32_t od = opaque(__builtin_amdgcn_perm(0u, codes, 0x0c030c01u));  // [b1, 0, b3, 0]
    acc = fmix(ev, false, x.x, acc);
    acc = fmix(od, false, x.y, acc);
    acc = fmix(ev, true, x.z, acc);
    acc = fmix(od, true, x.w, acc);
    return acc;
}

__device__ __forceinline__ uint32_t comp(const uint4& q, int i)
{
    return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Dot of N Q4_K blocks (same column, different rows/matrices) with the
// lane's 64 x values; adds d*sum(sc*qx) - dmin*sum(mn*sx) into acc[n].
// Low nibbles are read as fp16 subnormals q*2^-24 (w & 0x000f000f), high
// nibbles as q*2^-20 (w & 0x00f000f0); the staged x carries the inverse
// power of two.
template <int N>
__device__ __forceinline__ void q4_dot(const Q4Blk (&b)[N], const float* xs, int v, float (&acc)[N])
{
    float a[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) a[n][0] = a[n][1] = a[n][2] = a[n][3] = 0.0f;
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
        const float4 x0 = lds4(xs + dw * 4);
        const float4 x1 = lds4(xs + 16 + dw * 4);
        const float4 x2 = lds4(xs + 32 + dw * 4);
        const float4 x3 = lds4(xs + 48 + dw * 4);
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const uint32_t qa = comp(b[n].qa, dw), qb = comp(b[n].qb, dw);
            const uint32_t qa8 = qa >> 8, qb8 = qb >> 8;
            const uint32_t aL = opaque(qa & 0x000f000fu), aLo = opaque(qa8 & 0x000f000fu);
            const uint32_t aH = opaque(qa & 0x00f000f0u), aHo = opaque(qa8 & 0x00f000f0u);
            const uint32_t bL = opaque(qb & 0x000f000fu), bLo = opaque(qb8 & 0x000f000fu);
            const uint32_t bH = opaque(qb & 0x00f000f0u), bHo = opaque(qb8 & 0x00f000f0u);
            a[n][0] = fmix(aL, false, x0.x, a[n][0]);
            a[n][0] = fmix(aLo, false, x0.y, a[n][0]);
            a[n][0] = fmix(aL, true, x0.z, a[n][0]);
            a[n][0] = fmix(aLo, true, x0.w, a[n][0]);
            a[n][1] = fmix(aH, false, x1.x, a[n][1]);
            a[n][1] = fmix(aHo, false, x1.y, a[n][1]);
            a[n][1] = fmix(aH, true, x1.z, a[n][1]);
            a[n][1] = fmix(aHo, true, x1.w, a[n][1]);
            a[n][2] = fmix(bL, false, x2.x, a[n][2]);
            a[n][2] = fmix(bLo, false, x2.y, a[n][2]);
            a[n][2] = fmix(bL, true, x2.z, a[n][2]);
            a[n][2] = fmix(bLo, true, x2.w, a[n][2]);
            a[n][3] = fmix(bH, false, x3.x, a[n][3]);
            a[n][3] = fmix(bHo, false, x3.y, a[n][3]);
            a[n][3] = fmix(bH, true, x3.z, a[n][3]);
            a[n][3] = fmix(bHo, true, x3.w, a[n][3]);
        }
    }
    const float4 S = lds4(xs + 64);
    const int sh = 16 * (v >> 1);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        // bytes of sc/mn for this lane's sub-blocks (2g, 2g+1, 2g+4, 2g+5), g = v>>1
        const uint32_t yy = b[n].hdr.y >> sh, zz = b[n].hdr.z >> sh, ww = b[n].hdr.w >> sh;
        const uint32_t SC = (yy & 0x3f3fu) | (((ww & 0x0f0fu) | ((yy >> 2) & 0x3030u)) << 16);
        const uint32_t MN = (zz & 0x3f3fu) | ((((ww >> 4) & 0x0f0fu) | ((zz >> 2) & 0x3030u)) << 16);
        float qs = byte_f(SC, 0) * a[n][0];
        qs = __builtin_fmaf(byte_f(SC, 1), a[n][1], qs);
        qs = __builtin_fmaf(byte_f(SC, 2), a[n][2], qs);
        qs = __builtin_fmaf(byte_f(SC, 3), a[n][3], qs);
        float ms = byte_f(MN, 0) * S.x;
        ms = __builtin_fmaf(byte_f(MN, 1), S.y, ms);
        ms = __builtin_fmaf(byte_f(MN, 2), S.z, ms);
        ms = __builtin_fmaf(byte_f(MN, 3), S.w, ms);
        acc[n] = fmix(b[n].hdr.x, false, qs, acc[n]);   // + d * qs
        acc[n] = fmix(b[n].hdr.x, true, -ms, acc[n]);   // - dmin * ms
    }
}

// Q6_K: the 6-bit codes u of one ql/qh dword pair are assembled per byte,
// ua = low nibbles | bits (2qa, 2qa+1) of qh moved to bits 4-5, ub = high
// nibbles | bits (2qa+4, 2qa+5); then read as fp16 subnormals u*2^-24 (the
// staged x carries 2^24).
template <int N>
__device__ __forceinline__ void q6_dot(const Q6Blk (&b)[N], const float* xs, int v, float (&acc)[N])
{
    const int qa = v >> 1;
    const uint32_t s1 = 4u - 2u * qa, s2 = 2u * qa;
    float a[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) a[n][0] = a[n][1] = a[n][2] = a[n][3] = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const float4 xa = lds4(xs + (2 * h) * 16 + dw * 4);
            const float4 xb = lds4(xs + (2 * h + 1) * 16 + dw * 4);
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint32_t ql = b[n].ql[h][dw], qh = b[n].qh[h][dw];
                const uint32_t ua = (ql & 0x0f0f0f0fu) | ((qh << s1) & 0x30303030u);
                const uint32_t ub = ((ql >> 4) & 0x0f0f0f0fu) | ((qh >> s2) & 0x30303030u);
                a[n][2 * h] = mix4(ua, xa, a[n][2 * h]);
                a[n][2 * h + 1] = mix4(ub, xb, a[n][2 * h + 1]);
            }
        }
    }
    const float4 S = lds4(xs + 64);
    // scale of group t is byte i0 of scale dword t (i0 = (v&1) + 2*qa)
    const uint32_t i0 = 8u * ((v & 1) + 2 * qa);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        float t = float(int8_t(uint8_t(b[n].sc[0] >> i0))) * __builtin_fmaf(-32.0f, S.x, a[n][0]);
        t = __builtin_fmaf(float(int8_t(uint8_t(b[n].sc[1] >> i0))), __builtin_fmaf(-32.0f, S.y, a[n][1]), t);
        t = __builtin_fmaf(float(int8_t(uint8_t(b[n].sc[2] >> i0))), __builtin_fmaf(-32.0f, S.z, a[n][2]), t);
        t = __builtin_fmaf(float(int8_t(uint8_t(b[n].sc[3] >> i0))), __builtin_fmaf(-32.0f, S.w, a[n][3]), t);
        acc[n] = fmix(b[n].d, false, t, acc[n]);  // + d * t
    }
}

template <int FMT, int N>
__device__ __forceinline__ void blk_dot(const typename BlkOf<FMT>::T (&b)[N], const float* xs, int v,
                                        float (&acc)[N])
{
    if constexpr (FMT == kFmtQ4)
        q4_dot<N>(b, xs, v, acc);
    else
        q6_dot<N>(b, xs, v, acc);
}

template <int FMT>
__device__ __forceinline__ void blk_load(const uint8_t* blk, int v, typename BlkOf<FMT>::T& o)
{
    if constexpr (FMT == kFmtQ4)
        q4_load(blk, v, o);
    else
        q6_load(blk, v, o);
}

// ------------------------------------------------------------- reductions
template <int NT>
__device__ float block_sum(float v, float* red)
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

// 1/sqrt(mean(x^2) + eps) over n elements, fp32, fixed reduction order.
template <int NT>
__device__ float rms_inv(const float* x, uint32_t n, float eps, float* red)
{
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += NT) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = block_sum<NT>(ss, red);
    return 1.0f / sqrtf(ss / float(n) + eps);
}

// ------------------------------------------------------------- x staging
// Stage super-block columns [b0, b0+nbl) of x into LDS (layout in
// arc_device.hpp).  With norm, x is replaced by (x*inv)*normw.  The group
// sums are of x itself; the staged x values are pre-multiplied by the
// power of two that undoes the unit in which the dot loops read codes as
// fp16 subnormals (2^-24 for codes in bits 0..5, 2^-20 for Q4_K high
// nibbles in bits 4..7), which is exact.
template <int FMT, int NT>
__device__ void stage_x(float* lds, const float* __restrict__ x, uint32_t b0, uint32_t nbl, bool norm,
                        float inv, const float* __restrict__ normw)
{
    for (uint32_t gi = threadIdx.x; gi < nbl * 16u; gi += NT) {
        const uint32_t bl = gi >> 4, v = (gi >> 2) & 3u, t = gi & 3u;
        const uint32_t e = (b0 + bl) * kQK + x_group_offset<FMT>(int(v), int(t));
        const float4* src = reinterpret_cast<const float4*>(x + e);
        float4 q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = src[i];
        if (norm) {
            const float4* nw = reinterpret_cast<const float4*>(normw + e);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 w = nw[i];
                q[i].x = (q[i].x * inv) * w.x;
                q[i].y = (q[i].y * inv) * w.y;
                q[i].z = (q[i].z * inv) * w.z;
                q[i].w = (q[i].w * inv) * w.w;
            }
        }
        float* dst = lds + bl * kXBlk + v * kSlot + t * 16;
        const float unit = (FMT == kFmtQ4 && (t & 1u)) ? 1048576.0f : 16777216.0f;  // 2^20 : 2^24
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s += q[i].x;
            s += q[i].y;
            s += q[i].z;
            s += q[i].w;
            reinterpret_cast<float4*>(dst)[i] = make_float4(q[i].x * unit, q[i].y * unit, q[i].z * unit, q[i].w * unit);
        }
        lds[bl * kXBlk + v * kSlot + 64 + t] = s;
    }
}

__device__ __forceinline__ bool arg_better(float va, uint32_t ia, float vb, uint32_t ib)
{
    return va > vb || (va == vb && ia < ib);
}

// Argmax over a workgroup of (value, index) candidates, ties to the lowest
// index, plus a sum of the non-finite counts.  Called by every thread.
__device__ void wg_argmax(float bv, uint32_t bi, uint32_t nf, ArgBest* out)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        const uint32_t on = __shfl_xor(nf, off);
        if (oi != 0xffffffffu && arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
        nf += on;
    }
    __shared__ float sv[16];
    __shared__ uint32_t si[16], sn[16];
    const int nw = blockDim.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
        sn[wave] = nf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sv[0];
        uint32_t i = si[0], c = sn[0];
        for (int w = 1; w < nw; ++w) {
            if (si[w] != 0xffffffffu && arg_better(sv[w], si[w], b, i)) {
                b = sv[w];
                i = si[w];
            }
            c += sn[w];
        }
        *out = ArgBest{b, i, c, 0u};
    }
}

// --------------------------------------------------------------- GEMV core
template <int FMT, int BS, int RPL, int EPI>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvParams p)
{
    extern __shared__ float lds[];
    __shared__ float red[kWaves];
    constexpr int NMAT = (EPI == EPI_SWIGLU) ? 2 : 1;
    constexpr int N = NMAT * RPL;
    constexpr int RG = kWave / (4 * BS);
    constexpr int kTileRows = RG * RPL;
    using Blk = typename BlkOf<FMT>::T;
    constexpr int kBB = BlkOf<FMT>::bytes;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v = lane & 3, bs = (lane >> 2) % BS, rg = lane / (4 * BS);

    // super-block columns [kb, kb + nbl) of this split and launch
    const uint32_t split = blockIdx.y;
    const uint32_t kb = split * p.split_bps + p.kb_off;
    const uint32_t split_end = min((split + 1) * p.split_bps, p.nb);
    if (kb >= split_end) return;  // whole workgroup: this panel is past the split's end
    const uint32_t nbl = min(p.panel, split_end - kb);
    const uint32_t nj = (nbl + BS - 1) / BS;  // block slots per tile, uniform over the wave

    const uint32_t gw = blockIdx.x * kWaves + wave;
    const uint32_t stride = gridDim.x * kWaves;
    const uint32_t my_tiles = gw < p.ntiles ? (p.ntiles - gw + stride - 1) / stride : 0u;
    const uint32_t S = my_tiles * nj;

    auto tile_row = [&](uint32_t tile, int j) { return tile * kTileRows + rg * RPL + j; };
    // Loads are issued unconditionally (indices clamped to valid blocks and
    // rows) so the compiler can count the outstanding loads exactly and wait
    // only for the buffer being consumed, never for the prefetch in flight.
    auto load = [&](uint32_t ti, uint32_t j, Blk (&b)[N]) {
        const uint32_t bl = min(bs + BS * j, nbl - 1);
        const uint32_t tile = min(gw + ti * stride, p.ntiles - 1);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                const uint32_t row = min(tile_row(tile, r), p.rows - 1);  // clamp: result discarded
                const uint8_t* base = (m == 0 ? p.w0 : p.w1) + uint64_t(row) * p.row_bytes + uint64_t(kb + bl) * kBB;
                blk_load<FMT>(base, v, b[m * RPL + r]);
            }
        }
    };

    Blk bufA[N], bufB[N];
    load(0, 0, bufA);  // weight fetch overlaps the x staging below

    float inv = 1.0f;
    if (p.flags & F_NORM) inv = rms_inv<kThreads>(p.x, p.nb * kQK, p.eps, red);
    stage_x<FMT, kThreads>(lds, p.x, kb, nbl, (p.flags & F_NORM) != 0, inv, p.normw);
    __syncthreads();

    float acc[N];
#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = 0.0f;
    float best_v = -INFINITY;
    uint32_t best_i = 0xffffffffu, nonfinite = 0;

    auto compute = [&](uint32_t j, const Blk (&b)[N]) {
        const uint32_t bl = bs + BS * j;
        if (bl < nbl) blk_dot<FMT, N>(b, lds + bl * kXBlk + v * kSlot, v, acc);
    };
    // EPI_COLPART: quad sums of a tile's columns are held in registers and
    // stored once per tile (row-major partials, coalesced per slot).
    constexpr int kMaxNj = (EPI == EPI_COLPART) ? (kPanel + BS - 1) / BS : 1;
    float cp[RPL][kMaxNj];
    auto finish_column = [&](uint32_t ti, uint32_t j) {
        float tot[N];
#pragma unroll
        for (int n = 0; n < N; ++n) {
            tot[n] = group_sum<4>(acc[n]);
            acc[n] = 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kMaxNj; ++k)
            if (uint32_t(k) == j)
#pragma unroll
                for (int r = 0; r < RPL; ++r) cp[r][k] = tot[r];
        if (j != nj - 1 || v != 0) return;
        const uint32_t tile = gw + ti * stride;
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = tile_row(tile, r);
            if (row >= p.rows) continue;
            float* dst = p.y + uint64_t(row) * p.nsplit + kb + bs;
#pragma unroll
            for (int k = 0; k < kMaxNj; ++k)
                if (uint32_t(k) < nj && bs + BS * uint32_t(k) < nbl) dst[BS * k] = cp[r][k];
        }
    };
    auto finish = [&](uint32_t ti) {
        const uint32_t tile = gw + ti * stride;
        float tot[N];
#pragma unroll
        for (int n = 0; n < N; ++n) {
            tot[n] = group_sum<4 * BS>(acc[n]);
            acc[n] = 0.0f;
        }
        if (v != 0 || bs != 0) return;
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = tile_row(tile, r);
            if (row >= p.rows) continue;
            if constexpr (EPI == EPI_PLAIN) {
                float val = tot[r];
                if (p.flags & F_ACCUM) val = p.y[row] + val;
                if (p.flags & F_BIAS) val = val + p.bias[row];
                p.y[row] = val;
            } else if constexpr (EPI == EPI_SWIGLU) {
                const float g = tot[r], u = tot[RPL + r];
                p.y[row] = (g / (1.0f + expf(-g))) * u;
            } else if constexpr (EPI == EPI_PARTIAL) {
                float* dst = p.y + uint64_t(row) * p.nsplit + split;
                *dst = (p.flags & F_ACCUM) ? *dst + tot[r] : tot[r];
            } else {
                const float lv = tot[r];
                if (p.y) p.y[row] = lv;
                if (!isfinite(lv))
                    ++nonfinite;
                else if (arg_better(lv, row, best_v, best_i)) {
                    best_v = lv;
                    best_i = row;
                }
            }
        }
    };

    // Flattened (tile, block slot) walk with two register buffers: the item
    // in one buffer is consumed while the next item's loads are in flight.
    // Past the last item the "next" load repeats the current item (a cache
    // hit), keeping the load sequence free of branches.
    uint32_t ti = 0, tj = 0;
    for (uint32_t s = 0; s < S; s += 2) {
        uint32_t bi = ti, bj = tj + 1;
        if (bj == nj) {
            bj = 0;
            ++bi;
        }
        const bool has_b = s + 1 < S;
        load(has_b ? bi : ti, has_b ? bj : tj, bufB);
        compute(tj, bufA);
        if constexpr (EPI == EPI_COLPART)
            finish_column(ti, tj);
        else if (tj == nj - 1)
            finish(ti);
        if (!has_b) break;
        uint32_t ci = bi, cj = bj + 1;
        if (cj == nj) {
            cj = 0;
            ++ci;
        }
        const bool has_c = s + 2 < S;
        load(has_c ? ci : bi, has_c ? cj : bj, bufA);
        compute(bj, bufB);
        if constexpr (EPI == EPI_COLPART)
            finish_column(bi, bj);
        else if (bj == nj - 1)
            finish(bi);
        ti = ci;
        tj = cj;
    }

    if constexpr (EPI == EPI_ARGMAX) wg_argmax(best_v, best_i, nonfinite, p.best + blockIdx.x);
}

// Fixed-order second pass of the split-K GEMV: y[r] = ((p0 + p1) + ...) + res,
// with the partials of row r contiguous at part[r*splits].  Up to 128
// partials are fetched in one batch (all loads in flight), then added in order.
__global__ __launch_bounds__(64) void k_splitk_reduce(const float* __restrict__ part, uint32_t rows,
                                                       uint32_t splits, const float* __restrict__ residual,
                                                       float* __restrict__ y)
{
    const uint32_t r = blockIdx.x * 64u + threadIdx.x;
    if (r >= rows) return;
    const float* p = part + uint64_t(r) * splits;
    float s = 0.0f;
    for (uint32_t j0 = 0; j0 < splits; j0 += 128) {
        const uint32_t n = min(128u, splits - j0);
        float v[128];
#pragma unroll
        for (int i = 0; i < 128; ++i) v[i] = uint32_t(i) < n ? p[j0 + i] : 0.0f;
#pragma unroll
        for (int i = 0; i < 128; ++i)
            if (uint32_t(i) < n) s += v[i];
    }
    if (residual) s += residual[r];
    y[r] = s;
}

// Second stage of the LM-head argmax: one workgroup folds the per-workgroup
// bests in a fixed order.
__global__ __launch_bounds__(1024) void k_argmax_final(const ArgBest* __restrict__ best, uint32_t n,
                                                        uint32_t* __restrict__ out)
{
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu, nf = 0;
    for (uint32_t i0 = 0; i0 < n; i0 += 4096u) {
        ArgBest b[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t i = i0 + k * 1024u + threadIdx.x;
            b[k] = i < n ? best[i] : ArgBest{-INFINITY, 0xffffffffu, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (b[k].idx != 0xffffffffu && arg_better(b[k].val, b[k].idx, bv, bi)) {
                bv = b[k].val;
                bi = b[k].idx;
            }
            nf += b[k].nonfinite;
        }
    }
    __shared__ ArgBest res;
    wg_argmax(bv, bi, nf, &res);
    __syncthreads();
    if (threadIdx.x == 0) {
        out[0] = (res.idx == 0xffffffffu) ? 0u : res.idx;
        out[1] = res.nonfinite;
    }
}

__global__ __launch_bounds__(1024) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                  uint32_t n, float eps, float* __restrict__ y)
{
    __shared__ float red[16];
    const float inv = rms_inv<1024>(x, n, eps, red);
    for (uint32_t i = threadIdx.x; i < n; i += 1024u) y[i] = (x[i] * inv) * w[i];
}

// ------------------------------------------------------------ dequant dump
// One workgroup of 256 threads per super-block; thread k decodes element k
// with every product and the difference rounded separately, in the
// reference's order (no contraction).
__global__ __launch_bounds__(256) void k_dequant_q4(const uint8_t* __restrict__ w, float* __restrict__ out)
{
#pragma clang fp contract(off)
    const uint64_t blk = blockIdx.x;
    const uint32_t k = threadIdx.x;
    const uint8_t* b = w + blk * kQ4Bytes;
    const float d = f16_bits_to_f32(uint32_t(b[0]) | (uint32_t(b[1]) << 8));
    const float dm = f16_bits_to_f32(uint32_t(b[2]) | (uint32_t(b[3]) << 8));
    const uint32_t j = k >> 5;
    const uint8_t* s = b + 4;
    uint32_t sc, mn;
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | (uint32_t(s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | (uint32_t(s[j] >> 6) << 4);
    }
    const uint32_t l64 = k & 63u;
    const uint8_t qb = b[16 + (k >> 6) * 32 + (l64 & 31u)];
    const uint32_t q = l64 < 32u ? (qb & 15u) : (qb >> 4);
    const float t0 = d * float(sc);
    const float t1 = t0 * float(q);
    const float t2 = dm * float(mn);
    out[blk * kQK + k] = t1 - t2;
}

__global__ __launch_bounds__(256) void k_dequant_q6(const uint8_t* __restrict__ w, float* __restrict__ out)
{
#pragma clang fp contract(off)
    const uint64_t blk = blockIdx.x;
    const uint32_t k = threadIdx.x;
    const uint8_t* b = w + blk * kQ6Bytes;
    const uint32_t half = k >> 7, kk = k & 127u, l = kk & 31u, quarter = kk >> 5;
    const uint8_t* ql = b + half * 64u;
    const uint8_t* qh = b + 128u + half * 32u;
    const uint8_t* sc = b + 192u + half * 8u;
    const uint32_t lo = (quarter & 1u) ? ql[l + 32u] : ql[l];
    const uint32_t low = (quarter < 2u) ? (lo & 15u) : (lo >> 4);
    const uint32_t high = (qh[l] >> (2u * quarter)) & 3u;
    const int q = int(low | (high << 4)) - 32;
    const int scale = int(int8_t(sc[(l >> 4) + 2u * quarter]));
    const float d = f16_bits_to_f32(uint32_t(b[208]) | (uint32_t(b[209]) << 8));
    const float t0 = d * float(scale);
    out[blk * kQK + k] = t0 * float(q);
}

// --------------------------------------------------------------- launching
struct Cfg {
    int bs, rpl;
};

inline int tile_rows(const Cfg& c) { return (kWave / (4 * c.bs)) * c.rpl; }

static int cu_count()
{
    static int n = 0;
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    });
    return n;
}

// Resident workgroups per CU for one kernel instance (cached), >= 1.
template <int FMT, int EPI, int BS, int RPL>
int occupancy(size_t lds)
{
    static int occ[kPanel + 1] = {};
    const int slot = int(lds / (kXBlk * sizeof(float)));
    if (!occ[slot]) {
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<FMT, BS, RPL, EPI>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_gemv<FMT, BS, RPL, EPI>, kThreads, lds) != hipSuccess ||
            nb < 1)
            nb = 1;
        occ[slot] = nb;
    }
    return occ[slot];
}

static thread_local int g_wg_per_cu = 0;  // tuning override of resident workgroups per CU

template <int FMT, int EPI, int BS, int RPL>
hipError_t launch_one(GemvParams p, uint32_t splits, hipStream_t s, uint32_t* grid_x)
{
    const Cfg c{BS, RPL};
    p.ntiles = (p.rows + tile_rows(c) - 1) / tile_rows(c);
    const size_t lds = size_t(p.panel) * kXBlk * sizeof(float);
    const int per_cu = g_wg_per_cu > 0 ? g_wg_per_cu : occupancy<FMT, EPI, BS, RPL>(lds);
    const uint64_t resident = uint64_t(per_cu) * cu_count();
    const uint64_t want = (p.ntiles + kWaves - 1) / kWaves;  // one wave tile per wave
    uint64_t gx = (resident + splits - 1) / splits;
    if (gx > want) gx = want;  // want <= ceil(rows / 4): one wave tile holds at least one row
    if (gx > 65536) gx = 65536;
    if (gx < 1) gx = 1;
    if (grid_x) *grid_x = uint32_t(gx);
    hipLaunchKernelGGL((k_gemv<FMT, BS, RPL, EPI>), dim3(uint32_t(gx), splits), dim3(kThreads), lds, s, p);
    return hipGetLastError();
}

template <int FMT, int EPI>
hipError_t launch_cfg(const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s, uint32_t* gx)
{
#define ARC_CASE(B, R) \
    if (c.bs == B && c.rpl == R) return launch_one<FMT, EPI, B, R>(p, splits, s, gx);
    ARC_CASE(1, 1) ARC_CASE(1, 2) ARC_CASE(1, 4)
    ARC_CASE(2, 1) ARC_CASE(2, 2) ARC_CASE(2, 4)
    ARC_CASE(4, 1) ARC_CASE(4, 2)
    ARC_CASE(8, 1) ARC_CASE(8, 2)
    ARC_CASE(16, 1)
#undef ARC_CASE
    return hipErrorInvalidValue;
}

// Forced configuration for tuning sweeps (bs = 0: automatic).
static thread_local Cfg g_force{0, 0};

// Automatic lane layout.  Work is balanced over ~2048 resident waves: a
// layout is preferred when its wave tiles divide evenly over them and its
// quads are busy (few idle block slots), then when it reuses x over more rows.
inline Cfg choose_cfg(int epi, uint32_t rows, uint32_t blocks, uint32_t splits)
{
    if (g_force.bs) return g_force;
    static const Cfg cands[] = {{1, 1}, {1, 2}, {1, 4}, {2, 1}, {2, 2}, {2, 4}, {4, 1}, {4, 2}, {8, 1}, {8, 2}, {16, 1}};
    const double waves = 2048.0;
    Cfg best{1, 1};
    double best_score = -1.0;
    for (const Cfg& c : cands) {
        if (epi == EPI_SWIGLU && c.rpl > 2) continue;
        const uint32_t nj = (blocks + c.bs - 1) / c.bs;
        const double busy = double(blocks) / double(nj * c.bs);
        const double tiles = double((rows + tile_rows(c) - 1) / tile_rows(c)) * splits;
        const double per_wave = tiles / waves;
        const double balance = per_wave / std::ceil(per_wave);
        const double reuse = c.rpl >= 2 ? 1.0 : 0.97;
        const double score = busy * balance * reuse;
        if (score > best_score + 1e-9) {
            best_score = score;
            best = c;
        }
    }
    return best;
}

template <int EPI>
hipError_t launch_gemv(int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s, uint32_t* gx)
{
    if (qtype == kFmtQ4) return launch_cfg<kFmtQ4, EPI>(c, p, splits, s, gx);
    return launch_cfg<kFmtQ6, EPI>(c, p, splits, s, gx);
}

hipError_t launch_gemv_epi(int epi, int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s,
                           uint32_t* gx = nullptr)
{
    switch (epi) {
    case EPI_PLAIN: return launch_gemv<EPI_PLAIN>(qtype, c, p, splits, s, gx);
    case EPI_SWIGLU: return launch_gemv<EPI_SWIGLU>(qtype, c, p, splits, s, gx);
    case EPI_PARTIAL: return launch_gemv<EPI_PARTIAL>(qtype, c, p, splits, s, gx);
    case EPI_ARGMAX: return launch_gemv<EPI_ARGMAX>(qtype, c, p, splits, s, gx);
    default: return launch_gemv<EPI_COLPART>(qtype, c, p, splits, s, gx);
    }
}

static int block_bytes(int qtype) { return qtype == kFmtQ4 ? kQ4Bytes : kQ6Bytes; }

static int check_shape(int qtype, const void* w, uint32_t rows, uint32_t K)
{
    if (qtype != kFmtQ4 && qtype != kFmtQ6) return set_error(ARC_ERR_UNSUPPORTED, "unsupported qtype %d", qtype);
    if (!w) return set_error(ARC_ERR_INVALID_ARGUMENT, "null weight pointer");
    if (rows == 0 || K == 0 || (K % kQK) != 0)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad shape rows=%u K=%u (K must be a nonzero multiple of 256)",
                         rows, K);
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if (qtype == kFmtQ4 && (a & 15u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "Q4_K tensor not 16-byte aligned");
    if (qtype == kFmtQ6 && (a & 1u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "Q6_K tensor not 2-byte aligned");
    return ARC_OK;
}

static int check_vec(const float* p, const char* what)
{
    if (!p) return set_error(ARC_ERR_INVALID_ARGUMENT, "null %s", what);
    if (reinterpret_cast<uintptr_t>(p) & 15u) return set_error(ARC_ERR_INVALID_ARGUMENT, "%s not 16-byte aligned", what);
    return ARC_OK;
}

static GemvParams make_params(int qtype, const void* w0, const void* w1, uint32_t rows, uint32_t K, const float* x)
{
    GemvParams p{};
    p.w0 = static_cast<const uint8_t*>(w0);
    p.w1 = static_cast<const uint8_t*>(w1);
    p.row_bytes = uint64_t(K / kQK) * block_bytes(qtype);
    p.rows = rows;
    p.nb = K / kQK;
    p.split_bps = p.nb;
    p.kb_off = 0;
    p.panel = min(p.nb, uint32_t(kPanel));
    p.x = x;
    return p;
}

// Runs a GEMV whose split width may exceed one LDS panel as consecutive
// launches over panels; later panels accumulate into the output in order.
static int run_paneled(int epi, int qtype, GemvParams p, uint32_t splits, hipStream_t s, const char* what,
                       uint32_t* gx = nullptr)
{
    const Cfg c = choose_cfg(epi, p.rows, min(p.split_bps, uint32_t(kPanel)), splits);
    const uint32_t bias_flag = p.flags & F_BIAS;
    for (uint32_t off = 0; off < p.split_bps; off += kPanel) {
        GemvParams q = p;
        q.kb_off = off;
        q.panel = min(uint32_t(kPanel), p.split_bps - off);
        q.flags = (p.flags & ~(F_ACCUM | F_BIAS)) | (off ? F_ACCUM : 0u) |
                  (off + kPanel >= p.split_bps ? bias_flag : 0u);
        const int rc = check_hip(launch_gemv_epi(epi, qtype, c, q, splits, s, gx), what);
        if (rc) return rc;
    }
    return ARC_OK;
}

}  // namespace arc

using namespace arc;

extern "C" {

int arc_tune_force(int bs, int rpl)
{
    if (bs == 0) {
        g_force = Cfg{0, 0};
        g_wg_per_cu = 0;
        return ARC_OK;
    }
    if (bs < 0) {  // -n: size grids for n resident workgroups per CU
        if (bs < -32) return set_error(ARC_ERR_INVALID_ARGUMENT, "at most 32 workgroups per CU");
        g_wg_per_cu = -bs;
        return ARC_OK;
    }
    static const int ok[][2] = {{1, 1}, {1, 2}, {1, 4}, {2, 1}, {2, 2}, {2, 4}, {4, 1}, {4, 2}, {8, 1}, {8, 2}, {16, 1}};
    for (const auto& c : ok)
        if (c[0] == bs && c[1] == rpl) {
            g_force = Cfg{bs, rpl};
            return ARC_OK;
        }
    return set_error(ARC_ERR_INVALID_ARGUMENT, "no kernel instance for bs=%d rpl=%d", bs, rpl);
}

int arc_dequant(int qtype, const void* w, uint32_t rows, uint32_t K, float* out, arc_stream_t stream)
{
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if (!out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    const uint64_t blocks = uint64_t(rows) * (K / kQK);
    if (blocks > 0x7fffffffull) return set_error(ARC_ERR_UNSUPPORTED, "tensor too large for one dequant launch");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (qtype == kFmtQ4)
        hipLaunchKernelGGL(k_dequant_q4, dim3(uint32_t(blocks)), dim3(256), 0, s, static_cast<const uint8_t*>(w), out);
    else
        hipLaunchKernelGGL(k_dequant_q6, dim3(uint32_t(blocks)), dim3(256), 0, s, static_cast<const uint8_t*>(w), out);
    return check_hip(hipGetLastError(), "dequant launch");
}

int arc_gemv(int qtype, const void* w, uint32_t rows, uint32_t K, const float* x, const float* bias, float* y,
             arc_stream_t stream)
{
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if ((rc = check_vec(x, "x"))) return rc;
    if (!y) return set_error(ARC_ERR_INVALID_ARGUMENT, "null y");
    GemvParams p = make_params(qtype, w, nullptr, rows, K, x);
    p.bias = bias;
    p.y = y;
    p.flags = bias ? F_BIAS : 0u;
    return run_paneled(EPI_PLAIN, qtype, p, 1, static_cast<hipStream_t>(stream), "gemv launch");
}

int arc_gateup_swiglu(int qtype, const void* w_gate, const void* w_up, uint32_t rows, uint32_t K, const float* x,
                      float* s, arc_stream_t stream)
{
    int rc = check_shape(qtype, w_gate, rows, K);
    if (rc) return rc;
    if ((rc = check_shape(qtype, w_up, rows, K))) return rc;
    if ((rc = check_vec(x, "x"))) return rc;
    if (!s) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    if (K / kQK > uint32_t(kPanel))
        return set_error(ARC_ERR_UNSUPPORTED, "fused gate/up supports K <= %d", kPanel * kQK);
    GemvParams p = make_params(qtype, w_gate, w_up, rows, K, x);
    p.y = s;
    const Cfg c = choose_cfg(EPI_SWIGLU, rows, p.nb, 1);
    return check_hip(launch_gemv_epi(EPI_SWIGLU, qtype, c, p, 1, static_cast<hipStream_t>(stream)),
                     "gate/up launch");
}

int arc_gemv_splitk(int qtype, const void* w, uint32_t rows, uint32_t K, uint32_t splits, const float* x,
                    float* partials, const float* residual, float* y, arc_stream_t stream)
{
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if ((rc = check_vec(x, "x"))) return rc;
    if (!partials || !y) return set_error(ARC_ERR_INVALID_ARGUMENT, "null partials or y");
    const uint32_t nb = K / kQK;
    if (splits == 0 || splits > nb) return set_error(ARC_ERR_INVALID_ARGUMENT, "splits=%u outside [1, %u]", splits, nb);
    if (splits > 65535) return set_error(ARC_ERR_UNSUPPORTED, "too many splits");
    GemvParams p = make_params(qtype, w, nullptr, rows, K, x);
    p.split_bps = (nb + splits - 1) / splits;
    p.panel = min(p.split_bps, uint32_t(kPanel));
    const uint32_t used = (nb + p.split_bps - 1) / p.split_bps;  // splits owning at least one column
    p.y = partials;
    p.nsplit = used;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.split_bps == 1 && nb <= uint32_t(kPanel)) {
        // one column per split: all columns in one launch, partial per quad
        p.split_bps = nb;
        p.panel = nb;
        Cfg c = choose_cfg(EPI_PLAIN, rows, nb, 1);
        if (c.bs < 8) c = Cfg{8, 1};  // per-slot partials are held in registers: <= 10 slots
        rc = check_hip(launch_gemv_epi(EPI_COLPART, qtype, c, p, 1, s), "split-K pass 1");
    } else {
        rc = run_paneled(EPI_PARTIAL, qtype, p, used, s, "split-K pass 1");
    }
    if (rc) return rc;
    hipLaunchKernelGGL(k_splitk_reduce, dim3((rows + 63) / 64), dim3(64), 0, s, partials, rows, used, residual, y);
    return check_hip(hipGetLastError(), "split-K pass 2");
}

int arc_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, arc_stream_t stream)
{
    if (!x || !w || !y || n == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad rmsnorm arguments");
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, w, n, eps, y);
    return check_hip(hipGetLastError(), "rmsnorm launch");
}

// launch_one never makes the argmax grid larger than ceil(rows/4) (a wave
// tile holds at least one row, a workgroup four wave tiles) nor 65536.
static uint32_t lm_max_wgs(uint32_t rows) { return min((rows + 3u) / 4u, uint32_t(64 * 1024)); }

size_t arc_lmhead_workspace_bytes(int qtype, uint32_t rows, uint32_t K)
{
    if ((qtype != kFmtQ4 && qtype != kFmtQ6) || rows == 0 || K == 0 || K % kQK) return 0;
    return size_t(lm_max_wgs(rows)) * sizeof(ArgBest);
}

int arc_lmhead_argmax(int qtype, const void* w, uint32_t rows, uint32_t K, const float* h, const float* normw,
                      float eps, float* logits, void* workspace, uint32_t* out, arc_stream_t stream)
{
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if ((rc = check_vec(h, "h"))) return rc;
    if (normw && (rc = check_vec(normw, "normw"))) return rc;
    if (!workspace || !out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null workspace or out");
    if (K / kQK > uint32_t(kPanel)) return set_error(ARC_ERR_UNSUPPORTED, "LM head supports K <= %d", kPanel * kQK);
    GemvParams p = make_params(qtype, w, nullptr, rows, K, h);
    p.flags = normw ? F_NORM : 0u;
    p.normw = normw;
    p.eps = eps;
    p.y = logits;
    p.best = static_cast<ArgBest*>(workspace);
    const Cfg c = choose_cfg(EPI_ARGMAX, rows, p.nb, 1);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t gx = 0;
    rc = check_hip(launch_gemv_epi(EPI_ARGMAX, qtype, c, p, 1, s, &gx), "lm-head launch");
    if (rc) return rc;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, s, p.best, gx, out);
    return check_hip(hipGetLastError(), "argmax launch");
}

}  // extern "C"
