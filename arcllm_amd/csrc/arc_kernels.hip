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
//  * Each lane carries RPL rows (and NMAT matrices for the fused gate/up) so
//    one LDS read of x feeds RPL*NMAT rows.
//  * x is staged once per workgroup into LDS, permuted so each lane reads 64
//    contiguous floats per block, with the four 16-element group sums that
//    fold the Q4_K min and the Q6_K -32 offset out of the inner loop:
//      Q4_K: sum_k (d sc q - dmin mn) x = d sum_g sc_g (q.x)_g - dmin sum_g mn_g (sum x)_g
//      Q6_K: sum_k d sc (u - 32) x      = d sum_g sc_g ((u.x)_g - 32 (sum x)_g)
//  * Loads of the next super-block are issued before the current one is
//    consumed (register double buffering).
#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

namespace arc {

// Set by the runtime translation unit; declared here for the launchers.
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

constexpr int kPanel = 32;         // super-block columns of x staged per pass
constexpr int kWaves = 4;          // waves per GEMV workgroup
constexpr int kThreads = kWaves * kWave;

enum Epi { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_PARTIAL = 2, EPI_ARGMAX = 3 };

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
    uint32_t nb;    // super-blocks per row
    uint32_t bps;   // super-blocks per split (grid.y = splits)
    uint32_t norm;  // 1: x is RMS-normalised with normw/eps before use
    const float* x;
    const float* normw;
    float eps;
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

// Every chunk offset below is a multiple of 4 within the block, so its
// misalignment equals the block's (0 or 2).  The dwords read span at most
// [o-2, o+18) of the block; for o <= 192 that stays inside the block's own
// dword span, so no read leaves the tensor's pages.
__device__ __forceinline__ void q6_load(const uint8_t* blk, int v, Q6Blk& o)
{
    uint32_t t;
    ld16_realign(blk + v * 16, o.ql[0], t);
    ld16_realign(blk + 64 + v * 16, o.ql[1], t);
    ld16_realign(blk + 128 + (v & 1) * 16, o.qh[0], t);
    ld16_realign(blk + 160 + (v & 1) * 16, o.qh[1], t);
    ld16_realign(blk + 192, o.sc, t);
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

__device__ __forceinline__ float fma4(uint32_t codes, const float4& x, float acc)
{
    acc = __builtin_fmaf(byte_f(codes, 0), x.x, acc);
    acc = __builtin_fmaf(byte_f(codes, 1), x.y, acc);
    acc = __builtin_fmaf(byte_f(codes, 2), x.z, acc);
    acc = __builtin_fmaf(byte_f(codes, 3), x.w, acc);
    return acc;
}

__device__ __forceinline__ uint32_t comp(const uint4& q, int i)
{
    return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Dot of N Q4_K blocks (same column, different rows/matrices) with the
// lane's 64 x values; adds d*sum(sc*qx) - dmin*sum(mn*sx) into acc[n].
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
            a[n][0] = fma4(qa & 0x0f0f0f0fu, x0, a[n][0]);
            a[n][1] = fma4((qa >> 4) & 0x0f0f0f0fu, x1, a[n][1]);
            a[n][2] = fma4(qb & 0x0f0f0f0fu, x2, a[n][2]);
            a[n][3] = fma4((qb >> 4) & 0x0f0f0f0fu, x3, a[n][3]);
        }
    }
    const float4 S = lds4(xs + 64);
    const int sh = 16 * (v >> 1);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const uint32_t yy = b[n].hdr.y >> sh, zz = b[n].hdr.z >> sh, ww = b[n].hdr.w >> sh;
        const float sc0 = float(yy & 63u), sc1 = float((yy >> 8) & 63u);
        const float mn0 = float(zz & 63u), mn1 = float((zz >> 8) & 63u);
        const float sc2 = float((ww & 15u) | (((yy >> 6) & 3u) << 4));
        const float sc3 = float(((ww >> 8) & 15u) | (((yy >> 14) & 3u) << 4));
        const float mn2 = float(((ww >> 4) & 15u) | (((zz >> 6) & 3u) << 4));
        const float mn3 = float(((ww >> 12) & 15u) | (((zz >> 14) & 3u) << 4));
        const float d = f16_bits_to_f32(b[n].hdr.x);
        const float dm = f16_bits_to_f32(b[n].hdr.x >> 16);
        float qs = sc0 * a[n][0];
        qs = __builtin_fmaf(sc1, a[n][1], qs);
        qs = __builtin_fmaf(sc2, a[n][2], qs);
        qs = __builtin_fmaf(sc3, a[n][3], qs);
        float ms = mn0 * S.x;
        ms = __builtin_fmaf(mn1, S.y, ms);
        ms = __builtin_fmaf(mn2, S.z, ms);
        ms = __builtin_fmaf(mn3, S.w, ms);
        acc[n] = __builtin_fmaf(d, qs, acc[n]);
        acc[n] = __builtin_fmaf(-dm, ms, acc[n]);
    }
}

__device__ __forceinline__ int sbyte(const uint32_t (&w)[4], int idx)
{
    const uint32_t word = idx < 4 ? w[0] : idx < 8 ? w[1] : idx < 12 ? w[2] : w[3];
    return int(int8_t(uint8_t(word >> (8 * (idx & 3)))));
}

template <int N>
__device__ __forceinline__ void q6_dot(const Q6Blk (&b)[N], const float* xs, int v, float (&acc)[N])
{
    const int qa = v >> 1;
    const uint32_t shA = 2u * qa, shB = 2u * qa + 4u;
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
                const uint32_t ua = (ql & 0x0f0f0f0fu) | (((qh >> shA) & 0x03030303u) << 4);
                const uint32_t ub = ((ql >> 4) & 0x0f0f0f0fu) | (((qh >> shB) & 0x03030303u) << 4);
                a[n][2 * h] = fma4(ua, xa, a[n][2 * h]);
                a[n][2 * h + 1] = fma4(ub, xb, a[n][2 * h + 1]);
            }
        }
    }
    const float4 S = lds4(xs + 64);
    const int i0 = (v & 1) + 2 * qa;  // scale index of group t=0; t adds {0,4,8,12}
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float d = f16_bits_to_f32(b[n].d);
        float t = float(sbyte(b[n].sc, i0)) * __builtin_fmaf(-32.0f, S.x, a[n][0]);
        t = __builtin_fmaf(float(sbyte(b[n].sc, i0 + 4)), __builtin_fmaf(-32.0f, S.y, a[n][1]), t);
        t = __builtin_fmaf(float(sbyte(b[n].sc, i0 + 8)), __builtin_fmaf(-32.0f, S.z, a[n][2]), t);
        t = __builtin_fmaf(float(sbyte(b[n].sc, i0 + 12)), __builtin_fmaf(-32.0f, S.w, a[n][3]), t);
        acc[n] = __builtin_fmaf(d, t, acc[n]);
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
// arc_device.hpp).  With norm, x is replaced by (x*inv)*normw.
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
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            reinterpret_cast<float4*>(dst)[i] = q[i];
            s += q[i].x;
            s += q[i].y;
            s += q[i].z;
            s += q[i].w;
        }
        lds[bl * kXBlk + v * kSlot + 64 + t] = s;
    }
}

__device__ __forceinline__ bool arg_better(float va, uint32_t ia, float vb, uint32_t ib)
{
    return va > vb || (va == vb && ia < ib);
}

// --------------------------------------------------------------- GEMV core
template <int FMT, int BS, int RPL, int EPI>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvParams p)
{
    extern __shared__ float lds[];
    __shared__ float red[kWaves * 4];
    constexpr int NMAT = (EPI == EPI_SWIGLU) ? 2 : 1;
    constexpr int N = NMAT * RPL;
    constexpr int RG = kWave / (4 * BS);
    using Blk = typename BlkOf<FMT>::T;
    constexpr int kBB = BlkOf<FMT>::bytes;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v = lane & 3, bs = (lane >> 2) % BS, rg = lane / (4 * BS);
    const uint32_t kb0 = blockIdx.y * p.bps;
    const uint32_t kb1 = min(kb0 + p.bps, p.nb);

    uint32_t row[RPL];
    bool valid[RPL];
    const uint32_t rbase = (blockIdx.x * kWaves + wave) * (RG * RPL) + rg * RPL;
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        row[j] = rbase + j;
        valid[j] = row[j] < p.rows;
        if (!valid[j]) row[j] = p.rows - 1;  // clamp loads; result discarded
    }
    const uint8_t* wp[N];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            wp[m * RPL + j] = (m == 0 ? p.w0 : p.w1) + uint64_t(row[j]) * p.row_bytes;

    float inv = 1.0f;
    if (p.norm) inv = rms_inv<kThreads>(p.x, p.nb * kQK, p.eps, red);

    float acc[N];
#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = 0.0f;

    for (uint32_t pb = kb0; pb < kb1; pb += kPanel) {
        const uint32_t pn = min(uint32_t(kPanel), kb1 - pb);
        if (pb != kb0) __syncthreads();
        stage_x<FMT, kThreads>(lds, p.x, pb, pn, p.norm != 0, inv, p.normw);
        __syncthreads();

        uint32_t bl = bs;
        Blk cur[N];
        if (bl < pn) {
#pragma unroll
            for (int n = 0; n < N; ++n) blk_load<FMT>(wp[n] + uint64_t(pb + bl) * kBB, v, cur[n]);
        }
        for (; bl < pn; bl += BS) {
            Blk nxt[N];
            const bool more = bl + BS < pn;
            if (more) {
#pragma unroll
                for (int n = 0; n < N; ++n) blk_load<FMT>(wp[n] + uint64_t(pb + bl + BS) * kBB, v, nxt[n]);
            }
            blk_dot<FMT, N>(cur, lds + bl * kXBlk + v * kSlot, v, acc);
            if (more) {
#pragma unroll
                for (int n = 0; n < N; ++n) cur[n] = nxt[n];
            }
        }
    }

#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = group_sum<4 * BS>(acc[n]);
    const bool writer = (v == 0) && (bs == 0);

    if constexpr (EPI == EPI_PLAIN) {
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            if (writer && valid[j]) p.y[row[j]] = acc[j] + (p.bias ? p.bias[row[j]] : 0.0f);
    } else if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            if (writer && valid[j]) {
                const float g = acc[j], u = acc[RPL + j];
                p.y[row[j]] = (g / (1.0f + expf(-g))) * u;
            }
        }
    } else if constexpr (EPI == EPI_PARTIAL) {
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            if (writer && valid[j]) p.y[uint64_t(blockIdx.y) * p.rows + row[j]] = acc[j];
    } else {  // EPI_ARGMAX
        float bv = -INFINITY;
        uint32_t bi = 0xffffffffu, nf = 0;
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            if (writer && valid[j]) {
                const float lv = acc[j];
                if (p.y) p.y[row[j]] = lv;
                if (!isfinite(lv)) {
                    ++nf;
                } else if (arg_better(lv, row[j], bv, bi)) {
                    bv = lv;
                    bi = row[j];
                }
            }
        }
        // wave argmax, then across the workgroup's waves in order
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const uint32_t oi = __shfl_xor(bi, off);
            const uint32_t on = __shfl_xor(nf, off);
            if (arg_better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
            nf += on;
        }
        __shared__ float sv[kWaves];
        __shared__ uint32_t si[kWaves], sn[kWaves];
        if (lane == 0) {
            sv[wave] = bv;
            si[wave] = bi;
            sn[wave] = nf;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float b = sv[0];
            uint32_t i = si[0], c = sn[0];
            for (int w = 1; w < kWaves; ++w) {
                if (arg_better(sv[w], si[w], b, i)) {
                    b = sv[w];
                    i = si[w];
                }
                c += sn[w];
            }
            p.best[blockIdx.x] = ArgBest{b, i, c, 0u};
        }
    }
}

// Fixed-order second pass of the split-K GEMV.
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, uint32_t rows,
                                                        uint32_t splits, const float* __restrict__ residual,
                                                        float* __restrict__ y)
{
    const uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (r >= rows) return;
    float s = 0.0f;
    for (uint32_t j = 0; j < splits; ++j) s += part[uint64_t(j) * rows + r];
    if (residual) s += residual[r];
    y[r] = s;
}

// Second stage of the LM-head argmax: one workgroup folds the per-workgroup
// bests in a fixed order.
__global__ __launch_bounds__(256) void k_argmax_final(const ArgBest* __restrict__ best, uint32_t n,
                                                       uint32_t* __restrict__ out)
{
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu, nf = 0;
    for (uint32_t i = threadIdx.x; i < n; i += 256u) {
        const ArgBest b = best[i];
        if (b.idx != 0xffffffffu && arg_better(b.val, b.idx, bv, bi)) {
            bv = b.val;
            bi = b.idx;
        }
        nf += b.nonfinite;
    }
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
    __shared__ float sv[4];
    __shared__ uint32_t si[4], sn[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
        sn[wave] = nf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sv[0];
        uint32_t i = si[0], c = sn[0];
        for (int w = 1; w < 4; ++w) {
            if (si[w] != 0xffffffffu && arg_better(sv[w], si[w], b, i)) {
                b = sv[w];
                i = si[w];
            }
            c += sn[w];
        }
        out[0] = (i == 0xffffffffu) ? 0u : i;
        out[1] = c;
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

inline int rows_per_wg(const Cfg& c) { return kWaves * (kWave / (4 * c.bs)) * c.rpl; }

template <int FMT, int EPI, int BS, int RPL>
hipError_t launch_one(const GemvParams& p, uint32_t splits, hipStream_t s)
{
    const Cfg c{BS, RPL};
    const uint32_t gx = (p.rows + rows_per_wg(c) - 1) / rows_per_wg(c);
    const uint32_t pn = min(p.bps, uint32_t(kPanel));
    const size_t lds = size_t(pn) * kXBlk * sizeof(float);
    hipLaunchKernelGGL((k_gemv<FMT, BS, RPL, EPI>), dim3(gx, splits), dim3(kThreads), lds, s, p);
    return hipGetLastError();
}

template <int FMT, int EPI>
hipError_t launch_cfg(const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s)
{
#define ARC_CASE(B, R) \
    if (c.bs == B && c.rpl == R) return launch_one<FMT, EPI, B, R>(p, splits, s);
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

// Automatic choice: enough workgroups to fill 256 CUs several times over,
// preferring more rows per lane (x reuse) and fewer lanes per row.
inline Cfg choose_cfg(int epi, uint32_t rows, uint32_t blocks_per_split, uint32_t splits)
{
    if (g_force.bs) return g_force;
    static const Cfg order[] = {{2, 2}, {2, 1}, {4, 1}, {8, 1}, {16, 1}};
    const int nmat = epi == EPI_SWIGLU ? 2 : 1;
    for (const Cfg& c : order) {
        if (uint32_t(c.bs) > blocks_per_split) continue;
        if (nmat == 2 && c.rpl > 1) continue;
        const uint64_t wgs = uint64_t((rows + rows_per_wg(c) - 1) / rows_per_wg(c)) * splits;
        if (wgs >= 1024) return c;
    }
    if (blocks_per_split >= 16) return Cfg{16, 1};
    if (blocks_per_split >= 8) return Cfg{8, 1};
    if (blocks_per_split >= 4) return Cfg{4, 1};
    if (blocks_per_split >= 2) return Cfg{2, 1};
    return Cfg{1, 1};
}

template <int EPI>
hipError_t launch_gemv(int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s)
{
    if (qtype == kFmtQ4) return launch_cfg<kFmtQ4, EPI>(c, p, splits, s);
    return launch_cfg<kFmtQ6, EPI>(c, p, splits, s);
}

hipError_t launch_gemv_epi(int epi, int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s)
{
    switch (epi) {
    case EPI_PLAIN: return launch_gemv<EPI_PLAIN>(qtype, c, p, splits, s);
    case EPI_SWIGLU: return launch_gemv<EPI_SWIGLU>(qtype, c, p, splits, s);
    case EPI_PARTIAL: return launch_gemv<EPI_PARTIAL>(qtype, c, p, splits, s);
    default: return launch_gemv<EPI_ARGMAX>(qtype, c, p, splits, s);
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
    p.bps = p.nb;
    p.x = x;
    return p;
}

}  // namespace arc

using namespace arc;

extern "C" {

int arc_tune_force(int bs, int rpl)
{
    if (bs == 0) {
        g_force = Cfg{0, 0};
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
    const Cfg c = choose_cfg(EPI_PLAIN, rows, p.nb, 1);
    return check_hip(launch_gemv_epi(EPI_PLAIN, qtype, c, p, 1, static_cast<hipStream_t>(stream)), "gemv launch");
}

int arc_gateup_swiglu(int qtype, const void* w_gate, const void* w_up, uint32_t rows, uint32_t K, const float* x,
                      float* s, arc_stream_t stream)
{
    int rc = check_shape(qtype, w_gate, rows, K);
    if (rc) return rc;
    if ((rc = check_shape(qtype, w_up, rows, K))) return rc;
    if ((rc = check_vec(x, "x"))) return rc;
    if (!s) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    GemvParams p = make_params(qtype, w_gate, w_up, rows, K, x);
    p.y = s;
    Cfg c = choose_cfg(EPI_SWIGLU, rows, p.nb, 1);
    if (c.rpl > 1) c.rpl = 1;
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
    p.bps = (nb + splits - 1) / splits;
    const uint32_t used = (nb + p.bps - 1) / p.bps;  // splits that own at least one block
    p.y = partials;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const Cfg c = choose_cfg(EPI_PARTIAL, rows, p.bps, used);
    rc = check_hip(launch_gemv_epi(EPI_PARTIAL, qtype, c, p, used, s), "split-K pass 1");
    if (rc) return rc;
    if (used < splits) {  // splits past the last block contribute exact zeros
        rc = check_hip(hipMemsetAsync(partials + uint64_t(used) * rows, 0, sizeof(float) * uint64_t(splits - used) * rows, s),
                       "split-K zero fill");
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_splitk_reduce, dim3((rows + 255) / 256), dim3(256), 0, s, partials, rows, splits, residual, y);
    return check_hip(hipGetLastError(), "split-K pass 2");
}

int arc_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, arc_stream_t stream)
{
    if (!x || !w || !y || n == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad rmsnorm arguments");
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, w, n, eps, y);
    return check_hip(hipGetLastError(), "rmsnorm launch");
}

size_t arc_lmhead_workspace_bytes(int qtype, uint32_t rows, uint32_t K)
{
    if ((qtype != kFmtQ4 && qtype != kFmtQ6) || rows == 0 || K == 0 || K % kQK) return 0;
    const Cfg c = choose_cfg(EPI_ARGMAX, rows, K / kQK, 1);
    size_t wgs = (rows + rows_per_wg(c) - 1) / rows_per_wg(c);
    // room for the smallest rows-per-workgroup configuration a tuning override may pick
    const size_t worst = (rows + rows_per_wg(Cfg{16, 1}) - 1) / rows_per_wg(Cfg{16, 1});
    if (worst > wgs) wgs = worst;
    return wgs * sizeof(ArgBest);
}

int arc_lmhead_argmax(int qtype, const void* w, uint32_t rows, uint32_t K, const float* h, const float* normw,
                      float eps, float* logits, void* workspace, uint32_t* out, arc_stream_t stream)
{
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if ((rc = check_vec(h, "h"))) return rc;
    if (normw && (rc = check_vec(normw, "normw"))) return rc;
    if (!workspace || !out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null workspace or out");
    GemvParams p = make_params(qtype, w, nullptr, rows, K, h);
    p.norm = normw ? 1u : 0u;
    p.normw = normw;
    p.eps = eps;
    p.y = logits;
    p.best = static_cast<ArgBest*>(workspace);
    const Cfg c = choose_cfg(EPI_ARGMAX, rows, p.nb, 1);
    const uint32_t wgs = (rows + rows_per_wg(c) - 1) / rows_per_wg(c);
    hipStream_t s = static_cast<hipStream_t>(stream);
    rc = check_hip(launch_gemv_epi(EPI_ARGMAX, qtype, c, p, 1, s), "lm-head launch");
    if (rc) return rc;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, p.best, wgs, out);
    return check_hip(hipGetLastError(), "argmax launch");
}

}  // extern "C"
