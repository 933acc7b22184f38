// arc_gemv_rs.hpp -- the row-stream Q4_K GEMV for gfx950 (included by
// arc_gemv.hpp after the quad-layout GEMV), for rows of at most 14
// super-blocks (K <= 3584).
//
// Lane layout: lane l < 56 owns sub-block pair g = l % 4 of super-block
// k = l / 4 -- the 64 weights 256k + 64g + [0, 64), held by the two 16-byte
// nibble chunks 2g and 2g + 1 of the block (qs bytes 32g .. 32g + 31).
// Lanes 56 .. 63 load block headers (d, dmin, the 12 scale bytes): lane
// 56 + h those of blocks h and h + 8.  A row is two load instructions, every
// lane 16 bytes of one row (lanes past the row's blocks repeat its last
// block).  Measured on MI355X with loads alone over two 18944 x 3584 Q4_K
// matrices: 13.2 us with this pattern, 13.1 us for plain consecutive 16-byte
// pieces, 17.0 us for the quad layout's loads.
//
// Every lane works on the same 64 columns of every row, so its 64 x values
// live in registers for the whole launch: the workgroup stages x once into
// LDS (with the fused RMSNorm), then each lane copies out its 64 values.
// A nibble chunk byte i holds element 16h + i of sub-block 2g (low nibble)
// and of 2g + 1 (high nibble), h = 0 / 1 for chunk 2g / 2g + 1.  The codes are read as fp16 subnormals
// (low nibbles w & 0x000f000f = q 2^-24, high nibbles w & 0x00f000f0 =
// q 2^-20) against x scaled by 2^24 / 2^20, and
//   sum (d sc q - dmin mn) x = d (sc_lo (q.x)_lo + sc_hi (q.x)_hi) - dmin (mn_lo S_lo + mn_hi S_hi)
// with S the plain sums of x over each sub-block.  The block header comes
// from its header lane by ds_bpermute.  A row's value is the sum over the
// wave (fixed tree, deterministic).
//
// Measured on MI355X against the quad layout: 18944 x 3584 plain 10.9 vs
// 11.7 us (ring of 3; 2 and 4 slots 11.4 us), 3584 x 3584 plain 5.6 vs
// 5.0 us, fused gate/up 20.0 vs 17.4 us.  Without the dot products (loads,
// staging, ring, stores) the gate/up takes 15.3 us: the time over that is
// VALU issue (7.0M VALU instructions per gate/up launch, 6.3M for the quad
// layout), so the launcher gives this kernel only the large plain GEMVs.
#pragma once

namespace arc {

constexpr int kRsMaxBlocks = 14;  // super-blocks per row (56 owner lanes)
constexpr int kRsOwners = 4 * kRsMaxBlocks;
// x in LDS: 4 pad floats after every 64, so the 64-float runs that
// consecutive lanes read start 68 floats (4 banks) apart
__device__ __host__ constexpr uint32_t rs_lds_index(uint32_t e) { return e + 4u * (e >> 6); }
constexpr int kRsLdsFloats = kRsMaxBlocks * kQK / 64 * 68;
#ifndef ARC_RS_RING
#define ARC_RS_RING 3
#endif
constexpr int kRsRing = ARC_RS_RING;  // ring slots (tiles in flight + 1)
static_assert(kRsRing >= 2, "a ring holds at least two items");

__device__ __forceinline__ uint32_t bperm(uint32_t src4, uint32_t v)
{
    return uint32_t(__builtin_amdgcn_ds_bpermute(int(src4), int(v)));
}

// x of one lane: elements e + [0, 16) and e + [16, 32) (sub-block 2g) times
// 2^24, e + [32, 48) and e + [48, 64) (sub-block 2g + 1) times 2^20.
struct RsX {
    float4 a[4], b[4], c[4], d[4];
    float s_lo, s_hi;
};

__device__ __forceinline__ float sum4(const float4 (&q)[4])
{
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = (((s + q[i].x) + q[i].y) + q[i].z) + q[i].w;
    return s;
}

__device__ __forceinline__ void scale4(float4 (&q)[4], float f)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[i].x *= f;
        q[i].y *= f;
        q[i].z *= f;
        q[i].w *= f;
    }
}

// The 8 products of one dword of a nibble chunk with x: dword j holds bytes
// 4j .. 4j + 3 = elements 4j .. 4j + 3 of the chunk's low (xl) and high (xh)
// groups.
__device__ __forceinline__ void rs_dword(uint32_t w, const float4& xl, const float4& xh, float& lo, float& hi)
{
    const uint32_t w8 = w >> 8;
    const uint32_t el = opaque(w & 0x000f000fu), ol = opaque(w8 & 0x000f000fu);
    const uint32_t eh = opaque(w & 0x00f000f0u), oh = opaque(w8 & 0x00f000f0u);
    lo = fmix(el, false, xl.x, lo);
    hi = fmix(eh, false, xh.x, hi);
    lo = fmix(ol, false, xl.y, lo);
    hi = fmix(oh, false, xh.y, hi);
    lo = fmix(el, true, xl.z, lo);
    hi = fmix(eh, true, xh.z, hi);
    lo = fmix(ol, true, xl.w, lo);
    hi = fmix(oh, true, xh.w, hi);
}

// One workgroup's share of a row-stream GEMV: rows of w0 (and, NMAT = 2, the
// same rows of w1), RPL rows per wave item.  EPI_PLAIN: y = dot (+ bias)
// (+ res); EPI_SWIGLU: y = silu(dot0) * dot1.  NORM applies the RMSNorm of x
// (p.normw, p.eps) while x is staged.
template <int NMAT, int RPL, int EPI, bool NORM, int W>
__device__ __forceinline__ void gemv_rs_body(const GemvParams& p, uint32_t bx, uint32_t gx)
{
    static_assert(EPI == EPI_PLAIN || EPI == EPI_SWIGLU, "row-stream epilogues: plain, SwiGLU");
    static_assert(NMAT == (EPI == EPI_SWIGLU ? 2 : 1), "SwiGLU reads gate and up");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t nb = p.nb;  // 1 .. kRsMaxBlocks (checked by the launcher)
    const uint32_t ntiles = (p.rows + RPL - 1) / RPL;
    const uint32_t gw = bx * W + wave, stride = gx * W;
    const uint32_t my = gw < ntiles ? (ntiles - gw + stride - 1) / stride : 0u;
    __shared__ __align__(16) float xs[kRsLdsFloats];
    __shared__ float red[W];

    // this lane's block and pair (owners), or headers (lanes 56..63)
    const bool header = lane >= uint32_t(kRsOwners);
    const uint32_t k = header ? 0u : lane >> 2, g = lane & 3u;
    const bool owner = !header && k < nb;
    const uint32_t hk = lane - uint32_t(kRsOwners);  // header lanes: blocks hk, hk + 8
    const uint32_t oa = header ? min(hk, nb - 1u) * kQ4Bytes : min(k, nb - 1u) * kQ4Bytes + 16u + 32u * g;
    const uint32_t ob = header ? min(hk + 8u, nb - 1u) * kQ4Bytes : oa + 16u;
    // header of this lane's block: lane 56 + (k & 7), load a (k < 8) or b
    const uint32_t src4 = (uint32_t(kRsOwners) + (k & 7u)) << 2;
    const bool from_b = k >= 8u;
    // Where the lane's (scale, min) pairs of sub-blocks j = 2g, 2g + 1 sit in
    // the 12 scale bytes (s1, s2, s3 = bytes 0-3, 4-7, 8-11).  j < 4: scale j
    // = byte j & 63, min j = byte j + 4 & 63.  j >= 4: the low 4 bits of scale
    // / min j are the low / high nibble of byte j + 4, their top 2 bits the
    // top bits of byte j - 4 / byte j.  With sh = 16 (g & 1) each is a
    // bit-field extract of width fw (6 or 4) from s1 / s2 or s3, plus tw (0
    // or 2) top bits from s1 / s2.
    const bool hi = g >= 2u;
    const uint32_t sh = 16u * (g & 1u), fw = hi ? 4u : 6u, tw = hi ? 2u : 0u, om = hi ? sh + 4u : sh;

    // a ring item: one tile's chunks (or headers) and epilogue operands
    struct Item {
        uint4 a[NMAT][RPL], b[NMAT][RPL];
        float res[RPL], bias[RPL];
    };
    auto load = [&](uint32_t ti, Item& it) {
        const uint32_t tile = min(gw + ti * stride, ntiles - 1u);
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = min(tile * RPL + r, p.rows - 1u);  // clamp: result discarded
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const uint8_t* base = (m == 0 ? p.w0 : p.w1) + uint64_t(row) * p.row_bytes;
                it.a[m][r] = *reinterpret_cast<const uint4*>(base + oa);
                it.b[m][r] = *reinterpret_cast<const uint4*>(base + ob);
            }
            it.res[r] = 0.0f;
            it.bias[r] = 0.0f;
            if constexpr (EPI == EPI_PLAIN) {
                if (p.res) it.res[r] = p.res[row];
                if (p.flags & F_BIAS) it.bias[r] = p.bias[row];
            }
        }
    };

    // x of the workgroup, staged once into LDS with the norm: this thread's
    // float4s of x (and of the norm weights) are loaded before the ring
    // (loads complete in issue order, so the staging waits for x alone)
    constexpr int NT = W * kWave;
    constexpr int XQ = (kRsMaxBlocks * kQK / 4 + NT - 1) / NT;  // float4s of x per thread, at most
    const uint32_t nq = nb * (kQK / 4);
    float4 xq[XQ], wq[NORM ? XQ : 1];
#pragma unroll
    for (int i = 0; i < XQ; ++i) {
        const uint32_t q = min(threadIdx.x + uint32_t(i * NT), nq - 1u);
        xq[i] = reinterpret_cast<const float4*>(p.x)[q];
        if constexpr (NORM) wq[i] = reinterpret_cast<const float4*>(p.normw)[q];
    }
    Item buf[kRsRing];
#pragma unroll
    for (int i = 0; i < kRsRing - 1; ++i) load(uint32_t(i), buf[i]);

    float inv = 1.0f;
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XQ; ++i)
            if (threadIdx.x + uint32_t(i * NT) < nq) {
                ss = __builtin_fmaf(xq[i].x, xq[i].x, ss);
                ss = __builtin_fmaf(xq[i].y, xq[i].y, ss);
                ss = __builtin_fmaf(xq[i].z, xq[i].z, ss);
                ss = __builtin_fmaf(xq[i].w, xq[i].w, ss);
            }
        ss = block_sum<NT>(ss, red);
        inv = 1.0f / sqrtf(ss / float(nb * kQK) + p.eps);
    }
#pragma unroll
    for (int i = 0; i < XQ; ++i) {
        const uint32_t q = threadIdx.x + uint32_t(i * NT);
        if (q < nq) {
            float4 v = xq[i];
            if constexpr (NORM) {
                v.x = (v.x * inv) * wq[i].x;
                v.y = (v.y * inv) * wq[i].y;
                v.z = (v.z * inv) * wq[i].z;
                v.w = (v.w * inv) * wq[i].w;
            }
            *reinterpret_cast<float4*>(xs + rs_lds_index(q * 4u)) = v;
        }
    }
    __syncthreads();

    // this lane's 64 values into registers: e + [0, 32) (sub-block 2g) times
    // 2^24, e + [32, 64) (sub-block 2g + 1) times 2^20, with their plain sums
    RsX x;
    {
        const float* xe = xs + rs_lds_index(min(k, nb - 1u) * kQK + 64u * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x.a[i] = *reinterpret_cast<const float4*>(xe + 4 * i);
            x.b[i] = *reinterpret_cast<const float4*>(xe + 16 + 4 * i);
            x.c[i] = *reinterpret_cast<const float4*>(xe + 32 + 4 * i);
            x.d[i] = *reinterpret_cast<const float4*>(xe + 48 + 4 * i);
        }
    }
    x.s_lo = sum4(x.a) + sum4(x.b);
    x.s_hi = sum4(x.c) + sum4(x.d);
    scale4(x.a, 16777216.0f);
    scale4(x.b, 16777216.0f);
    scale4(x.c, 1048576.0f);
    scale4(x.d, 1048576.0f);

    auto consume = [&](uint32_t ti, const Item& it) {
        const uint32_t tile = gw + ti * stride;
        float acc[NMAT][RPL];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                // the block header from its header lane (every lane permutes)
                const uint32_t dm_a = bperm(src4, it.a[m][r].x), dm_b = bperm(src4, it.b[m][r].x);
                const uint32_t s1a = bperm(src4, it.a[m][r].y), s1b = bperm(src4, it.b[m][r].y);
                const uint32_t s2a = bperm(src4, it.a[m][r].z), s2b = bperm(src4, it.b[m][r].z);
                const uint32_t s3a = bperm(src4, it.a[m][r].w), s3b = bperm(src4, it.b[m][r].w);
                acc[m][r] = 0.0f;
                if (owner) {
                    const uint32_t dm = from_b ? dm_b : dm_a, s1 = from_b ? s1b : s1a;
                    const uint32_t s2 = from_b ? s2b : s2a, s3 = from_b ? s3b : s3a;
                    const uint32_t ls = hi ? s3 : s1, lm = hi ? s3 : s2;
                    const float sc0 = float(__builtin_amdgcn_ubfe(ls, sh, fw) | (__builtin_amdgcn_ubfe(s1, sh + 6u, tw) << 4));
                    const float sc1 =
                        float(__builtin_amdgcn_ubfe(ls, sh + 8u, fw) | (__builtin_amdgcn_ubfe(s1, sh + 14u, tw) << 4));
                    const float mn0 = float(__builtin_amdgcn_ubfe(lm, om, fw) | (__builtin_amdgcn_ubfe(s2, sh + 6u, tw) << 4));
                    const float mn1 =
                        float(__builtin_amdgcn_ubfe(lm, om + 8u, fw) | (__builtin_amdgcn_ubfe(s2, sh + 14u, tw) << 4));
                    // four chains: chunk 2g / 2g + 1, low / high nibbles
                    float alo = 0.0f, ahi = 0.0f, blo = 0.0f, bhi = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        rs_dword(comp(it.a[m][r], j), x.a[j], x.c[j], alo, ahi);
                        rs_dword(comp(it.b[m][r], j), x.b[j], x.d[j], blo, bhi);
                    }
                    float qs = sc0 * (alo + blo);
                    qs = __builtin_fmaf(sc1, ahi + bhi, qs);
                    float ms = mn0 * x.s_lo;
                    ms = __builtin_fmaf(mn1, x.s_hi, ms);
                    acc[m][r] = fmix(dm, false, qs, 0.0f);        // d * qs
                    acc[m][r] = fmix(dm, true, -ms, acc[m][r]);   // - dmin * ms
                }
                acc[m][r] = group_sum<kWave>(acc[m][r]);
            }
        if (lane != 0) return;
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = tile * RPL + r;
            if (row >= p.rows) continue;
            if constexpr (EPI == EPI_SWIGLU) {
                const float gv = acc[0][r], uv = acc[1][r];
                p.y[row] = (gv / (1.0f + expf(-gv))) * uv;
            } else {
                float val = acc[0][r];
                if (p.flags & F_BIAS) val = val + it.bias[r];
                if (p.res) val = it.res[r] + val;
                p.y[row] = val;
            }
        }
    };

    // the ring: kRsRing - 1 tiles' loads in flight while one is used (loads
    // past the last tile repeat it; items t .. t + kRsRing - 2 sit in slots
    // 0 .. kRsRing - 2 whenever t is a multiple of kRsRing)
    uint32_t t = 0;
    for (; t + kRsRing <= my; t += kRsRing) {
#pragma unroll
        for (int u = 0; u < kRsRing; ++u) {
            load(t + uint32_t(u + kRsRing - 1), buf[(u + kRsRing - 1) % kRsRing]);
            consume(t + uint32_t(u), buf[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < kRsRing - 1; ++u)
        if (t + uint32_t(u) < my) consume(t + uint32_t(u), buf[u]);
}

template <int NMAT, int RPL, int EPI, bool NORM, int W>
__global__ __launch_bounds__(W * kWave) void k_gemv_rs(GemvParams p)
{
    clear_done_copies(p);
    gemv_rs_body<NMAT, RPL, EPI, NORM, W>(p, blockIdx.x, gridDim.x);
}

}  // namespace arc
