// arc_gemv.hpp -- the packed Q4_K/Q6_K GEMV core for gfx950 (device code and
// its launch helpers), shared by the standalone kernels (arc_kernels.hip) and
// the decode-step runtime (arc_decode.hip).
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
#pragma once

#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

namespace arc {


constexpr int kPanel = 80;  // max super-block columns of x staged per launch (87 KB LDS)
constexpr int kWaves = 4;   // waves per GEMV workgroup (default layout)
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxWaves = 8;  // larger workgroups share one staged x when LDS limits residency

// EPI_COLPART: split-K with one super-block column per split -- each quad's
// own sum is the partial of (column, row), written without a cross-quad
// reduction, so every column of a row is handled by one launch; with y2 set
// the owning wave also adds the row's partials in column order.
// EPI_QKROPE: decode q/k projection -- rows [0, row_split) of w0 (q) then
// rows of w1 (k), + bias, RoPE on adjacent row pairs (2m, 2m+1) of each
// 128-wide head (RPL = 2 keeps a pair in one lane), q -> y (fp32), k -> fp16
// cache row at the current position.  EPI_VSTORE: + bias -> fp16 cache row.
enum Epi {
    EPI_PLAIN = 0,
    EPI_SWIGLU = 1,
    EPI_PARTIAL = 2,
    EPI_ARGMAX = 3,
    EPI_COLPART = 4,
    EPI_QKROPE = 5,
    EPI_VSTORE = 6
};

// F_EMBED: x is row ctl->token of the Q4_K table `emb`, decoded while it is
// staged (with F_NORM over the whole of x); workgroup 0 also writes the raw
// row to h_out.  F_ARGNEXT (EPI_ARGMAX): the launch finishes the argmax
// itself -- the last workgroup to arrive folds every workgroup's best and
// advances the decode control block (token, position, step, out_tokens).
enum Flag : uint32_t { F_NORM = 1u, F_ACCUM = 2u, F_BIAS = 4u, F_EMBED = 8u, F_ARGNEXT = 16u };

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
    // decode-step extensions
    const float* res;         // PLAIN: y = res + dot (+ bias) when set
    const float* bias2;       // QKROPE: bias of the rows from w1
    uint32_t row_split;       // QKROPE: first row taken from w1
    uint32_t kv_dim;          // QKROPE/VSTORE: cache row width (kv heads * 128)
    _Float16* cache;          // QKROPE/VSTORE: this layer's cache, [ctx][kv_dim]
    const float2* rope;       // QKROPE: (cos, sin) of pos * theta^(-2p/128), [ctx][64]
    DecodeCtl* ctl;           // QKROPE/VSTORE: current position; F_EMBED: token; F_ARGNEXT: advanced
    float* y2;                // COLPART over all of K: y2 = res + fixed-order sum of the row's partials
    const uint8_t* emb;       // F_EMBED: Q4_K token table, rows of nb super-blocks
    float* h_out;             // F_EMBED: workgroup 0 writes the decoded row here
    uint32_t* counter;        // F_ARGNEXT: arrival counter (zero between launches)
    uint32_t* out_tokens;     // F_ARGNEXT: token of decode step ctl->step, if step < out_cap
    uint32_t out_cap;
    uint32_t emb_rows;        // F_EMBED: rows of `emb` (a token id past them reads row 0)
    uint32_t ctx_rows;        // QKROPE/VSTORE: rows of the cache and RoPE table (positions clamped below)
    uint32_t* clear_done;     // when set: the kDoneCopies copies of a done counter the previous launch
                              // waited on, zeroed by workgroup 0 (that launch has ended)
};

// Zeroes the done-counter copies p.clear_done (workgroup 0 of the launch).
__device__ __forceinline__ void clear_done_copies(const GemvParams& p)
{
    if (p.clear_done && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < unsigned(kDoneCopies))
        p.clear_done[threadIdx.x * kDoneStride] = 0u;
}

// ------------------------------------------------------------ block loads
// The header is read as the d/dmin dword and the 12 scale bytes separately:
// held as one 16-byte register tuple, its parts live for different times and
// the register allocator copied them out right after the load, a copy that
// waits for the load (the prefetch a block ahead then gains nothing).
typedef uint32_t u32x3a4 __attribute__((ext_vector_type(3), aligned(4)));
struct Q4Blk {
    uint32_t dm;    // d | dmin << 16
    u32x3a4 sc;     // the 12 packed 6-bit scale/min bytes
    uint4 qa, qb;
};

__device__ __forceinline__ void q4_load(const uint8_t* blk, int v, Q4Blk& o)
{
    o.dm = *reinterpret_cast<const uint32_t*>(blk);
    o.sc = *reinterpret_cast<const u32x3a4*>(blk + opaque(4u));  // kept apart from the dword before it
    o.qa = ld16_aligned(blk + 16 + v * 16);
    o.qb = ld16_aligned(blk + 80 + v * 16);
}

// A Q6_K block (210 bytes) starts 0 or 2 bytes past a dword boundary.  It is
// read with buffer loads over the whole tensor (a uniform descriptor in
// SGPRs, 32-bit byte offsets: no 64-bit address arithmetic per load).  Each
// 16-byte chunk is read as a dwordx4 plus the following dword from the
// dword-aligned address below it and kept as read; q6_dot realigns it (by sh
// bytes) where it is consumed, so nothing waits for a load right after
// issuing it.  The dwords read cover block bytes [o-2, o+18) for o <= 192;
// past the tensor's end the hardware returns zeros instead of reading.
// Pieces: 0, 1 ql of both 128-element halves, 2, 3 the matching qh, 4 the
// int8 scales (its trailing dword holds d).
struct Q6Blk {
    uint32_t w[5][5];
    uint32_t sh;
};

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Raw buffer descriptor of `bytes` bytes at `base` (uniform arguments).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tensor_rsrc(const uint8_t* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, int(bytes), 0x00020000);
}

// The block at byte offset `off` of a tensor that starts base_sh bytes past
// the dword-aligned base of descriptor r.
__device__ __forceinline__ void q6_load(__amdgpu_buffer_rsrc_t r, uint32_t base_sh, uint32_t off, int v, Q6Blk& o)
{
    const uint32_t sh = (off + base_sh) & 3u;
    const uint32_t a = off + base_sh - sh;
    const uint32_t ql = a + uint32_t(v) * 16u, qh = a + uint32_t(v & 1) * 16u;
    const uint32_t at[5] = {ql, ql + 64u, qh + 128u, qh + 160u, a + 192u};
#pragma unroll
    for (int p = 0; p < 5; ++p) {
        const u32x4v x = __builtin_amdgcn_raw_buffer_load_b128(r, at[p], 0, 0);
        o.w[p][0] = x.x;
        o.w[p][1] = x.y;
        o.w[p][2] = x.z;
        o.w[p][3] = x.w;
        o.w[p][4] = __builtin_amdgcn_raw_buffer_load_b32(r, at[p] + 16u, 0, 0);
    }
    o.sh = sh;
}

// Padded Q6_K (212-byte blocks, each at a dword boundary): the same pieces
// read at their own addresses, nothing to realign; d is the low half of the
// dword at 208.
__device__ __forceinline__ void q6p_load(__amdgpu_buffer_rsrc_t r, uint32_t off, int v, Q6Blk& o)
{
    const uint32_t ql = off + uint32_t(v) * 16u, qh = off + uint32_t(v & 1) * 16u;
    const uint32_t at[5] = {ql, ql + 64u, qh + 128u, qh + 160u, off + 192u};
#pragma unroll
    for (int p = 0; p < 5; ++p) {
        const u32x4v x = __builtin_amdgcn_raw_buffer_load_b128(r, at[p], 0, 0);
        o.w[p][0] = x.x;
        o.w[p][1] = x.y;
        o.w[p][2] = x.z;
        o.w[p][3] = x.w;
        o.w[p][4] = 0u;
    }
    o.w[4][4] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 208u, 0, 0);
    o.sh = 0u;
}

// EXEC148 block (148 bytes, 4-byte aligned): bytes 0..3 d, dmin; 4 + 2j,
// 5 + 2j the unpacked (sc_j, mn_j); from 20 the codes, element k in byte
// 20 + k/2 (low nibble for even k).  Lane v reads the d/dmin dword, the dword
// of its two sub-blocks' (sc, mn) and the 32 code bytes of its 64 elements;
// every read lies inside the block.
struct E148Blk {
    uint32_t dm;    // d | dmin << 16
    uint32_t sc;    // sc_{2v}, mn_{2v}, sc_{2v+1}, mn_{2v+1}
    uint32_t c[8];  // elements 64v + 8i .. +7 in dword i
};

__device__ __forceinline__ void e148_load(const uint8_t* blk, int v, E148Blk& o)
{
    const uint32_t* w = reinterpret_cast<const uint32_t*>(blk);
    o.dm = w[0];
    o.sc = w[1 + v];
    const u32x4a4 a = *reinterpret_cast<const u32x4a4*>(blk + 20 + 32 * v);
    const u32x4a4 b = *reinterpret_cast<const u32x4a4*>(blk + 36 + 32 * v);
    o.c[0] = a.x;
    o.c[1] = a.y;
    o.c[2] = a.z;
    o.c[3] = a.w;
    o.c[4] = b.x;
    o.c[5] = b.y;
    o.c[6] = b.z;
    o.c[7] = b.w;
}

template <int FMT>
struct BlkOf;
template <>
struct BlkOf<kFmtE148> {
    using T = E148Blk;
    static constexpr int bytes = kE148Bytes;
};
template <>
struct BlkOf<kFmtQ4> {
    using T = Q4Blk;
    static constexpr int bytes = kQ4Bytes;
};
template <>
struct BlkOf<kFmtQ6P> {
    using T = Q6Blk;
    static constexpr int bytes = kQ6PBytes;
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

// Two mix4 chains advanced in turn (no back-to-back dependent v_fma_mix).
__device__ __forceinline__ void mix4x2(uint32_t ca, const float4& xa, float& aa, uint32_t cb, const float4& xb,
                                       float& ab)
{
    const uint32_t eva = opaque(ca & 0x00ff00ffu);
    const uint32_t oda = opaque(__builtin_amdgcn_perm(0u, ca, 0x0c030c01u));
    const uint32_t evb = opaque(cb & 0x00ff00ffu);
    const uint32_t odb = opaque(__builtin_amdgcn_perm(0u, cb, 0x0c030c01u));
    aa = fmix(eva, false, xa.x, aa);
    ab = fmix(evb, false, xb.x, ab);
    aa = fmix(oda, false, xa.y, aa);
    ab = fmix(odb, false, xb.y, ab);
    aa = fmix(eva, true, xa.z, aa);
    ab = fmix(evb, true, xb.z, ab);
    aa = fmix(oda, true, xa.w, aa);
    ab = fmix(odb, true, xb.w, ab);
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
            // the four group chains advance in turn, so consecutive
            // v_fma_mix never depend on each other
            a[n][0] = fmix(aL, false, x0.x, a[n][0]);
            a[n][1] = fmix(aH, false, x1.x, a[n][1]);
            a[n][2] = fmix(bL, false, x2.x, a[n][2]);
            a[n][3] = fmix(bH, false, x3.x, a[n][3]);
            a[n][0] = fmix(aLo, false, x0.y, a[n][0]);
            a[n][1] = fmix(aHo, false, x1.y, a[n][1]);
            a[n][2] = fmix(bLo, false, x2.y, a[n][2]);
            a[n][3] = fmix(bHo, false, x3.y, a[n][3]);
            a[n][0] = fmix(aL, true, x0.z, a[n][0]);
            a[n][1] = fmix(aH, true, x1.z, a[n][1]);
            a[n][2] = fmix(bL, true, x2.z, a[n][2]);
            a[n][3] = fmix(bH, true, x3.z, a[n][3]);
            a[n][0] = fmix(aLo, true, x0.w, a[n][0]);
            a[n][1] = fmix(aHo, true, x1.w, a[n][1]);
            a[n][2] = fmix(bLo, true, x2.w, a[n][2]);
            a[n][3] = fmix(bHo, true, x3.w, a[n][3]);
        }
    }
    const float4 S = lds4(xs + 64);
    const int sh = 16 * (v >> 1);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        // bytes of sc/mn for this lane's sub-blocks (2g, 2g+1, 2g+4, 2g+5), g = v>>1
        const uint32_t yy = b[n].sc.x >> sh, zz = b[n].sc.y >> sh, ww = b[n].sc.z >> sh;
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
        acc[n] = fmix(b[n].dm, false, qs, acc[n]);   // + d * qs
        acc[n] = fmix(b[n].dm, true, -ms, acc[n]);   // - dmin * ms
    }
}

// Q6_K: the 6-bit codes u of one ql/qh dword pair are assembled per byte,
// ua = low nibbles | bits (2qa, 2qa+1) of qh moved to bits 4-5, ub = high
// nibbles | bits (2qa+4, 2qa+5); then read as fp16 subnormals u*2^-24 (the
// staged x carries 2^24).
template <int N, bool PADDED>
__device__ __forceinline__ void q6_dot(const Q6Blk (&b)[N], const float* xs, int v, float (&acc)[N])
{
    // dword i of piece p of the block itself
    auto q6w = [](const Q6Blk& bb, int p, int i) -> uint32_t {
        if constexpr (PADDED)
            return bb.w[p][i];
        else
            return __builtin_amdgcn_alignbyte(bb.w[p][i + 1], bb.w[p][i], bb.sh);
    };
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
                const uint32_t ql = q6w(b[n], h, dw), qh = q6w(b[n], 2 + h, dw);
                const uint32_t ua = (ql & 0x0f0f0f0fu) | ((qh << s1) & 0x30303030u);
                const uint32_t ub = ((ql >> 4) & 0x0f0f0f0fu) | ((qh >> s2) & 0x30303030u);
                mix4x2(ua, xa, a[n][2 * h], ub, xb, a[n][2 * h + 1]);
            }
        }
    }
    const float4 S = lds4(xs + 64);
    // scale of group t is byte i0 of scale dword t (i0 = (v&1) + 2*qa)
    const uint32_t i0 = 8u * ((v & 1) + 2 * qa);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        float t = float(int8_t(uint8_t(q6w(b[n], 4, 0) >> i0))) * __builtin_fmaf(-32.0f, S.x, a[n][0]);
        t = __builtin_fmaf(float(int8_t(uint8_t(q6w(b[n], 4, 1) >> i0))), __builtin_fmaf(-32.0f, S.y, a[n][1]), t);
        t = __builtin_fmaf(float(int8_t(uint8_t(q6w(b[n], 4, 2) >> i0))), __builtin_fmaf(-32.0f, S.z, a[n][2]), t);
        t = __builtin_fmaf(float(int8_t(uint8_t(q6w(b[n], 4, 3) >> i0))), __builtin_fmaf(-32.0f, S.w, a[n][3]), t);
        const uint32_t d = PADDED ? b[n].w[4][4] : b[n].w[4][4] >> (8u * b[n].sh);  // bytes 208, 209 in the low half
        acc[n] = fmix(d, false, t, acc[n]);  // + d * t
    }
}

// EXEC148: each code dword holds 8 consecutive elements, two per byte; the
// even elements are read as fp16 subnormals q*2^-24 (w & 0x000f000f and the
// same of w >> 8), the odd ones as q*2^-20 (w & 0x00f000f0, ...): the staged
// x carries 2^24 on even and 2^20 on odd elements.  Groups 0, 1 belong to
// sub-block 2v, groups 2, 3 to 2v+1:
//   sum_k (d sc q - dmin mn) x = d sum_g sc_g (q.x)_g - dmin sum_g mn_g (sum x)_g
template <int N>
__device__ __forceinline__ void e148_dot(const E148Blk (&b)[N], const float* xs, float (&acc)[N])
{
    float a[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) a[n][0] = a[n][1] = a[n][2] = a[n][3] = 0.0f;
#pragma unroll
    for (int dw = 0; dw < 2; ++dw) {
        float4 xl[4], xh[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            xl[t] = lds4(xs + t * 16 + dw * 8);
            xh[t] = lds4(xs + t * 16 + dw * 8 + 4);
        }
#pragma unroll
        for (int n = 0; n < N; ++n) {
            uint32_t L[4], H[4], Lo[4], Ho[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t w = b[n].c[2 * t + dw], w8 = w >> 8;
                L[t] = opaque(w & 0x000f000fu);
                H[t] = opaque(w & 0x00f000f0u);
                Lo[t] = opaque(w8 & 0x000f000fu);
                Ho[t] = opaque(w8 & 0x00f000f0u);
            }
            // the four group chains advance in turn
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(L[t], false, xl[t].x, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(H[t], false, xl[t].y, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(Lo[t], false, xl[t].z, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(Ho[t], false, xl[t].w, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(L[t], true, xh[t].x, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(H[t], true, xh[t].y, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(Lo[t], true, xh[t].z, a[n][t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) a[n][t] = fmix(Ho[t], true, xh[t].w, a[n][t]);
        }
    }
    const float4 S = lds4(xs + 64);
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float sc0 = byte_f(b[n].sc, 0), mn0 = byte_f(b[n].sc, 1);
        const float sc1 = byte_f(b[n].sc, 2), mn1 = byte_f(b[n].sc, 3);
        float qs = sc0 * a[n][0];
        qs = __builtin_fmaf(sc0, a[n][1], qs);
        qs = __builtin_fmaf(sc1, a[n][2], qs);
        qs = __builtin_fmaf(sc1, a[n][3], qs);
        float ms = mn0 * S.x;
        ms = __builtin_fmaf(mn0, S.y, ms);
        ms = __builtin_fmaf(mn1, S.z, ms);
        ms = __builtin_fmaf(mn1, S.w, ms);
        acc[n] = fmix(b[n].dm, false, qs, acc[n]);   // + d * qs
        acc[n] = fmix(b[n].dm, true, -ms, acc[n]);   // - dmin * ms
    }
}

template <int FMT, int N>
__device__ __forceinline__ void blk_dot(const typename BlkOf<FMT>::T (&b)[N], const float* xs, int v,
                                        float (&acc)[N])
{
    if constexpr (FMT == kFmtQ4)
        q4_dot<N>(b, xs, v, acc);
    else if constexpr (FMT == kFmtE148)
        e148_dot<N>(b, xs, acc);
    else
        q6_dot<N, FMT == kFmtQ6P>(b, xs, v, acc);
}

// Q4_K and EXEC148 blocks (16- and 4-byte aligned) are read through their
// address; Q6_K blocks through the tensor's buffer descriptor (q6_load).
template <int FMT>
__device__ __forceinline__ void blk_load(const uint8_t* blk, int v, typename BlkOf<FMT>::T& o)
{
    static_assert(FMT != kFmtQ6, "Q6_K blocks are read with q6_load");
    if constexpr (FMT == kFmtQ4)
        q4_load(blk, v, o);
    else
        e148_load(blk, v, o);
}

// ------------------------------------------------------------- reductions
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
template <int FMT>
__device__ __forceinline__ void put_group(float* lds, uint32_t gi, const float4 (&q)[4])
{
    const uint32_t bl = gi >> 4, v = (gi >> 2) & 3u, t = gi & 3u;
    float* dst = lds + bl * kXBlk + v * kSlot + t * 16;
    const float unit = (FMT == kFmtQ4 && (t & 1u)) ? 1048576.0f : 16777216.0f;  // 2^20 : 2^24
    // EXEC148: 2^24 on even elements, 2^20 on odd ones
    const float uo = FMT == kFmtE148 ? 1048576.0f : unit;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s += q[i].x;
        s += q[i].y;
        s += q[i].z;
        s += q[i].w;
        reinterpret_cast<float4*>(dst)[i] = make_float4(q[i].x * unit, q[i].y * uo, q[i].z * unit, q[i].w * uo);
    }
    lds[bl * kXBlk + v * kSlot + 64 + t] = s;
}

template <int FMT>
__device__ __forceinline__ uint32_t group_elem(uint32_t b0, uint32_t gi)
{
    return (b0 + (gi >> 4)) * kQK + x_group_offset<FMT>(int((gi >> 2) & 3u), int(gi & 3u));
}

__device__ __forceinline__ void ld_group(const float* p, float4 (&q)[4])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = reinterpret_cast<const float4*>(p)[i];
}

__device__ __forceinline__ void scale_group(float4 (&q)[4], float inv, const float4 (&w)[4])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[i].x = (q[i].x * inv) * w[i].x;
        q[i].y = (q[i].y * inv) * w[i].y;
        q[i].z = (q[i].z * inv) * w[i].z;
        q[i].w = (q[i].w * inv) * w[i].w;
    }
}

// The first groups of x a thread stages (with the fused RMSNorm: its one
// first group, and that group of the norm weights), loaded before the
// weight ring's first loads.  Loads complete in issue order, so staging
// then waits for x alone, not for the ring's HBM loads behind it.  With
// 8-wave workgroups these are all of the thread's groups of an 80-block
// panel (the FFN down's 74 blocks: 1184 groups over 512 threads, 3 each),
// so a wide panel waits for one round trip, not one per group; 4-wave
// workgroups stage at most 37 blocks (wider panels take 8 waves) and spend
// their registers on the prefetch ring.
template <int NT>
struct XPre {
    static constexpr int G = NT >= 512 ? (kPanel * 16 + NT - 1) / NT : 1;
    float4 q[G][4];
    float4 w[4];
};

template <int FMT, int NT>
__device__ __forceinline__ void x_pre(XPre<NT>& pre, const float* __restrict__ x, uint32_t b0, uint32_t nbl, bool rms,
                                      const float* __restrict__ normw)
{
    // Indices are clamped into the panel instead of branching around the
    // loads (registers loaded under a branch are waited for where it joins);
    // groups past the panel load a valid group and are not stored.  The
    // fused RMSNorm stages the whole row (b0 = 0), so its first group is
    // q[0] here too; the embedding row (erow) is decoded in stage_x_rms.
    const uint32_t last = nbl * 16u - 1u;
#pragma unroll
    for (int i = 0; i < XPre<NT>::G; ++i)
        ld_group(x + group_elem<FMT>(b0, min(threadIdx.x + uint32_t(i * NT), last)), pre.q[i]);
    if (rms) ld_group(normw + group_elem<FMT>(0, min(uint32_t(threadIdx.x), last)), pre.w);
}

template <int FMT, int NT>
__device__ void stage_x(float* lds, XPre<NT>& pre, const float* __restrict__ x, uint32_t b0, uint32_t nbl, bool norm,
                        float inv, const float* __restrict__ normw)
{
    constexpr int G = XPre<NT>::G;
    const uint32_t ng = nbl * 16u;
    auto put = [&](uint32_t gi, float4 (&q)[4]) {
        if (norm) {
            float4 w[4];
            ld_group(normw + group_elem<FMT>(b0, gi), w);
            scale_group(q, inv, w);
        }
        put_group<FMT>(lds, gi, q);
    };
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const uint32_t gi = threadIdx.x + uint32_t(i * NT);
        if (gi < ng) put(gi, pre.q[i]);
    }
    for (uint32_t gi = threadIdx.x + uint32_t(G * NT); gi < ng; gi += NT) {
        float4 r[4];
        ld_group(x + group_elem<FMT>(b0, gi), r);
        put(gi, r);
    }
}

// Elements e .. e+15 (16-aligned, so inside one 32-element sub-block) of a
// Q4_K row, each decoded as the reference does: (d*sc)*q - dmin*mn with every
// product and the difference rounded separately
// (src/sa1_component_benchmark.cpp:105-116).
__device__ __forceinline__ void emb_group(const uint8_t* __restrict__ row, uint32_t e, float4 (&q)[4])
{
#pragma clang fp contract(off)
    const uint8_t* b = row + (e >> 8) * kQ4Bytes;
    const uint32_t k0 = e & 255u, j = k0 >> 5;
    const float d = f16_bits_to_f32(uint32_t(b[0]) | (uint32_t(b[1]) << 8));
    const float dm = f16_bits_to_f32(uint32_t(b[2]) | (uint32_t(b[3]) << 8));
    const uint8_t* sb = b + 4;
    uint32_t sc, mn;
    if (j < 4) {
        sc = sb[j] & 63u;
        mn = sb[j + 4] & 63u;
    } else {
        sc = (sb[j + 4] & 15u) | (uint32_t(sb[j - 4] >> 6) << 4);
        mn = (sb[j + 4] >> 4) | (uint32_t(sb[j] >> 6) << 4);
    }
    const float t0 = d * float(sc);
    const float t2 = dm * float(mn);
    const uint32_t l64 = k0 & 63u;
    const uint8_t* nib = b + 16 + (k0 >> 6) * 32 + (l64 & 31u);
    const uint32_t sh = l64 < 32u ? 0u : 4u;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float t1 = t0 * float((uint32_t(nib[i]) >> sh) & 15u);
        v[i] = t1 - t2;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

// One group of x: loaded from x, or (F_EMBED) decoded from the token's row.
__device__ __forceinline__ void x_group(const float* __restrict__ x, const uint8_t* __restrict__ erow, uint32_t e,
                                        float4 (&q)[4])
{
    if (erow)
        emb_group(erow, e, q);
    else
        ld_group(x + e, q);
}

__device__ __forceinline__ void st_group(float* p, const float4 (&q)[4])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float4*>(p)[i] = q[i];
}

// RMSNorm fused into the staging of the whole of x (nbl super-blocks): the
// thread's first group of x and of the norm weights is loaded once (by
// x_pre, ahead of the weight ring), its
// squares enter the block-wide sum of squares (fp32, fixed order: the
// thread's other groups first, then the first one, then the wave and
// workgroup trees), and it is scaled and stored without a second read.
template <int FMT, int NT>
__device__ void stage_x_rms(float* lds, XPre<NT>& pre, const float* x, uint32_t nbl, float eps,
                            const float* __restrict__ normw, float* red, const uint8_t* __restrict__ erow,
                            float* raw_out)
{
    const uint32_t ng = nbl * 16u, gi0 = threadIdx.x;
    const bool have = gi0 < ng;
    float4 (&q0)[4] = pre.q[0];
    float4 (&w0)[4] = pre.w;
    if (have && erow) {
        const uint32_t e = group_elem<FMT>(0, gi0);
        emb_group(erow, e, q0);
        if (raw_out) st_group(raw_out + e, q0);
    }
    float ss = 0.0f;
    for (uint32_t gi = gi0 + NT; gi < ng; gi += NT) {
        const uint32_t e = group_elem<FMT>(0, gi);
        float4 q[4];
        x_group(x, erow, e, q);
        if (raw_out) st_group(raw_out + e, q);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ss = __builtin_fmaf(q[i].x, q[i].x, ss);
            ss = __builtin_fmaf(q[i].y, q[i].y, ss);
            ss = __builtin_fmaf(q[i].z, q[i].z, ss);
            ss = __builtin_fmaf(q[i].w, q[i].w, ss);
        }
    }
    if (have)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ss = __builtin_fmaf(q0[i].x, q0[i].x, ss);
            ss = __builtin_fmaf(q0[i].y, q0[i].y, ss);
            ss = __builtin_fmaf(q0[i].z, q0[i].z, ss);
            ss = __builtin_fmaf(q0[i].w, q0[i].w, ss);
        }
    ss = block_sum<NT>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(nbl * kQK) + eps);
    if (have) {
        scale_group(q0, inv, w0);
        put_group<FMT>(lds, gi0, q0);
    }
    for (uint32_t gi = gi0 + NT; gi < ng; gi += NT) {
        const uint32_t e = group_elem<FMT>(0, gi);
        float4 q[4], w[4];
        x_group(x, erow, e, q);
        ld_group(normw + e, w);
        scale_group(q, inv, w);
        put_group<FMT>(lds, gi, q);
    }
}

__device__ __forceinline__ bool arg_better(float va, uint32_t ia, float vb, uint32_t ib)
{
    return va > vb || (va == vb && ia < ib);
}

// Argmax over a workgroup of (value, index) candidates, ties to the lowest
// index, plus a sum of the non-finite counts.  Called by every thread; every
// thread receives the result.
__device__ ArgBest wg_argmax(float bv, uint32_t bi, uint32_t nf)
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
    __shared__ ArgBest res;
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
        res = ArgBest{b, i, c, 0u};
    }
    __syncthreads();
    return res;
}

__device__ __forceinline__ void st_agent_best(ArgBest* p, const ArgBest& b)
{
    uint32_t* w = reinterpret_cast<uint32_t*>(p);
    st_agent(w, __builtin_bit_cast(uint32_t, b.val));
    st_agent(w + 1, b.idx);
    st_agent(w + 2, b.nonfinite);
}

// Second argmax stage inside the LM-head launch (F_ARGNEXT): the last
// workgroup to arrive folds the n per-workgroup bests (read past the L2, as
// the other workgroups wrote them) and advances the decode control block:
// token = argmax (0 if every logit was non-finite), out_tokens[step] = token,
// non-finite count, step + 1, position + 1.
template <int NT>
__device__ void argmax_finish(const GemvParams& p, uint32_t n)
{
    __shared__ uint32_t flag;
    if (!arrive_last(p.counter, n, &flag)) return;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu, nf = 0;
    for (uint32_t i = threadIdx.x; i < n; i += NT) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(p.best + i);
        const float v = __builtin_bit_cast(float, ld_agent(w));
        const uint32_t idx = ld_agent(w + 1);
        nf += ld_agent(w + 2);
        if (idx != 0xffffffffu && arg_better(v, idx, bv, bi)) {
            bv = v;
            bi = idx;
        }
    }
    const ArgBest r = wg_argmax(bv, bi, nf);
    if (threadIdx.x == 0) {
        DecodeCtl* ctl = p.ctl;
        const uint32_t tok = r.idx < p.rows ? r.idx : 0u;  // none (all non-finite): 0
        const uint32_t step = ctl->step;
        if (step < p.out_cap) p.out_tokens[step] = tok;
        ctl->token = tok;
        ctl->nonfinite += r.nonfinite;
        ctl->step = step + 1;
        ctl->pos += 1;
    }
}

// Register buffers in a GEMV's prefetch ring (PF - 1 items in flight while
// one is consumed).
#ifndef ARC_PF_Q4
#define ARC_PF_Q4 2
#endif
#ifndef ARC_PF_Q6
#define ARC_PF_Q6 2
#endif
#ifndef ARC_PF_E148
#define ARC_PF_E148 2
#endif
template <int FMT, int EPI>
constexpr int ring_depth()
{
    return FMT == kFmtQ4 ? ARC_PF_Q4 : (FMT == kFmtQ6 || FMT == kFmtQ6P) ? ARC_PF_Q6 : ARC_PF_E148;
}
static_assert(ARC_PF_Q4 >= 2 && ARC_PF_Q6 >= 2 && ARC_PF_E148 >= 2, "a ring holds at least two buffers");

// --------------------------------------------------------------- GEMV core
// When x is ready: at the launch's start (NoXWait), or, in a launch whose
// other part produces x, once a hook called by every thread of the
// workgroup returns (kWaits).  A waiting GEMV issues its ring's first loads
// before the wait and its x loads after it, with one more ring buffer, so
// the weights are in flight while x is being produced.
struct NoXWait {
    static constexpr bool kWaits = false;
    __device__ void operator()() const {}
};

// One workgroup's share of a GEMV launch: workgroup bx of gx (x dimension)
// and split blockIdx.y.  k_gemv runs it over the whole grid; a fused launch
// can give disjoint workgroup ranges to different GEMVs.
template <int FMT, int BS, int RPL, int EPI, int W, class XWait = NoXWait>
__device__ __forceinline__ void gemv_body(const GemvParams& p, uint32_t bx, uint32_t gx, const XWait& xwait = XWait{})
{
    static_assert(W == 4 || W == 8, "4 or 8 waves per workgroup");
    constexpr int NT = W * kWave;
    constexpr int PF = ring_depth<FMT, EPI>() + (XWait::kWaits ? 1 : 0);  // register buffers in the prefetch ring
    // 16-byte aligned: the staged x is read as float4; the base follows the
    // kernel's static LDS, whose size is not a multiple of 16 in general
    extern __shared__ __align__(16) float lds[];
    __shared__ float red[W];
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

    const uint32_t gw = bx * W + wave;
    const uint32_t stride = gx * W;
    const uint32_t my_tiles = gw < p.ntiles ? (p.ntiles - gw + stride - 1) / stride : 0u;
    const uint32_t S = my_tiles * nj;

    auto tile_row = [&](uint32_t tile, int j) { return tile * kTileRows + rg * RPL + j; };
    // Q6_K and padded Q6_K: a buffer descriptor over each matrix (the host
    // keeps such a tensor below 4 GiB); unused, and removed, for the other
    // formats (descriptor bases at the dword boundary at or below each tensor,
    // where a padded tensor starts; a Q6_K block's final dword holds 2 bytes
    // past the tensor, hence + 4)
    const uint32_t rows0 = EPI == EPI_QKROPE ? p.row_split : p.rows;
    const uint8_t* w1 = NMAT == 2 || EPI == EPI_QKROPE ? p.w1 : p.w0;
    const uint32_t sh0 = uint32_t(reinterpret_cast<uintptr_t>(p.w0)) & 3u;
    const uint32_t sh1 = uint32_t(reinterpret_cast<uintptr_t>(w1)) & 3u;
    const __amdgpu_buffer_rsrc_t q6r0 = tensor_rsrc(p.w0 - sh0, uint32_t(uint64_t(rows0) * p.row_bytes) + sh0 + 4u);
    const __amdgpu_buffer_rsrc_t q6r1 =
        tensor_rsrc(w1 - sh1, uint32_t(uint64_t(p.rows - (EPI == EPI_QKROPE ? rows0 : 0u)) * p.row_bytes) + sh1 + 4u);
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
                if constexpr (FMT == kFmtQ6P) {
                    const uint32_t col = (kb + bl) * uint32_t(kBB);
                    if constexpr (EPI == EPI_QKROPE) {
                        if (row < p.row_split)
                            q6p_load(q6r0, row * uint32_t(p.row_bytes) + col, v, b[m * RPL + r]);
                        else
                            q6p_load(q6r1, (row - p.row_split) * uint32_t(p.row_bytes) + col, v, b[m * RPL + r]);
                    } else {
                        q6p_load(m == 0 ? q6r0 : q6r1, row * uint32_t(p.row_bytes) + col, v, b[m * RPL + r]);
                    }
                } else if constexpr (FMT == kFmtQ6) {
                    const uint32_t col = (kb + bl) * uint32_t(kBB);
                    if constexpr (EPI == EPI_QKROPE) {
                        if (row < p.row_split)
                            q6_load(q6r0, sh0, row * uint32_t(p.row_bytes) + col, v, b[m * RPL + r]);
                        else
                            q6_load(q6r1, sh1, (row - p.row_split) * uint32_t(p.row_bytes) + col, v,
                                    b[m * RPL + r]);
                    } else {
                        q6_load(m == 0 ? q6r0 : q6r1, m == 0 ? sh0 : sh1, row * uint32_t(p.row_bytes) + col, v,
                                b[m * RPL + r]);
                    }
                } else {
                    const uint8_t* base;
                    if constexpr (EPI == EPI_QKROPE)
                        base = row < p.row_split ? p.w0 + uint64_t(row) * p.row_bytes
                                                 : p.w1 + uint64_t(row - p.row_split) * p.row_bytes;
                    else
                        base = (m == 0 ? p.w0 : p.w1) + uint64_t(row) * p.row_bytes;
                    blk_load<FMT>(base + uint64_t(kb + bl) * kBB, v, b[m * RPL + r]);
                }
            }
        }
    };

    // Ring of PF register buffers over the wave's flattened (tile, block
    // slot) items: PF-1 items are in flight while one is consumed (deeper
    // rings measured slower: the registers cost more residency than the
    // extra loads in flight recover).  The
    // first PF-1 loads are issued before the x staging.  Past the last item
    // the loads repeat it (a cache hit), keeping the sequence branch-free.
    // (Refilling each buffer after it is consumed instead, with all PF
    // first loads before the staging, measured slower: config-0 gate GEMV
    // 12.3 -> 14.7 us, decode 610 -> 585 tokens/s at 512 positions.)
    Blk buf[PF][N];
    uint32_t li = 0, lj = 0, lnext = 1;  // next item to load; items issued so far
    auto advance = [&](uint32_t& i, uint32_t& j) {
        if (++j == nj) {
            j = 0;
            ++i;
        }
    };
    auto load_next = [&](Blk (&b)[N]) {
        load(li, lj, b);
        if (lnext < S) advance(li, lj);
        ++lnext;
    };
    // x first (see XPre), then the ring's first loads
    const bool rms = (p.flags & F_NORM) && kb == 0 && nbl == p.nb;
    const uint8_t* erow = nullptr;
    // the embedding path exists only in the q/k/v epilogues (the first
    // layer's projections): its code costs the other GEMVs registers
    if constexpr (EPI == EPI_QKROPE || EPI == EPI_VSTORE)
        if (rms && (p.flags & F_EMBED)) {
            // the control block is device memory: an id past the table reads row 0, never past it
            const uint32_t tok = p.ctl->token;
            erow = p.emb + uint64_t(tok < p.emb_rows ? tok : 0u) * p.nb * kQ4Bytes;
        }
    XPre<NT> pre;
    if constexpr (!XWait::kWaits) x_pre<FMT, NT>(pre, p.x, kb, nbl, rms, p.normw);
#pragma unroll
    for (int u = 0; u < PF - 1; ++u) load_next(buf[u]);
    if constexpr (XWait::kWaits) {
        xwait();
        x_pre<FMT, NT>(pre, p.x, kb, nbl, rms, p.normw);
    }

    // Epilogue operands (bias, residual, accumulated output, RoPE factors) of
    // the tile being consumed, loaded at its first item ahead of that item's
    // prefetch: the epilogue then waits only for loads issued before the
    // prefetch, not for the prefetch itself (the load counter is in order).
    // The first tile's are fetched under the x staging.
    float ep_b[RPL], ep_r[RPL], ep_y[RPL];
    float2 ep_cs = {1.0f, 0.0f};
    uint32_t pos = 0;
    if constexpr (EPI == EPI_QKROPE || EPI == EPI_VSTORE) pos = min(p.ctl->pos, p.ctx_rows - 1u);
    auto load_ep = [&](uint32_t ti) {
        const uint32_t tile = min(gw + ti * stride, p.ntiles - 1);
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = min(tile_row(tile, r), p.rows - 1);
            ep_b[r] = 0.0f;
            ep_r[r] = 0.0f;
            ep_y[r] = 0.0f;
            if constexpr (EPI == EPI_PLAIN) {
                if (p.flags & F_BIAS) ep_b[r] = p.bias[row];
                if (p.res) ep_r[r] = p.res[row];
                if (p.flags & F_ACCUM) ep_y[r] = p.y[row];
            } else if constexpr (EPI == EPI_COLPART) {
                if (p.y2 && p.res) ep_r[r] = p.res[row];
            } else if constexpr (EPI == EPI_PARTIAL) {
                if (p.flags & F_ACCUM) ep_y[r] = p.y[uint64_t(row) * p.nsplit + split];
            } else if constexpr (EPI == EPI_VSTORE) {
                ep_b[r] = p.bias[row];
            } else if constexpr (EPI == EPI_QKROPE) {
                ep_b[r] = row < p.row_split ? p.bias[row] : p.bias2[row - p.row_split];
            }
        }
        if constexpr (EPI == EPI_QKROPE) {
            const uint32_t row = min(tile_row(tile, 0), p.rows - 1);
            const uint32_t lr = row < p.row_split ? row : row - p.row_split;
            ep_cs = p.rope[uint64_t(pos) * 64 + ((lr & 127u) >> 1)];
        }
    };
    load_ep(0);

    if (rms) {
        float* raw = erow && bx == 0 ? p.h_out : nullptr;
        stage_x_rms<FMT, NT>(lds, pre, p.x, nbl, p.eps, p.normw, red, erow, raw);
    } else {
        float inv = 1.0f;
        if (p.flags & F_NORM) inv = rms_inv<NT>(p.x, p.nb * kQK, p.eps, red);
        stage_x<FMT, NT>(lds, pre, p.x, kb, nbl, (p.flags & F_NORM) != 0, inv, p.normw);
    }
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
    // EPI_COLPART: each quad's column sum goes to the wave's rows in LDS
    // (after the staged x, row stride = panel).  At a tile's last column the
    // wave stores its rows' partials (row-major, consecutive lanes on
    // consecutive columns) and, with y2 set (the panel is all of K), lane 0 of
    // each row group adds the row's partials in column order, then res: the
    // split-K second pass, done by the wave that owns the row.
    float* colp = lds + p.panel * kXBlk + uint32_t(wave * kTileRows) * p.panel;
    auto finish_column = [&](uint32_t ti, uint32_t j) {
        float tot[N];
#pragma unroll
        for (int n = 0; n < N; ++n) {
            tot[n] = group_sum<4>(acc[n]);
            acc[n] = 0.0f;
        }
        const uint32_t c = bs + BS * j;
        if (v == 0 && c < nbl)
#pragma unroll
            for (int r = 0; r < RPL; ++r) colp[uint32_t(rg * RPL + r) * p.panel + c] = tot[r];
        if (j != nj - 1) return;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint32_t tile = gw + ti * stride, li = uint32_t(lane) & (4u * BS - 1u);
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = tile_row(tile, r);
            if (row >= p.rows) continue;
            const float* src = colp + uint32_t(rg * RPL + r) * p.panel;
            float* dst = p.y + uint64_t(row) * p.nsplit + kb;
            for (uint32_t cc = li; cc < nbl; cc += 4u * BS) dst[cc] = src[cc];
            if (p.y2 && li == 0) {
                float sum = 0.0f;
                for (uint32_t cc = 0; cc < nbl; ++cc) sum += src[cc];
                if (p.res) sum += ep_r[r];
                p.y2[row] = sum;
            }
        }
        // the next tile's column sums overwrite these rows
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
        if constexpr (EPI == EPI_QKROPE) {
            static_assert(RPL == 2, "RoPE pairs must sit in one lane");
            const uint32_t row = tile_row(tile, 0);  // even; row + 1 is its pair
            if (row >= p.rows) return;
            const bool isq = row < p.row_split;
            const uint32_t lr = isq ? row : row - p.row_split;
            const float a = tot[0] + ep_b[0], b = tot[1] + ep_b[1];
            const float c = ep_cs.x, sv = ep_cs.y;
            const float ra = a * c - b * sv, rb = a * sv + b * c;
            if (isq) {
                p.y[lr] = ra;
                p.y[lr + 1] = rb;
            } else {
                _Float16* dst = p.cache + uint64_t(pos) * p.kv_dim + lr;
                dst[0] = _Float16(ra);
                dst[1] = _Float16(rb);
            }
            return;
        }
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const uint32_t row = tile_row(tile, r);
            if (row >= p.rows) continue;
            if constexpr (EPI == EPI_PLAIN) {
                float val = tot[r];
                if (p.flags & F_ACCUM) val = ep_y[r] + val;
                if (p.flags & F_BIAS) val = val + ep_b[r];
                if (p.res) val = ep_r[r] + val;
                p.y[row] = val;
            } else if constexpr (EPI == EPI_VSTORE) {
                const float val = tot[r] + ep_b[r];
                p.cache[uint64_t(pos) * p.kv_dim + row] = _Float16(val);
            } else if constexpr (EPI == EPI_SWIGLU) {
                const float g = tot[r], u = tot[RPL + r];
                p.y[row] = (g / (1.0f + expf(-g))) * u;
            } else if constexpr (EPI == EPI_PARTIAL) {
                float* dst = p.y + uint64_t(row) * p.nsplit + split;
                *dst = (p.flags & F_ACCUM) ? ep_y[r] + tot[r] : tot[r];
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

    uint32_t ci = 0, cj = 0;  // item being consumed
    auto step = [&](Blk (&next)[N], const Blk (&cur)[N]) {
        if constexpr (EPI == EPI_PLAIN || EPI == EPI_PARTIAL || EPI == EPI_VSTORE || EPI == EPI_QKROPE ||
                      EPI == EPI_COLPART)
            if (cj == 0 && ci != 0) load_ep(ci);
        load_next(next);
        compute(cj, cur);
        if constexpr (EPI == EPI_COLPART)
            finish_column(ci, cj);
        else if (cj == nj - 1)
            finish(ci);
        advance(ci, cj);
    };
    // Whole rounds of the ring as straight-line code with no exit between
    // its items, so each buffer keeps its registers: when the items sat
    // behind a per-item exit test, the compiler folded them into one item per
    // iteration with copies between the buffers, and copying a buffer just
    // loaded waited for its loads, losing the prefetch.
    // Item k consumes buffer k % PF and loads into (k + PF - 1) % PF; the
    // unrolled indices are constants, so no buffer is ever copied.
    uint32_t s = 0;
    for (; s + PF <= S; s += PF) {
#pragma unroll
        for (int k = 0; k < PF; ++k) step(buf[(k + PF - 1) % PF], buf[k]);
    }
#pragma unroll
    for (int k = 0; k < PF - 1; ++k)
        if (s + k < S) step(buf[(k + PF - 1) % PF], buf[k]);

    if constexpr (EPI == EPI_ARGMAX) {
        const ArgBest r = wg_argmax(best_v, best_i, nonfinite);
        if (p.flags & F_ARGNEXT) {
            if (threadIdx.x == 0) st_agent_best(p.best + bx, r);
            argmax_finish<NT>(p, gx);
        } else if (threadIdx.x == 0) {
            p.best[bx] = r;
        }
    }
}

template <int FMT, int BS, int RPL, int EPI, int W>
__global__ __launch_bounds__(W * kWave) void k_gemv(GemvParams p)
{
    clear_done_copies(p);
    gemv_body<FMT, BS, RPL, EPI, W>(p, blockIdx.x, gridDim.x);
}

}  // namespace arc

#include "arc_gemv_rs.hpp"

namespace arc {

// --------------------------------------------------------------- launching
struct Cfg {
    int bs, rpl, waves;  // quads per row, rows per lane, waves per workgroup (0 = default)
};

inline int tile_rows(const Cfg& c) { return (kWave / (4 * c.bs)) * c.rpl; }

inline int cu_count()
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
template <int FMT, int EPI, int BS, int RPL, int W>
int occupancy(size_t lds, uint32_t panel)
{
    static int occ[kPanel + 1] = {};
    const int slot = int(panel);
    if (!occ[slot]) {
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<FMT, BS, RPL, EPI, W>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_gemv<FMT, BS, RPL, EPI, W>, W * kWave, lds) != hipSuccess ||
            nb < 1)
            nb = 1;
        occ[slot] = nb;
    }
    return occ[slot];
}

// Launch state shared by every translation unit that includes this header
// (inline variables: one definition in the library, so a launch helper
// instantiated in one source file sees the flag another one set).
inline thread_local int g_wg_per_cu = 0;     // tuning override of resident workgroups per CU
inline thread_local bool g_dry_run = false;  // size grids and fill caches without launching

template <int FMT, int EPI, int BS, int RPL, int W = kWaves>
hipError_t launch_one(GemvParams p, uint32_t splits, hipStream_t s, uint32_t* grid_x)
{
    const Cfg c{BS, RPL, W};
    p.ntiles = (p.rows + tile_rows(c) - 1) / tile_rows(c);
    size_t lds = size_t(p.panel) * kXBlk * sizeof(float);
    if constexpr (EPI == EPI_COLPART) lds += size_t(W) * tile_rows(c) * p.panel * sizeof(float);
    const int per_cu = g_wg_per_cu > 0 ? g_wg_per_cu : occupancy<FMT, EPI, BS, RPL, W>(lds, p.panel);
    const uint64_t resident = uint64_t(per_cu) * cu_count();
    const uint64_t want = (p.ntiles + W - 1) / W;  // one wave tile per wave
    uint64_t gx = (resident + splits - 1) / splits;
    if (gx > want) gx = want;  // want <= ceil(rows / 4): one wave tile holds at least one row
    if (gx > 65536) gx = 65536;
    if (gx < 1) gx = 1;
    if (grid_x) *grid_x = uint32_t(gx);
    if (g_dry_run) return hipSuccess;
    hipLaunchKernelGGL((k_gemv<FMT, BS, RPL, EPI, W>), dim3(uint32_t(gx), splits), dim3(W * kWave), lds, s, p);
    return hipGetLastError();
}

// Row-stream launches (arc_gemv_rs.hpp): 12-wave workgroups (one per CU at
// 3 waves per SIMD: x is staged once per CU), the grid sized to the resident
// workgroups and to one row tile per wave.
constexpr int kRsWaves = 12;
inline thread_local int g_rowstream = -1;  // -1 automatic, 0 quad layout only, 1 row-stream where eligible

template <int NMAT, int RPL, int EPI, bool NORM, int W>
hipError_t launch_rs(const GemvParams& p, hipStream_t s, uint32_t* grid_x)
{
    static int occ = 0;
    if (!occ) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv_rs<NMAT, RPL, EPI, NORM, W>, W * kWave, 0) !=
                hipSuccess ||
            n < 1)
            n = 1;
        occ = n;
    }
    const int per_cu = g_wg_per_cu > 0 ? g_wg_per_cu : occ;
    const uint64_t tiles = (p.rows + RPL - 1) / RPL;
    const uint64_t want = (tiles + W - 1) / W;  // one tile per wave
    uint64_t gx = uint64_t(per_cu) * cu_count();
    if (gx > want) gx = want;
    if (gx > 65536) gx = 65536;
    if (grid_x) *grid_x = uint32_t(gx);
    if (g_dry_run) return hipSuccess;
    hipLaunchKernelGGL((k_gemv_rs<NMAT, RPL, EPI, NORM, W>), dim3(uint32_t(gx)), dim3(W * kWave), 0, s, p);
    return hipGetLastError();
}

// Whether a launch takes the row-stream kernel: Q4_K, plain (without the
// fused norm: no caller asks for it) or gate/up + SwiGLU, all of K (at most
// 14 super-blocks) in this launch, no split-K, no embedding decode or
// accumulation.  Automatic choice: plain GEMVs of 8192 rows or more, the
// shapes it measured faster on (MI355X, 18944 x 3584: 10.9 vs 11.7 us;
// 3584 x 3584: 5.6 vs 5.0 us, and the fused gate/up 20.0 vs 17.4 us).
inline bool rs_eligible(int epi, const GemvParams& p, uint32_t splits)
{
    if (!g_rowstream || (epi != EPI_PLAIN && epi != EPI_SWIGLU)) return false;
    if (splits != 1 || p.kb_off != 0 || p.panel != p.nb || p.split_bps != p.nb) return false;
    if (p.nb < 1 || p.nb > uint32_t(kRsMaxBlocks)) return false;
    if (p.flags & (F_EMBED | F_ACCUM | F_ARGNEXT)) return false;
    if (epi == EPI_PLAIN && (p.flags & F_NORM)) return false;
    if (g_rowstream < 0) return epi == EPI_PLAIN && p.rows >= 8192;
    return true;
}

inline hipError_t launch_rs_epi(int epi, const GemvParams& p, hipStream_t s, uint32_t* gx)
{
    if (epi == EPI_SWIGLU)
        return (p.flags & F_NORM) ? launch_rs<2, 1, EPI_SWIGLU, true, kRsWaves>(p, s, gx)
                                  : launch_rs<2, 1, EPI_SWIGLU, false, kRsWaves>(p, s, gx);
    return launch_rs<1, 1, EPI_PLAIN, false, kRsWaves>(p, s, gx);
}

// Forced configuration for tuning sweeps (bs = 0: automatic; waves = 0: automatic).
inline thread_local Cfg g_force{0, 0, 0};
inline thread_local int g_force_waves = 0;

// Q6_K layouts with 4 rows per lane (256 VGPRs plus spills into AGPRs) are
// not built: the 2-quad one took a GPU memory fault once, with no cause found
// in its source or its code.  An automatic choice of 4 rows per lane runs
// with 2 on Q6_K; a forced one is refused.
template <int FMT>
constexpr bool layout_built(int rpl)
{
    return !((FMT == kFmtQ6 || FMT == kFmtQ6P) && rpl == 4);
}

template <int FMT, int EPI>
hipError_t launch_cfg(Cfg c, const GemvParams& p, uint32_t splits, hipStream_t s, uint32_t* gx)
{
    if (!layout_built<FMT>(c.rpl)) {
        if (g_force.bs) return hipErrorInvalidValue;
        c.rpl = 2;
    }
#define ARC_CASE(B, R)                                                         \
    if constexpr (layout_built<FMT>(R))                                        \
        if (c.bs == B && c.rpl == R)                                           \
            return c.waves == 8 ? launch_one<FMT, EPI, B, R, 8>(p, splits, s, gx)  \
                                : launch_one<FMT, EPI, B, R, 4>(p, splits, s, gx);
    ARC_CASE(1, 1) ARC_CASE(1, 2) ARC_CASE(1, 4)
    ARC_CASE(2, 1) ARC_CASE(2, 2) ARC_CASE(2, 4)
    ARC_CASE(4, 1) ARC_CASE(4, 2)
    ARC_CASE(8, 1) ARC_CASE(8, 2)
    ARC_CASE(16, 1)
#undef ARC_CASE
    return hipErrorInvalidValue;
}

// Waves per workgroup.  A staged panel wider than 37 super-blocks (> 40 KB
// of LDS) caps residency at 2-3 workgroups per CU, so 8-wave workgroups
// share one staged x and double the resident waves (measured +8% on the
// 74-block FFN-down); the one-column split-K layout also gains from 8.  A
// plain GEMV of 2048+ rows stages x in half as many workgroups with 8
// (3584 x 3584 Q4_K: 4.74 vs 5.23 us); the fused gate/up and small GEMVs
// measured faster with 4.
inline int choose_waves(int epi, uint32_t rows, uint32_t blocks)
{
    if (g_force_waves) return g_force_waves;
    if (blocks > 37 || epi == EPI_COLPART) return 8;
    return (epi == EPI_PLAIN && rows >= 2048) ? 8 : kWaves;
}

// Automatic lane layout.  Work is balanced over ~2048 resident waves: a
// layout is preferred when its wave tiles divide evenly over them and its
// quads are busy (few idle block slots), then when it reuses x over more rows.
inline Cfg choose_cfg(int epi, uint32_t rows, uint32_t blocks, uint32_t splits)
{
    if (g_force.bs) return Cfg{g_force.bs, g_force.rpl, choose_waves(epi, rows, blocks)};
    // fused gate/up: 4 quads per row (4 rows per wave tile) measured 5% faster
    // than the 8 the balance score picks (Qwen2.5-7B shape, 17.8 vs 18.8 us)
    if (epi == EPI_SWIGLU && blocks <= 16) return Cfg{4, 1, choose_waves(epi, rows, blocks)};
    // LM head + argmax: 2 quads per row, one row per lane measured fastest of
    // every layout (Q6_K 152064 x 3584: 91.8 vs 99.6 us for the (2, 2) the
    // balance score picks)
    if (epi == EPI_ARGMAX && blocks <= 16) return Cfg{2, 1, choose_waves(epi, rows, blocks)};
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
    best.waves = choose_waves(epi, rows, blocks);
    return best;
}

template <int EPI>
hipError_t launch_gemv(int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s, uint32_t* gx)
{
    if constexpr (EPI == EPI_PLAIN || EPI == EPI_SWIGLU)
        if (qtype == kFmtQ4 && !g_force.bs && rs_eligible(EPI, p, splits)) return launch_rs_epi(EPI, p, s, gx);
    if (qtype == kFmtQ4) return launch_cfg<kFmtQ4, EPI>(c, p, splits, s, gx);
    if (qtype == kFmtQ6P) return launch_cfg<kFmtQ6P, EPI>(c, p, splits, s, gx);
    if (qtype == kFmtE148) {
        // EXEC148 is the down projection's representation: plain and split-K only
        if constexpr (EPI == EPI_PLAIN || EPI == EPI_PARTIAL || EPI == EPI_COLPART)
            return launch_cfg<kFmtE148, EPI>(c, p, splits, s, gx);
        return hipErrorInvalidValue;
    }
    return launch_cfg<kFmtQ6, EPI>(c, p, splits, s, gx);
}

inline hipError_t launch_gemv_epi(int epi, int qtype, const Cfg& c, const GemvParams& p, uint32_t splits, hipStream_t s,
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

static int block_bytes(int qtype)
{
    return qtype == kFmtQ4 ? kQ4Bytes : qtype == kFmtE148 ? kE148Bytes : qtype == kFmtQ6P ? kQ6PBytes : kQ6Bytes;
}

static int check_shape(int qtype, const void* w, uint32_t rows, uint32_t K)
{
    if (qtype != kFmtQ4 && qtype != kFmtQ6 && qtype != kFmtQ6P && qtype != kFmtE148)
        return set_error(ARC_ERR_UNSUPPORTED, "unsupported qtype %d", qtype);
    if (!w) return set_error(ARC_ERR_INVALID_ARGUMENT, "null weight pointer");
    if (rows == 0 || K == 0 || (K % kQK) != 0)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad shape rows=%u K=%u (K must be a nonzero multiple of 256)",
                         rows, K);
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if (qtype == kFmtQ4 && (a & 15u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "Q4_K tensor not 16-byte aligned");
    if (qtype == kFmtQ6 && (a & 1u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "Q6_K tensor not 2-byte aligned");
    if (qtype == kFmtQ6 && uint64_t(rows) * (K / kQK) * kQ6Bytes > 0xfffffff0ull)
        return set_error(ARC_ERR_UNSUPPORTED, "Q6_K tensor of %u x %u exceeds 4 GiB", rows, K);
    if (qtype == kFmtE148 && (a & 3u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "EXEC148 tensor not 4-byte aligned");
    if (qtype == kFmtQ6P && (a & 3u)) return set_error(ARC_ERR_INVALID_ARGUMENT, "padded Q6_K tensor not 4-byte aligned");
    if (qtype == kFmtQ6P && uint64_t(rows) * (K / kQK) * kQ6PBytes > 0xfffffff0ull)
        return set_error(ARC_ERR_UNSUPPORTED, "padded Q6_K tensor of %u x %u exceeds 4 GiB", rows, K);
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
        if (off + kPanel < p.split_bps) q.res = nullptr;  // the residual enters once, with the last panel
        const int rc = check_hip(launch_gemv_epi(epi, qtype, c, q, splits, s, gx), what);
        if (rc) return rc;
    }
    return ARC_OK;
}

}  // namespace arc
