// arc_prefill.hip -- the batched prompt pass on gfx950 MFMA (the reference's
// build_prefill, src/arcllm_v1_runtime.cpp:340-369, which runs dequant-in-LDS
// fp32 tiles).
//
// A prompt of M <= 256 tokens at positions pos0 .. pos0+M-1 is processed as
// matrices: per layer (8 launches)
//   [q|k|v] = X [Wq|Wk|Wv]^T  (split-K partials, one launch)   k_pf_gemm_qkv
//   + bias, RoPE on q and k, q -> fp32, k and v -> fp16 cache  k_pf_qkv_epi
//   causal GQA over the cache (positions <= own) -> X (fp16)    k_pf_attn
//   H += X Wo^T, X = RMSNorm(H) (ffn norm)                      k_pf_gemm, k_pf_res_norm
//   s = silu(X Wg^T) * (X Wu^T) -> fp16                         k_pf_gemm<SWIGLU>
//   H += s Wd^T, X = RMSNorm(H) (next layer's attention norm)   k_pf_gemm, k_pf_res_norm
// after the embedding and the first layer's attention norm (k_pf_embed,
// k_pf_rmsnorm), then the output RMSNorm + LM head + argmax on the last row
// only (the decode step's kernels), leaving the argmax as the next token.
//
// GEMM (pf_gemm_body): Y[m][n] = sum_k X[m][k] W[n][k] with
// v_mfma_f32_32x32x16_f16.  A workgroup owns all M rows (MB blocks of 32) and
// 128*NF weight rows (4 waves, NF rows per lane); X is staged through LDS in
// half-super-block tiles (double-buffered, rows padded by 8 halves so the
// 16-byte fragment reads are bank-conflict free); each lane dequantises its
// own B fragments (8 weights of one row per 16-wide K step) straight from the
// packed super-block into fp16 registers with the element decode's fp32
// arithmetic, software-pipelined against the MFMAs.  Operands are fp16,
// accumulation fp32.
#include "arc_session.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>

namespace arc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // native vector: stays in registers

constexpr int kPfKT = 128;         // K columns per LDS stage (half a super-block)
constexpr int kPfLd = kPfKT + 8;   // padded LDS row, in halves

// ------------------------------------------------------------------ GEMM
struct PfGemm {
    const uint8_t* w0;   // PLAIN: rows [0, ncol0); SWIGLU: gate
    const uint8_t* w1;   // PLAIN: rows [ncol0, N) (row index - ncol0); SWIGLU: up
    uint64_t row_bytes;
    uint32_t ncol0;
    uint32_t N;          // output columns
    uint32_t nb;         // super-blocks per weight row
    uint32_t bps;        // super-blocks per split (grid.y = splits)
    uint32_t M;          // valid rows
    uint32_t mpad;       // rows of the partial buffer per split
    const _Float16* x;   // [>= MB*32 rows][ldx]
    uint32_t ldx;
    float* out;          // PLAIN: [split][mpad][ldo], columns [0, N)
    uint32_t ldo;
    uint32_t tiles;      // column tiles (workgroups along x) of this operand
    _Float16* s;         // SWIGLU: [M][lds_out]
    uint32_t lds_out;
};

// K order inside a super-block.  The GEMM sums over K, so X and W only have
// to agree on which element each MFMA K slot holds.  Step t (0..7) of half
// block hb gives the lane of half kh (lane / 32) the 8 consecutive elements
// hb*128 + acol(t) + kh*16 .. +7, with acol(t) = (t/2)*32 + (t%2)*8, so one
// lane's elements for a whole super-block come from a few contiguous 16-byte
// pieces of the packed block:
//   Q4_K: qs bytes c*32 + kh*16 .. +15 of chunk c hold elements
//         c*64 + kh*16 + 0..15 (low nibbles) and c*64 + 32 + kh*16 + 0..15
//         (high nibbles); steps t = 4(c%2) + r take the low nibbles of bytes
//         0..7 (r=0) / 8..15 (r=1), the high nibbles of 0..7 (r=2) / 8..15 (r=3);
//   Q6_K: ql bytes h*64 + 32*(q%2) + kh*16 .. +15 and qh bytes
//         128 + h*32 + kh*16 .. +15 hold quarter q of half h, elements
//         h*128 + q*32 + kh*16 + 0..15; step t = 2q + u takes bytes 8u .. 8u+7.
__device__ __forceinline__ constexpr uint32_t acol(int t) { return uint32_t((t >> 1) * 32 + (t & 1) * 8); }

// The packed bytes of one super-block row that one lane consumes, loaded a
// super-block ahead of their use.
template <int FMT>
struct WRaw;
template <>
struct WRaw<kFmtQ4> {
    u32x4 hdr;    // d, dmin, 12 scale bytes
    u32x4 qs[4];  // qs chunk c, bytes kh*16 .. +15
};
template <>
struct WRaw<kFmtQ6> {
    u32x4 v[7];      // 16-byte pieces read from the dword floor: ql h*64 + {0,32} + kh*16 (h = 0, 1),
    uint32_t e[7];   // qh 128 + h*32 + kh*16, scales 192; e = the dword after each piece
    uint32_t d;      // bytes 208..209
    uint32_t sh;     // block address mod 4 (0 or 2: Q6_K blocks are 210 bytes)
};

// The same bytes ready for the element decode, with the per-step factors
// (codes are read as fp16 subnormals, q * 2^-24, so the factor carries
// 2^24): Q4_K f[j] = d*sc_j * 2^24 (odd j: 2^20, as those steps read 16*q),
// g[j] = -dmin*mn_j; Q6_K f[h*4 + q] = d*sc * 2^24 and n = -32*d*sc for
// sc = sc_{h*8 + 2q + kh}, this lane's 16-element sub-block of quarter q.
template <int FMT>
struct WDec;
template <>
struct WDec<kFmtQ4> {
    u32x4 qs[4];
    float f[8], g[8];
};
template <>
struct WDec<kFmtQ6> {
    u32x4 ql[4], qh[2];
    float f[8], n[8];
};
// Padded Q6_K (the model's Q6_K tensors): the same block bytes at a dword
// boundary, so load_w reads them with sh = 0; only the block stride differs.
template <>
struct WRaw<kFmtQ6P> : WRaw<kFmtQ6> {};
template <>
struct WDec<kFmtQ6P> : WDec<kFmtQ6> {};
template <int FMT>
constexpr int pf_block_bytes()
{
    return FMT == kFmtQ4 ? kQ4Bytes : FMT == kFmtQ6P ? kQ6PBytes : kQ6Bytes;
}

template <int FMT>
__device__ __forceinline__ void load_w(const uint8_t* blk, uint32_t kh, WRaw<FMT>& r)
{
    if constexpr (FMT == kFmtQ4) {
        r.hdr = *reinterpret_cast<const u32x4*>(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) r.qs[c] = *reinterpret_cast<const u32x4*>(blk + 16 + c * 32 + kh * 16);
    } else if constexpr (FMT == kFmtQ6P) {
        // padded block at a dword boundary: the pieces as they are
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            const uint32_t o = i < 4 ? uint32_t(i) * 32u + kh * 16u : i < 6 ? 128u + uint32_t(i - 4) * 32u + kh * 16u : 192u;
            r.v[i] = *reinterpret_cast<const u32x4a4*>(blk + o);
            r.e[i] = 0u;
        }
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
        r.sh = 0u;
    } else {
        // every dword read lies inside the 210-byte block: a piece at offset o
        // reads [o - sh, o - sh + 20) when sh = 2 and [o, o + 16) plus the
        // dword at o + 12 when sh = 0
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk)) & 3u;
        const uint8_t* b = blk - sh;
        const uint32_t eo = sh ? 16u : 12u;
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            const uint32_t o = i < 4 ? uint32_t(i) * 32u + kh * 16u : i < 6 ? 128u + uint32_t(i - 4) * 32u + kh * 16u : 192u;
            r.v[i] = *reinterpret_cast<const u32x4a4*>(b + o);
            r.e[i] = *reinterpret_cast<const uint32_t*>(b + o + eo);
        }
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
        r.sh = sh;
    }
}

template <int FMT>
__device__ __forceinline__ void decode_w(const WRaw<FMT>& r, uint32_t kh, WDec<FMT>& w)
{
#pragma clang fp contract(off)
    if constexpr (FMT == kFmtQ4) {
        const float d = f16_bits_to_f32(r.hdr.x), dmin = f16_bits_to_f32(r.hdr.x >> 16);
        const float d24 = d * 16777216.0f, d20 = d * 1048576.0f;  // exact
        const uint32_t b[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
        auto byte = [&](int i) { return (b[i >> 2] >> (8 * (i & 3))) & 0xffu; };
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            if (j < 4) {
                sc = byte(j) & 63u;
                mn = byte(j + 4) & 63u;
            } else {
                sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
                mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
            }
            w.f[j] = ((j & 1) ? d20 : d24) * float(sc);
            w.g[j] = -(dmin * float(mn));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) w.qs[c] = r.qs[c];
        (void)kh;
    } else {
        u32x4 al[7];
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            if constexpr (FMT == kFmtQ6P) {
                al[i] = r.v[i];
                continue;
            }
            al[i].x = __builtin_amdgcn_alignbyte(r.v[i].y, r.v[i].x, r.sh);
            al[i].y = __builtin_amdgcn_alignbyte(r.v[i].z, r.v[i].y, r.sh);
            al[i].z = __builtin_amdgcn_alignbyte(r.v[i].w, r.v[i].z, r.sh);
            al[i].w = __builtin_amdgcn_alignbyte(r.e[i], r.v[i].w, r.sh);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) w.ql[i] = al[i];
        w.qh[0] = al[4];
        w.qh[1] = al[5];
        const float d = f16_bits_to_f32(r.d);
        const uint32_t s = 8u * kh;
        const uint32_t sw[4] = {al[6].x >> s, al[6].y >> s, al[6].z >> s, al[6].w >> s};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const float f = d * float(int8_t(uint8_t(sw[h * 2 + (q >> 1)] >> (16 * (q & 1)))));
                w.f[h * 4 + q] = f * 16777216.0f;
                w.n[h * 4 + q] = f * -32.0f;
            }
    }
}

// Two codes held in the low bits of the fp16 halves of `pair` read as exact
// subnormals (bits c -> c * 2^-24); fmaf(code * 2^-24, A, n) with A the
// element factor times 2^24 is v_fma_mix.
__device__ __forceinline__ float mixc(uint32_t pair, bool hi, float A, float n)
{
    const half2_t h = __builtin_bit_cast(half2_t, pair);
    return __builtin_fmaf(static_cast<float>(hi ? h.y : h.x), A, n);
}

__device__ __forceinline__ float opaque_f(float v)
{
    asm("" : "+v"(v));
    return v;
}

// Four weights from the four bytes of `codes` (each code < 2^10, in the low
// bits of its byte or, for Q4_K high nibbles, times 16): bytes 0 and 2 are
// the halves of codes & 0x00ff00ff, bytes 1 and 3 moved down by v_perm_b32.
// Each weight is the element decode's fp32 value rounded to fp16.  Left to
// itself the compiler fuses the fp32 FMA and the fp16 conversion into one
// v_fma_mix{lo,hi}_f16, which rounds the exact d*sc*q - dmin*mn to fp16
// directly; for Q4_K that value can need more bits than fp32 holds, and
// where its fp32 rounding is an fp16 tie the two roundings differ by an fp16
// ulp.  ROUND32 keeps the fp32 value (the reference's weight) in a register
// first.  Q6_K's d*sc*(q-32) is exact in fp32, so the fused form is the same.
template <bool ROUND32>
__device__ __forceinline__ void mix4w(uint32_t codes, float A, float n, half8& o, int at)
{
    const uint32_t ev = opaque(codes & 0x00ff00ffu);
    const uint32_t od = opaque(__builtin_amdgcn_perm(0u, codes, 0x0c030c01u));  // [b1, 0, b3, 0]
    float w[4] = {mixc(ev, false, A, n), mixc(od, false, A, n), mixc(ev, true, A, n), mixc(od, true, A, n)};
#pragma unroll
    for (int i = 0; i < 4; ++i) o[at + i] = _Float16(ROUND32 ? opaque_f(w[i]) : w[i]);
}

// Step T of half HB: this lane's 8 weights as fp16, decoded in fp32 as one
// fused multiply-add per element on the code read as an fp16 subnormal:
// Q4_K fmaf(q * 2^-24, d*sc * 2^24, -dmin*mn) (high nibbles: 16q * 2^-24
// against d*sc * 2^20), Q6_K fmaf((q+32) * 2^-24, d*sc * 2^24, -32*d*sc)
// with q+32 the stored 6-bit code.  The scalings by powers of two are exact,
// and both equal the element decode's (d*sc)*q - dmin*mn and (d*sc)*(q-32)
// bit for bit: d has 11 significant bits, sc at most 6 (Q4_K) or 7 (Q6_K)
// and q at most 4 or 6, so the product is exact in fp32 and only the final
// add rounds.
template <int FMT, int HB, int T>
__device__ __forceinline__ half8 dequant_step(const WDec<FMT>& w)
{
    half8 o;
    if constexpr (FMT == kFmtQ4) {
        constexpr int c = HB * 2 + (T >> 2), r = T & 3, j = 2 * c + (r >> 1);
        constexpr uint32_t mask = r < 2 ? 0x0f0f0f0fu : 0xf0f0f0f0u;
        const float A = w.f[j], n = w.g[j];
        mix4w<true>(w.qs[c][(r & 1) * 2] & mask, A, n, o, 0);
        mix4w<true>(w.qs[c][(r & 1) * 2 + 1] & mask, A, n, o, 4);
    } else {
        constexpr int q = T >> 1, u = T & 1;
        constexpr uint32_t lsh = (q >> 1) * 4u, hsh = q * 2u;
        const u32x4& l = w.ql[HB * 2 + (q & 1)];
        const u32x4& hh = w.qh[HB];
        const uint32_t c0 = ((l[2 * u] >> lsh) & 0x0f0f0f0fu) | (((hh[2 * u] >> hsh) & 0x03030303u) << 4);
        const uint32_t c1 = ((l[2 * u + 1] >> lsh) & 0x0f0f0f0fu) | (((hh[2 * u + 1] >> hsh) & 0x03030303u) << 4);
        const float A = w.f[HB * 4 + q], n = w.n[HB * 4 + q];
        mix4w<false>(c0, A, n, o, 0);
        mix4w<false>(c1, A, n, o, 4);
    }
    return o;
}

// X staging of one LDS stage: K columns [k0, k0+128) of rows [0, MB*32),
// MB*32*16 pieces of 16 bytes, MB*2 per thread, moved in two parts of MB
// pieces (part P: pieces P*MB .. P*MB + MB-1 of each thread).  Piece i of a
// thread is row (tid/16) + 16*i, columns (tid%16)*8 .. +7: the global loads
// are buffer loads with the lane's byte offset `voff` and the uniform row and
// column offset in a scalar register; the LDS stores use one base and
// immediate offsets.
struct XSrc {
    __amdgpu_buffer_rsrc_t rsrc;  // X, MB*32 rows of ldx fp16
    uint32_t voff;                // ((tid/16)*ldx + (tid%16)*8) * 2
    uint32_t ldx;
};

template <int MB, int P>
__device__ __forceinline__ void x_fetch(const XSrc& xs, uint32_t k0, u32x4 (&reg)[MB])
{
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const uint32_t soff = (16u * uint32_t(P * MB + i) * xs.ldx + k0) * 2u;
        reg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xs.rsrc, xs.voff, soff, 0));
    }
}

template <int MB, int P>
__device__ __forceinline__ void x_store(_Float16* stage, const u32x4 (&reg)[MB])
{
    _Float16* base = stage + (P * MB * 16) * kPfLd + (threadIdx.x >> 4) * kPfLd + (threadIdx.x & 15u) * 8u;
#pragma unroll
    for (int i = 0; i < MB; ++i) *reinterpret_cast<u32x4*>(base + i * 16 * kPfLd) = reg[i];
}

template <int MB>
__device__ __forceinline__ void load_a(const _Float16* a, half8 (&f)[MB])
{
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) f[mb] = *reinterpret_cast<const half8*>(a + mb * 32 * kPfLd);
}

// Workgroup barrier ordering LDS only: global loads in flight (the next
// super-block's weights, the next X stage) stay in flight across it.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Per-lane state of the GEMM pipeline: NF B fragments (weight rows) per
// lane against MB A fragments (32-row blocks of X).
template <int FMT, int MB, int NF>
struct PfState {
    f32x16 acc[NF][MB];
    half8 af[MB];          // A fragments of the step being issued
    WDec<FMT> dec[NF];     // the current super-block, decoded
    WRaw<FMT> raw[NF];     // the next super-block, as loaded
};

// Step T of half HB.  The NF*MB MFMAs of this step (B fragments `bc`, A
// fragments in s.af) issue one A block at a time; right behind each block's
// MFMAs its A fragment for step T+1 is read from LDS into the same registers,
// and the B fragments of the next step are decoded into `bn` in between.  At
// T = 7 the next step is step 0 of the next half: half 1 of this super-block,
// or, once s.raw is decoded into s.dec, half 0 of the next super-block (its A
// fragments are read after the barrier).  The sched_group_barrier pattern
// keeps MFMA, LDS read and VALU interleaved so one wave per SIMD keeps the
// matrix pipe busy.
template <int FMT, int MB, int NF, int HB, int T>
__device__ __forceinline__ void pf_step(PfState<FMT, MB, NF>& s, const _Float16* a, uint32_t kh, const half8 (&bc)[NF],
                                        half8 (&bn)[NF])
{
    constexpr bool kNextSb = T == 7 && HB == 1;
    if constexpr (kNextSb) {
#pragma unroll
        for (int j = 0; j < NF; ++j) decode_w<FMT>(s.raw[j], kh, s.dec[j]);
    }
#pragma unroll
    for (int j = 0; j < NF; ++j) bn[j] = dequant_step<FMT, (T == 7 ? 1 - HB : HB), (T + 1) & 7>(s.dec[j]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int j = 0; j < NF; ++j)
            s.acc[j][mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(s.af[mb], bc[j], s.acc[j][mb], 0, 0, 0);
        if constexpr (T < 7) s.af[mb] = *reinterpret_cast<const half8*>(a + acol(T + 1) + mb * 32 * kPfLd);
    }
    constexpr int kValu = ((kNextSb ? 110 : 34) * NF + MB - 1) / MB;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, NF, 0);  // MFMA
        if constexpr (T < 7) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
}

// One half super-block of MFMAs from LDS stage `a`, while the other stage
// (not read during this half) is filled with K columns [xk0, xk0+128) of X
// in two parts.  Half 1 also issues the weight loads of the next super-block
// (after the first X part, so that waiting for X never waits for them); they
// are decoded in its last step.  b0 holds the B fragments of step 0 on entry
// and of the next half's step 0 on exit.
template <int FMT, int MB, int NF, int HB>
__device__ __forceinline__ void pf_half(const XSrc& p, PfState<FMT, MB, NF>& s, const _Float16* a, uint32_t xk0,
                                        _Float16* xdst, const uint8_t* const (&wnext)[NF], uint32_t kh,
                                        half8 (&b0)[NF], half8 (&b1)[NF])
{
    u32x4 xr[MB];
    x_fetch<MB, 0>(p, xk0, xr);
    if constexpr (HB == 1) {
#pragma unroll
        for (int j = 0; j < NF; ++j) load_w<FMT>(wnext[j], kh, s.raw[j]);
    }
    load_a<MB>(a, s.af);
    __builtin_amdgcn_sched_barrier(0);
    pf_step<FMT, MB, NF, HB, 0>(s, a, kh, b0, b1);
    pf_step<FMT, MB, NF, HB, 1>(s, a, kh, b1, b0);
    pf_step<FMT, MB, NF, HB, 2>(s, a, kh, b0, b1);
    pf_step<FMT, MB, NF, HB, 3>(s, a, kh, b1, b0);
    x_store<MB, 0>(xdst, xr);
    x_fetch<MB, 1>(p, xk0, xr);
    __builtin_amdgcn_sched_barrier(0);
    pf_step<FMT, MB, NF, HB, 4>(s, a, kh, b0, b1);
    pf_step<FMT, MB, NF, HB, 5>(s, a, kh, b1, b0);
    pf_step<FMT, MB, NF, HB, 6>(s, a, kh, b0, b1);
    pf_step<FMT, MB, NF, HB, 7>(s, a, kh, b1, b0);
    x_store<MB, 1>(xdst, xr);
}

// D[m][c]: register i of block mb holds row mb*32 + (i/4)*8 + (lane/32)*4 + i%4
__device__ __forceinline__ uint32_t acc_row(int mb, int i, int lane)
{
    return uint32_t(mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3));
}

// ------------------------------------------ gate/up + SwiGLU in 8 waves
// The fused gate/up GEMM with one weight row per lane (NF = 1): waves 0-3
// own the tile's 128 gate rows, waves 4-7 its 128 up rows.  A wave then
// needs half the accumulators of the NF = 2 layout, so two waves fit per
// SIMD and one wave's dequantisation overlaps the other's MFMAs; every
// weight is still dequantised once.  Each wave group stages one part of
// every X tile (threads t & 255 of group g move part g), and SwiGLU is
// joined through LDS at the end: the gate waves store silu(g) by
// (row, column), the up waves multiply.
// Pieces part*MB + sub*NP + i (i < NP, sub*NP + i < MB) of thread t & 255,
// NP = ceil(MB / 2): each group moves its part in two halves.
template <int MB>
constexpr int gu_np()
{
    return (MB + 1) / 2;
}

template <int MB>
__device__ __forceinline__ void x_fetch_part(const XSrc& xs, uint32_t k0, uint32_t part, int sub,
                                             u32x4 (&reg)[gu_np<MB>()])
{
    constexpr int NP = gu_np<MB>();
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        if (sub * NP + i >= MB) break;
        const uint32_t soff = (16u * (part * MB + uint32_t(sub * NP + i)) * xs.ldx + k0) * 2u;
        reg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xs.rsrc, xs.voff, soff, 0));
    }
}

template <int MB>
__device__ __forceinline__ void x_store_part(_Float16* stage, uint32_t part, int sub, const u32x4 (&reg)[gu_np<MB>()])
{
    constexpr int NP = gu_np<MB>();
    const uint32_t t = threadIdx.x & 255u;
    _Float16* base = stage + (part * MB * 16) * kPfLd + (t >> 4) * kPfLd + (t & 15u) * 8u;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        if (sub * NP + i >= MB) break;
        *reinterpret_cast<u32x4*>(base + (sub * NP + i) * 16 * kPfLd) = reg[i];
    }
}

template <int FMT, int MB, int HB>
__device__ __forceinline__ void pf_half_gu(const XSrc& p, PfState<FMT, MB, 1>& s, const _Float16* a, uint32_t xk0,
                                           _Float16* xdst, const uint8_t* const (&wnext)[1], uint32_t kh, uint32_t part,
                                           half8 (&b0)[1], half8 (&b1)[1])
{
    u32x4 xr[gu_np<MB>()];
    x_fetch_part<MB>(p, xk0, part, 0, xr);
    if constexpr (HB == 1) load_w<FMT>(wnext[0], kh, s.raw[0]);
    load_a<MB>(a, s.af);
    __builtin_amdgcn_sched_barrier(0);
    pf_step<FMT, MB, 1, HB, 0>(s, a, kh, b0, b1);
    pf_step<FMT, MB, 1, HB, 1>(s, a, kh, b1, b0);
    pf_step<FMT, MB, 1, HB, 2>(s, a, kh, b0, b1);
    pf_step<FMT, MB, 1, HB, 3>(s, a, kh, b1, b0);
    x_store_part<MB>(xdst, part, 0, xr);
    x_fetch_part<MB>(p, xk0, part, 1, xr);
    __builtin_amdgcn_sched_barrier(0);
    pf_step<FMT, MB, 1, HB, 4>(s, a, kh, b0, b1);
    pf_step<FMT, MB, 1, HB, 5>(s, a, kh, b1, b0);
    pf_step<FMT, MB, 1, HB, 6>(s, a, kh, b0, b1);
    pf_step<FMT, MB, 1, HB, 7>(s, a, kh, b1, b0);
    x_store_part<MB>(xdst, part, 1, xr);
}

template <int FMT, int MB>
__global__ __launch_bounds__(512, 1) void k_pf_gemm_gu(PfGemm p)
{
    extern __shared__ __align__(16) _Float16 ash[];  // [2][MB*32][kPfLd]
    constexpr int kStage = MB * 32 * kPfLd;
    constexpr int kBB = pf_block_bytes<FMT>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t part = uint32_t(wave) >> 2, kh = uint32_t(lane) >> 5;
    const uint32_t c = uint32_t(wave & 3) * 32 + uint32_t(lane & 31);  // column within the tile
    const uint32_t col = blockIdx.x * 128 + c;
    const uint8_t* wrow = (part == 0 ? p.w0 : p.w1) + uint64_t(min(col, p.N - 1)) * p.row_bytes;

    PfState<FMT, MB, 1> s;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s.acc[0][mb][i] = 0.0f;

    XSrc xs;
    xs.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(p.x), (short)0, int(MB * 32 * p.ldx * 2u),
                                                0x00020000);
    const uint32_t t = uint32_t(tid) & 255u;
    xs.voff = ((t >> 4) * p.ldx + (t & 15u) * 8u) * 2u;
    xs.ldx = p.ldx;

    // prologue: weights of super-block 0, stage 0 = half 0 of super-block 0
    load_w<FMT>(wrow, kh, s.raw[0]);
    {
        u32x4 xr[gu_np<MB>()];
        x_fetch_part<MB>(xs, 0, part, 0, xr);
        x_store_part<MB>(ash, part, 0, xr);
        x_fetch_part<MB>(xs, 0, part, 1, xr);
        x_store_part<MB>(ash, part, 1, xr);
    }
    half8 b0[1], b1[1];
    decode_w<FMT>(s.raw[0], kh, s.dec[0]);
    b0[0] = dequant_step<FMT, 0, 0>(s.dec[0]);
    lds_barrier();
    const uint32_t ao = (lane & 31) * kPfLd + kh * 16;
    const _Float16* a0 = ash + ao;
    const _Float16* a1 = ash + opaque(ao + kStage);
    for (uint32_t kb = 0; kb < p.nb; ++kb) {
        const uint32_t kn = kb + 1 < p.nb ? kb + 1 : kb;  // the last super-block re-loads and re-stages itself
        const uint8_t* wn[1] = {wrow + uint64_t(kn) * kBB};
        pf_half_gu<FMT, MB, 0>(xs, s, a0, kb * kQK + kPfKT, ash + kStage, wn, kh, part, b0, b1);
        lds_barrier();
        pf_half_gu<FMT, MB, 1>(xs, s, a1, kn * kQK, ash, wn, kh, part, b0, b1);
        lds_barrier();
    }

    // SwiGLU across the wave groups: silu(gate) by (row, column) in the free stages
    float* sg = reinterpret_cast<float*>(ash);  // [MB*32][128]
    if (part == 0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float g = s.acc[0][mb][i];
                sg[acc_row(mb, i, lane) * 128 + c] = g / (1.0f + expf(-g));
            }
    }
    __syncthreads();
    if (part == 1 && col < p.N) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t m = acc_row(mb, i, lane);
                if (m < p.M) p.s[uint64_t(m) * p.lds_out + col] = _Float16(sg[m * 128 + c] * s.acc[0][mb][i]);
            }
    }
}

// Y = X W^T over super-blocks [kb0, kb1) of K for MB*32 rows of X.
// Workgroup: 4 waves, one per SIMD; lane (l%32) of wave w owns weight row(s)
//   SWIGLU (NF = 2): gate and up row c = tile*128 + w*32 + l%32, and
//                    writes s[m][c] = silu(X Wg^T)[m][c] * (X Wu^T)[m][c];
//   PLAIN:           rows c_j = tile*128*NF + w*32*NF + j*32 + l%32
//                    (row c < ncol0 from w0, else row c - ncol0 of w1), and
//                    writes split partials out[blockIdx.y][m][c] (row stride ldo).
// X is staged in LDS half a super-block (128 K columns) at a time, double-
// buffered; the weights of super-block kb+1 are loaded during kb.
template <int FMT, int MB, int NF, bool SWIGLU>
__device__ __forceinline__ void pf_gemm_body(const PfGemm& p, uint32_t tile)
{
    static_assert(!SWIGLU || NF == 2, "SwiGLU pairs a gate and an up row per lane");
    extern __shared__ __align__(16) _Float16 ash[];  // [2][MB*32][kPfLd]
    constexpr int kStage = MB * 32 * kPfLd;
    constexpr int kBB = pf_block_bytes<FMT>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kh = uint32_t(lane) >> 5;

    uint32_t col[NF];
    const uint8_t* wrow[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        if constexpr (SWIGLU) {
            col[j] = tile * 128 + wave * 32 + (lane & 31);
            wrow[j] = (j == 0 ? p.w0 : p.w1) + uint64_t(min(col[j], p.N - 1)) * p.row_bytes;
        } else {
            col[j] = tile * (128 * NF) + wave * (32 * NF) + j * 32 + (lane & 31);
            const uint32_t r = min(col[j], p.N - 1);
            wrow[j] = r < p.ncol0 ? p.w0 + uint64_t(r) * p.row_bytes : p.w1 + uint64_t(r - p.ncol0) * p.row_bytes;
        }
    }
    const uint32_t kb0 = blockIdx.y * p.bps, kb1 = min(p.nb, kb0 + p.bps);

    PfState<FMT, MB, NF> s;
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) s.acc[j][mb][i] = 0.0f;

    XSrc xs;
    xs.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(p.x), (short)0, int(MB * 32 * p.ldx * 2u),
                                                0x00020000);
    xs.voff = ((uint32_t(tid) >> 4) * p.ldx + (uint32_t(tid) & 15u) * 8u) * 2u;
    xs.ldx = p.ldx;

    // prologue: weights of kb0, stage 0 = half 0 of kb0
#pragma unroll
    for (int j = 0; j < NF; ++j) load_w<FMT>(wrow[j] + uint64_t(kb0) * kBB, kh, s.raw[j]);
    {
        u32x4 xr[MB];
        x_fetch<MB, 0>(xs, kb0 * kQK, xr);
        x_store<MB, 0>(ash, xr);
        x_fetch<MB, 1>(xs, kb0 * kQK, xr);
        x_store<MB, 1>(ash, xr);
    }
    half8 b0[NF], b1[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        decode_w<FMT>(s.raw[j], kh, s.dec[j]);
        b0[j] = dequant_step<FMT, 0, 0>(s.dec[j]);
    }
    lds_barrier();
    // stage 1's A base is a separate register (its offsets from stage 0 exceed
    // the 16-bit LDS immediate)
    const uint32_t ao = (lane & 31) * kPfLd + kh * 16;
    const _Float16* a0 = ash + ao;
    const _Float16* a1 = ash + opaque(ao + kStage);
    for (uint32_t kb = kb0; kb < kb1; ++kb) {
        // the last super-block of the range re-loads and re-stages itself
        const uint32_t kn = kb + 1 < kb1 ? kb + 1 : kb;
        const uint8_t* wn[NF];
#pragma unroll
        for (int j = 0; j < NF; ++j) wn[j] = wrow[j] + uint64_t(kn) * kBB;
        pf_half<FMT, MB, NF, 0>(xs, s, a0, kb * kQK + kPfKT, ash + kStage, wn, kh, b0, b1);
        lds_barrier();
        pf_half<FMT, MB, NF, 1>(xs, s, a1, kn * kQK, ash, wn, kh, b0, b1);
        lds_barrier();
    }

    // D[m][c]: register i of block mb holds row mb*32 + (i/4)*8 + (lane/32)*4 + i%4
    if constexpr (SWIGLU) {
        if (col[0] < p.N) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t m = mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                    if (m < p.M) {
                        const float g = s.acc[0][mb][i], u = s.acc[1][mb][i];
                        p.s[uint64_t(m) * p.lds_out + col[0]] = _Float16((g / (1.0f + expf(-g))) * u);
                    }
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            if (col[j] >= p.N) continue;
            float* o = p.out + uint64_t(blockIdx.y) * p.mpad * p.ldo + col[j];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t m = mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                    if (m < p.M) o[uint64_t(m) * p.ldo] = s.acc[j][mb][i];
                }
        }
    }
}

template <int FMT, int MB, int NF, bool SWIGLU>
__global__ __launch_bounds__(256, 1) void k_pf_gemm(PfGemm p)
{
    pf_gemm_body<FMT, MB, NF, SWIGLU>(p, blockIdx.x);
}

// The q|k (Q4_K) and v (format VF) projections of one layer in one launch:
// tiles [0, qk.tiles) are q|k, the rest v; both write split partials into
// one [split][mpad][hidden + 2*kv_dim] buffer (v after q|k).
template <int MB, int VF>
__global__ __launch_bounds__(256, 1) void k_pf_gemm_qkv(PfGemm qk, PfGemm v)
{
    if (blockIdx.x < qk.tiles)
        pf_gemm_body<kFmtQ4, MB, 1, false>(qk, blockIdx.x);
    else
        pf_gemm_body<VF, MB, 1, false>(v, blockIdx.x - qk.tiles);
}

// --------------------------------------------------------- small kernels
// H[m] = dequant(token_embd[tokens[m]]); grid (nb, M), element formula of
// the decode embedding.
__global__ __launch_bounds__(256) void k_pf_embed(const uint8_t* __restrict__ emb, uint32_t nb,
                                                  const uint32_t* __restrict__ tokens, float* __restrict__ h)
{
#pragma clang fp contract(off)
    const uint32_t m = blockIdx.y, e = blockIdx.x * kQK + threadIdx.x;
    const uint8_t* b = emb + (uint64_t(tokens[m]) * nb + blockIdx.x) * kQ4Bytes;
    const uint32_t k = threadIdx.x, j = k >> 5;
    const float d = f16_bits_to_f32(uint32_t(b[0]) | (uint32_t(b[1]) << 8));
    const float dm = f16_bits_to_f32(uint32_t(b[2]) | (uint32_t(b[3]) << 8));
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
    h[uint64_t(m) * nb * kQK + e] = t1 - t2;
}

// X[m] = fp16((H[m] * inv) * w), inv = 1/sqrt(mean(H[m]^2) + eps); grid M.
__global__ __launch_bounds__(256) void k_pf_rmsnorm(const float* __restrict__ h, uint32_t n, const float* __restrict__ w,
                                                    float eps, _Float16* __restrict__ x, uint32_t ldx)
{
    __shared__ float red[4];
    const float* r = h + uint64_t(blockIdx.x) * n;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) ss = __builtin_fmaf(r[i], r[i], ss);
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(n) + eps);
    _Float16* o = x + uint64_t(blockIdx.x) * ldx;
    for (uint32_t i = threadIdx.x; i < n; i += 256) o[i] = _Float16((r[i] * inv) * w[i]);
}

// q|k|v epilogue, per (m, column pair) of the [hidden | kv_dim | kv_dim]
// partials: fixed-order sum over the splits + bias; q and k pairs are
// rotated (RoPE at position pos0 + m), q -> fp32, k and v -> fp16 cache row
// pos0 + m.
__global__ __launch_bounds__(256) void k_pf_qkv_epi(const float* __restrict__ part, uint32_t splits, uint32_t mpad,
                                                    uint32_t hidden, uint32_t kv_dim, const float* __restrict__ qb,
                                                    const float* __restrict__ kb, const float* __restrict__ vb,
                                                    const float2* __restrict__ rope, uint32_t pos0,
                                                    float* __restrict__ q, _Float16* __restrict__ kc,
                                                    _Float16* __restrict__ vc)
{
    const uint32_t N = hidden + 2 * kv_dim, m = blockIdx.y;
    const uint32_t c = 2 * (blockIdx.x * 256 + threadIdx.x);
    if (c >= N) return;
    float a = 0.0f, b = 0.0f;
    for (uint32_t s0 = 0; s0 < splits; s0 += 8) {  // 8 splits' loads in flight, added in split order
        float2 v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            v[u] = s0 + u < splits ? *reinterpret_cast<const float2*>(part + (uint64_t(s0 + u) * mpad + m) * N + c)
                                   : float2{0.0f, 0.0f};
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (s0 + u < splits) {
                a += v[u].x;
                b += v[u].y;
            }
    }
    if (c >= hidden + kv_dim) {
        const uint32_t lc = c - hidden - kv_dim;
        _Float16* dst = vc + uint64_t(pos0 + m) * kv_dim + lc;
        dst[0] = _Float16(a + vb[lc]);
        dst[1] = _Float16(b + vb[lc + 1]);
        return;
    }
    const bool isq = c < hidden;
    const uint32_t lc = isq ? c : c - hidden;
    const float* bias = isq ? qb : kb;
    a = a + bias[lc];
    b = b + bias[lc + 1];
    const float2 cs = rope[uint64_t(pos0 + m) * 64 + ((lc & 127u) >> 1)];
    const float ra = a * cs.x - b * cs.y, rb = a * cs.y + b * cs.x;
    if (isq) {
        q[uint64_t(m) * hidden + lc] = ra;
        q[uint64_t(m) * hidden + lc + 1] = rb;
    } else {
        _Float16* dst = kc + uint64_t(pos0 + m) * kv_dim + lc;
        dst[0] = _Float16(ra);
        dst[1] = _Float16(rb);
    }
}

// Fixed-order second pass of a split-K projection with the residual and
// (NORM) the next RMSNorm: H[m][c] += sum_s part[s][m][c] (s in order), X[m] =
// fp16((H[m] * inv) * w), inv = 1/sqrt(mean(H[m]^2) + eps).  Grid M, one row
// per workgroup of 1024 threads; thread t owns columns t + 1024*k (k < KC,
// n <= 1024*KC), and loads the partials of 8 splits at a time, all in flight,
// before adding them in split order.
constexpr int kResCols = 20;  // n <= 20480, the model limit on hidden
template <bool NORM, int KC>
__global__ __launch_bounds__(1024) void k_pf_res_norm(const float* __restrict__ part, uint32_t splits, uint32_t mpad,
                                                      uint32_t n, float* __restrict__ h, const float* __restrict__ w,
                                                      float eps, _Float16* __restrict__ x, uint32_t ldx)
{
    static_assert(KC >= 1 && KC <= kResCols, "columns per thread");
    constexpr uint32_t kBatch = 8;
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, t = threadIdx.x;
    float* r = h + uint64_t(m) * n;
    const float* pm = part + uint64_t(m) * n;
    const uint64_t sstride = uint64_t(mpad) * n;
    float a[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) a[k] = 0.0f;
    for (uint32_t s0 = 0; s0 < splits; s0 += kBatch) {
        float v[kBatch][KC];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
#pragma unroll
            for (int k = 0; k < KC; ++k) {
                const uint32_t c = t + 1024u * k;
                v[u][k] = (s0 + u < splits && c < n) ? pm[(s0 + u) * sstride + c] : 0.0f;
            }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
#pragma unroll
            for (int k = 0; k < KC; ++k)
                if (s0 + u < splits) a[k] += v[u][k];
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
        const uint32_t c = t + 1024u * k;
        if (c < n) {
            a[k] = r[c] + a[k];
            r[c] = a[k];
            if constexpr (NORM) ss = __builtin_fmaf(a[k], a[k], ss);
        }
    }
    if constexpr (NORM) {
        ss = block_sum<1024>(ss, red);
        const float inv = 1.0f / sqrtf(ss / float(n) + eps);
        _Float16* o = x + uint64_t(m) * ldx;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            const uint32_t c = t + 1024u * k;
            if (c < n) o[c] = _Float16((a[k] * inv) * w[c]);
        }
    }
}

template <bool NORM>
void launch_res_norm(uint32_t M, hipStream_t st, const float* part, uint32_t splits, uint32_t mpad, uint32_t n,
                     float* h, const float* w, float eps, _Float16* x, uint32_t ldx)
{
    const uint32_t kc = (n + 1023u) / 1024u;
    if (kc <= 4)
        hipLaunchKernelGGL((k_pf_res_norm<NORM, 4>), dim3(M), dim3(1024), 0, st, part, splits, mpad, n, h, w, eps, x, ldx);
    else if (kc <= 8)
        hipLaunchKernelGGL((k_pf_res_norm<NORM, 8>), dim3(M), dim3(1024), 0, st, part, splits, mpad, n, h, w, eps, x, ldx);
    else
        hipLaunchKernelGGL((k_pf_res_norm<NORM, kResCols>), dim3(M), dim3(1024), 0, st, part, splits, mpad, n, h, w, eps,
                           x, ldx);
}

// Causal GQA for query row m (position pos0 + m) and kv head g: the HPK q
// heads of g attend to cache positions 0 .. pos0 + m in chunks of 64 with an
// online softmax (running max and sum, rescaled per chunk); output fp16 into
// the GEMM input X[m][head*128 + d].
template <int HPK>
__global__ __launch_bounds__(256) void k_pf_attn(const float* __restrict__ q, const _Float16* __restrict__ kc,
                                                 const _Float16* __restrict__ vc, uint32_t kv_heads, uint32_t pos0,
                                                 float scale, _Float16* __restrict__ x, uint32_t ldx)
{
    const uint32_t m = blockIdx.x, g = blockIdx.y, kvd = kv_heads * kHeadDim;
    const uint32_t hidden = kv_heads * HPK * kHeadDim;
    const uint32_t T = pos0 + m + 1;
    const int tid = threadIdx.x;
    __shared__ float qs[HPK][kHeadDim];
    __shared__ float sc[HPK][kChunk];
    __shared__ float alpha[HPK], lsum[HPK], mrun[HPK];
    __shared__ float ored[4][HPK][kHeadDim];
    for (uint32_t i = tid; i < HPK * kHeadDim; i += 256)
        qs[i >> 7][i & 127u] = q[uint64_t(m) * hidden + g * HPK * kHeadDim + i];
    if (tid < HPK) {
        mrun[tid] = -INFINITY;
        lsum[tid] = 0.0f;
    }
    const uint32_t tk = uint32_t(tid) >> 2, part = tid & 3;
    const int vi = tid & 63, pg = tid >> 6;
    float o[HPK][2];
#pragma unroll
    for (int h = 0; h < HPK; ++h) o[h][0] = o[h][1] = 0.0f;
    __syncthreads();
    for (uint32_t t0 = 0; t0 < T; t0 += kChunk) {
        const uint32_t nt = min(uint32_t(kChunk), T - t0);
        // every K and V load of the chunk is issued here, so the chunk costs
        // one memory round trip
        uint4 kraw[4];
        half2_t vraw[16];
        {
            const uint4* kp = reinterpret_cast<const uint4*>(kc + uint64_t(t0 + min(tk, nt - 1)) * kvd + g * kHeadDim +
                                                             part * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) kraw[i] = kp[i];
            const _Float16* vb = vc + uint64_t(t0) * kvd + g * kHeadDim + 2 * vi;
#pragma unroll
            for (int tt = 0; tt < 16; ++tt)
                vraw[tt] = *reinterpret_cast<const half2_t*>(vb + uint64_t(min(uint32_t(pg * 16 + tt), nt - 1)) * kvd);
        }
        {   // scores of positions t0 + tk
            float s[HPK];
#pragma unroll
            for (int h = 0; h < HPK; ++h) s[h] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 raw = kraw[i];
                const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float kv = static_cast<float>(__builtin_bit_cast(half2_t, w4[e >> 1])[e & 1]);
                    const int d = part * 32 + i * 8 + e;
#pragma unroll
                    for (int h = 0; h < HPK; ++h) s[h] = __builtin_fmaf(qs[h][d], kv, s[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < HPK; ++h) s[h] = group_sum<4>(s[h]);
            if (part == 0 && tk < nt)
#pragma unroll
                for (int h = 0; h < HPK; ++h) sc[h][tk] = s[h] * scale;
        }
        __syncthreads();
        {   // online softmax update: wave w handles heads w, w+4
            const int w = tid >> 6, lane = tid & 63;
            for (int h = w; h < HPK; h += 4) {
                const float sv = uint32_t(lane) < nt ? sc[h][lane] : -INFINITY;
                const float cm = wave_max(sv);
                const float mnew = fmaxf(mrun[h], cm);
                const float e = uint32_t(lane) < nt ? expf(sv - mnew) : 0.0f;
                const float l = group_sum<kWave>(e);
                sc[h][lane] = e;
                if (lane == 0) {
                    const float a = expf(mrun[h] - mnew);  // 0 on the first chunk
                    alpha[h] = a;
                    lsum[h] = lsum[h] * a + l;
                    mrun[h] = mnew;
                }
            }
        }
        __syncthreads();
        {   // o = o * alpha + sum_t p_t v_t over this chunk
#pragma unroll
            for (int h = 0; h < HPK; ++h) {
                o[h][0] *= alpha[h];
                o[h][1] *= alpha[h];
            }
#pragma unroll
            for (int tt = 0; tt < 16; ++tt) {
                const uint32_t t = pg * 16 + tt;
                const bool in = t < nt;
                const half2_t vv = vraw[tt];
                const float v0 = in ? static_cast<float>(vv.x) : 0.0f, v1 = in ? static_cast<float>(vv.y) : 0.0f;
#pragma unroll
                for (int h = 0; h < HPK; ++h) {
                    const float pr = sc[h][t];
                    o[h][0] = __builtin_fmaf(pr, v0, o[h][0]);
                    o[h][1] = __builtin_fmaf(pr, v1, o[h][1]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < HPK; ++h) {
        ored[pg][h][2 * vi] = o[h][0];
        ored[pg][h][2 * vi + 1] = o[h][1];
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < HPK * kHeadDim; idx += 256) {
        const uint32_t h = idx >> 7, d = idx & 127u;
        const float v = ((ored[0][h][d] + ored[1][h][d]) + ored[2][h][d]) + ored[3][h][d];
        x[uint64_t(m) * ldx + (g * HPK + h) * kHeadDim + d] = _Float16(v / lsum[h]);
    }
}

// Causal GQA of the prompt pass on MFMA.  Workgroup (query block b of 32
// rows, q head hq of kv head hq / hpk): 4 waves; wave w takes the
// 64-position key chunks w, w + 4, ... of positions 0 .. the block's last,
// with its own online softmax per query; at the end the waves' states are
// combined through LDS in wave order.
//  scores  S^T = K Q^T per 32-key tile on v_mfma_f32_32x32x16_f16: A = K
//          rows straight from the cache (lane -> key lane%32; step s: dims
//          16s + 8(lane/32) .. +7, 16 bytes of the row), B = Q^T (lane ->
//          query lane%32, the same dims) as fp16 hi + lo parts (q = hi + lo
//          to 2^-22 relative; K*hi and K*lo are exact products).  D: lane ->
//          query lane%32, value i -> key 8(i/4) + 4(lane/32) + i%4.
//  softmax the chunk maximum of a query from the lane's 32 scores and its
//          partner half-wave's (lane ^ 32); positions past the query's own
//          are masked.  Weights e^(x - max), rescaling the running sum and
//          the output by e^(max_old - max_new).
//  values  O^T = V^T P^T: B = P^T straight from the lane's weights (step s of
//          a tile: values 8s .. 8s+7, keys 16s + 8(j/4) + 4(lane/32) + j%4)
//          as fp16 hi + lo; A = V^T from LDS, where the wave stages its chunk
//          transposed with key k at column k with bits 2 and 3 swapped, so a
//          lane's 8 keys of a step are 16 contiguous bytes.  D: lane ->
//          query lane%32, value i of dim tile t -> dim 32t + 8(i/4) +
//          4(lane/32) + i%4.
// Semantics as k_pf_attn (src/arcllm_v1_runtime.cpp:340-369 per row).
constexpr int kVtLd = kChunk + 8;  // halves per V^T row in LDS (padded)

__device__ __forceinline__ uint32_t swap_bits_2_3(uint32_t k)
{
    return (k & ~12u) | ((k & 4u) << 1) | ((k & 8u) >> 1);
}

__global__ __launch_bounds__(256, 2) void k_pf_attn_mf(const float* __restrict__ q, const _Float16* __restrict__ kc,
                                                       const _Float16* __restrict__ vc, uint32_t kv_heads,
                                                       uint32_t hpk, uint32_t pos0, uint32_t M, uint32_t max_ctx,
                                                       float scale, _Float16* __restrict__ x, uint32_t ldx)
{
    __shared__ __align__(16) _Float16 vt[4][kHeadDim][kVtLd];  // per wave: its chunk's V^T; then the outputs
    __shared__ float mw[4][32], lw[4][32];
    const uint32_t b = blockIdx.x, hq = blockIdx.y, g = hq / hpk;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l32 = lane & 31, h2 = lane >> 5;
    const uint32_t kvd = kv_heads * kHeadDim, hidden = kv_heads * hpk * kHeadDim;
    const uint32_t q0 = b * 32, qlast = min(q0 + 31, M - 1);
    const uint32_t qpos = pos0 + q0 + uint32_t(l32);  // this lane's query position
    const uint32_t nkc = (pos0 + qlast + kChunk) / kChunk;  // chunks holding positions 0 .. pos0 + qlast

    half8 qh[8], ql[8];  // B operand of the scores: query l32, dims 16s + 8 h2 .. +7
    {
        const float* qp = q + uint64_t(min(q0 + uint32_t(l32), M - 1)) * hidden + hq * kHeadDim + 8 * h2;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const float4 a = *reinterpret_cast<const float4*>(qp + 16 * st);
            const float4 c = *reinterpret_cast<const float4*>(qp + 16 * st + 4);
            const float f[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const _Float16 hi = static_cast<_Float16>(f[j]);
                qh[st][j] = hi;
                ql[st][j] = static_cast<_Float16>(f[j] - static_cast<float>(hi));
            }
        }
    }
    f32x16 o[4];  // O^T: dim tile t, query l32
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.0f;
    float mrun = -INFINITY, lrun = 0.0f;  // lrun: this half-wave's share
    _Float16(*vw)[kVtLd] = vt[w];

    for (uint32_t c = uint32_t(w); c < nkc; c += 4) {
        const uint32_t kbase = c * kChunk;
        // this chunk's V rows (lane -> key kbase + lane), 16 bytes at a time,
        // and both tiles' K fragments, all issued before any is used
        uint4 vr[16];
        {
            const uint4* vp = reinterpret_cast<const uint4*>(vc + uint64_t(min(kbase + uint32_t(lane), max_ctx - 1)) * kvd +
                                                             g * kHeadDim);
#pragma unroll
            for (int e = 0; e < 16; ++e) vr[e] = vp[e];
        }
        uint4 kf[2][8];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const uint4* kp = reinterpret_cast<const uint4*>(
                kc + uint64_t(min(kbase + 32u * kt + uint32_t(l32), max_ctx - 1)) * kvd + g * kHeadDim + 8 * h2);
#pragma unroll
            for (int st = 0; st < 8; ++st) kf[kt][st] = kp[2 * st];
        }
        // scores of the two 32-key tiles
        f32x16 sc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[kt][i] = 0.0f;
#pragma unroll
            for (int st = 0; st < 8; ++st) {
                const half8 kfr = __builtin_bit_cast(half8, kf[kt][st]);
                sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr, qh[st], sc[kt], 0, 0, 0);
                sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr, ql[st], sc[kt], 0, 0, 0);
            }
        }
        // V^T of the chunk into the wave's LDS rows (key k -> column swap_bits_2_3(k))
        {
            const uint32_t col = swap_bits_2_3(uint32_t(lane));
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const half8 v8 = __builtin_bit_cast(half8, vr[e]);
#pragma unroll
                for (int j = 0; j < 8; ++j) vw[8 * e + j][col] = v8[j];
            }
        }
        // masked, scaled scores; the chunk maximum per query
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t kpos = kbase + 32u * kt + 8u * (i >> 2) + 4u * h2 + (i & 3);
                const float v = kpos <= qpos ? sc[kt][i] * scale : -INFINITY;
                sc[kt][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = xor_max<32>(mx);
        const float mnew = fmaxf(mrun, mx);
        const float mr = mnew == -INFINITY ? 0.0f : mnew;  // no position <= the query's yet: all weights 0
        const float alpha = expf(mrun - mr);              // mrun = -inf: 0
        float es = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = expf(sc[kt][i] - mr);
                sc[kt][i] = e;
                es += e;
            }
        lrun = lrun * alpha + es;
        mrun = mnew;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[t][i] *= alpha;
        // the wave's own V^T rows: its LDS writes above complete before these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                half8 ph, pl;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float pv = sc[kt][8 * st + j];
                    const _Float16 hi = static_cast<_Float16>(pv);
                    ph[j] = hi;
                    pl[j] = static_cast<_Float16>(pv - static_cast<float>(hi));
                }
                const uint32_t k0 = 32u * kt + 16u * st + 8u * h2;  // the lane's 8 keys, contiguous in LDS
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const half8 va = *reinterpret_cast<const half8*>(&vw[32 * t + l32][k0]);
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[t], 0, 0, 0);
                }
            }
        // the next chunk's V^T overwrites these rows
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // the waves' states, combined in wave order: M = max m_w, f_w = e^(m_w - M),
    // out = sum_w f_w o_w / sum_w f_w l_w (waves without a chunk: m = -inf, f = 0)
    const float ltot = xor_sum<32>(lrun);
    __syncthreads();  // every wave is done with its V^T rows
    float* ot = reinterpret_cast<float*>(&vt[0][0][0]);  // [4][128 dims][32 queries]
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t d = 32u * t + 8u * (i >> 2) + 4u * h2 + (i & 3);
            ot[(w * kHeadDim + d) * 32 + l32] = o[t][i];
        }
    if (h2 == 0) {
        mw[w][l32] = mrun;
        lw[w][l32] = ltot;
    }
    __syncthreads();
    const uint32_t qq = uint32_t(tid) & 31u, d0 = (uint32_t(tid) >> 5) * 16u;
    float Mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) Mx = fmaxf(Mx, mw[v][qq]);  // finite: chunk 0 holds position 0 <= every query's
    float f[4], L = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        f[v] = expf(mw[v][qq] - Mx);
        L = __builtin_fmaf(lw[v][qq], f[v], L);
    }
    const float li = 1.0f / L;
    if (q0 + qq < M) {
        _Float16* dst = x + uint64_t(q0 + qq) * ldx + hq * kHeadDim + d0;
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            float acc = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) acc = __builtin_fmaf(ot[(v * kHeadDim + d0 + d) * 32 + qq], f[v], acc);
            dst[d] = _Float16(acc * li);
        }
    }
}

// ------------------------------------------------------------------ host
namespace {

constexpr uint32_t kPfTargetWgs = 256;
thread_local int g_pf_attn_mfma = 1;  // 0: the VALU attention kernel (k_pf_attn)

template <int FMT, int MB, int NF, bool SW>
hipError_t launch_gemm_t(const PfGemm& p, uint32_t gx, uint32_t splits, hipStream_t st)
{
    const size_t lds = size_t(2) * MB * 32 * kPfLd * sizeof(_Float16);
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm<FMT, MB, NF, SW>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((k_pf_gemm<FMT, MB, NF, SW>), dim3(gx, splits), dim3(256), lds, st, p);
    return hipGetLastError();
}

template <int MB>
hipError_t launch_gu_t(const PfGemm& p, uint32_t gx, hipStream_t st)
{
    const size_t lds = size_t(2) * MB * 32 * kPfLd * sizeof(_Float16);
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm_gu<kFmtQ4, MB>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((k_pf_gemm_gu<kFmtQ4, MB>), dim3(gx), dim3(512), lds, st, p);
    return hipGetLastError();
}

hipError_t launch_gateup(const PfGemm& p, uint32_t mb, uint32_t gx, hipStream_t st)
{
    switch (mb) {
    case 1: return launch_gu_t<1>(p, gx, st);
    case 2: return launch_gu_t<2>(p, gx, st);
    case 4: return launch_gu_t<4>(p, gx, st);
    default: return launch_gu_t<8>(p, gx, st);
    }
}

template <int FMT, int NF, bool SW>
hipError_t launch_gemm_mb(const PfGemm& p, uint32_t mb, uint32_t gx, uint32_t splits, hipStream_t st)
{
    switch (mb) {
    case 1: return launch_gemm_t<FMT, 1, NF, SW>(p, gx, splits, st);
    case 2: return launch_gemm_t<FMT, 2, NF, SW>(p, gx, splits, st);
    case 4: return launch_gemm_t<FMT, 4, NF, SW>(p, gx, splits, st);
    default: return launch_gemm_t<FMT, 8, NF, SW>(p, gx, splits, st);
    }
}

template <int MB, int VF>
hipError_t launch_qkv_t(const PfGemm& qk, const PfGemm& v, uint32_t splits, hipStream_t st)
{
    const size_t lds = size_t(2) * MB * 32 * kPfLd * sizeof(_Float16);
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm_qkv<MB, VF>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((k_pf_gemm_qkv<MB, VF>), dim3(qk.tiles + v.tiles, splits), dim3(256), lds, st, qk, v);
    return hipGetLastError();
}

template <int VF>
hipError_t launch_qkv_mb(const PfGemm& qk, const PfGemm& v, uint32_t mb, uint32_t splits, hipStream_t st)
{
    switch (mb) {
    case 1: return launch_qkv_t<1, VF>(qk, v, splits, st);
    case 2: return launch_qkv_t<2, VF>(qk, v, splits, st);
    case 4: return launch_qkv_t<4, VF>(qk, v, splits, st);
    default: return launch_qkv_t<8, VF>(qk, v, splits, st);
    }
}

hipError_t launch_qkv(const PfGemm& qk, const PfGemm& v, int vtype, uint32_t mb, uint32_t splits, hipStream_t st)
{
    return vtype == kFmtQ4 ? launch_qkv_mb<kFmtQ4>(qk, v, mb, splits, st) : launch_qkv_mb<kFmtQ6P>(qk, v, mb, splits, st);
}

uint32_t m_blocks(uint32_t M)
{
    const uint32_t b = (M + 31) / 32;
    return b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : 8;
}

// Split-K plan of a PLAIN projection (NF = 1, 128 columns per workgroup):
// the split count whose super-blocks per workgroup times rounds of
// workgroups over the CUs (one resident workgroup per CU) is smallest, the
// fewest splits (least partial traffic) among equals.
void split_plan(uint32_t N, uint32_t nb, uint32_t& gx, uint32_t& splits, uint32_t& bps)
{
    gx = (N + 127) / 128;
    uint32_t best = ~0u;
    for (uint32_t want = 1; want <= nb; ++want) {
        const uint32_t b = (nb + want - 1) / want, sp = (nb + b - 1) / b;
        const uint32_t rounds = (gx * sp + kPfTargetWgs - 1) / kPfTargetWgs;
        if (b * rounds < best) {
            best = b * rounds;
            bps = b;
            splits = sp;
        }
    }
}

template <int H>
void launch_attn_t(dim3 grid, hipStream_t st, const float* q, const _Float16* kc, const _Float16* vc, uint32_t kvh,
                   uint32_t pos0, float scale, _Float16* x, uint32_t ldx)
{
    hipLaunchKernelGGL(k_pf_attn<H>, grid, dim3(256), 0, st, q, kc, vc, kvh, pos0, scale, x, ldx);
}

void launch_attn(uint32_t hpk, dim3 grid, hipStream_t st, const float* q, const _Float16* kc, const _Float16* vc,
                 uint32_t kvh, uint32_t pos0, float scale, _Float16* x, uint32_t ldx)
{
    switch (hpk) {
    case 1: launch_attn_t<1>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 2: launch_attn_t<2>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 3: launch_attn_t<3>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 4: launch_attn_t<4>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 5: launch_attn_t<5>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 6: launch_attn_t<6>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    case 7: launch_attn_t<7>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    default: launch_attn_t<8>(grid, st, q, kc, vc, kvh, pos0, scale, x, ldx); break;
    }
}

}  // namespace

uint64_t prefill_part_elems(const arc_model_dims& d)
{
    // q|k|v (one launch), o, down: [split][256][columns] partials
    const uint32_t kvd = d.kv_heads * kHeadDim;
    uint32_t gx, sp, bps;
    uint64_t part = 0;
    const uint32_t qkv_cols = ((d.hidden + kvd + 127) / 128 + (kvd + 127) / 128) * 128;
    split_plan(qkv_cols, d.hidden / kQK, gx, sp, bps);
    part = std::max(part, uint64_t(sp) * kPfMaxM * (d.hidden + 2 * kvd));
    split_plan(d.hidden, d.hidden / kQK, gx, sp, bps);
    part = std::max(part, uint64_t(sp) * kPfMaxM * d.hidden);
    split_plan(d.hidden, d.ffn / kQK, gx, sp, bps);
    part = std::max(part, uint64_t(sp) * kPfMaxM * d.hidden);
    return part;
}

int run_prefill(arc_session* S, const uint32_t* tokens, uint32_t n, uint32_t pos0, bool logits)
{
    int rc = ARC_OK;
    PrefillBufs* pf = &S->pf;
    const arc_model* Mdl = S->model;
    const arc_model_dims& d = Mdl->dims;
    const uint32_t H = d.hidden, F = d.ffn, kvd = d.kv_heads * kHeadDim, hpk = d.q_heads / d.kv_heads;
    const uint32_t passes = (n + kPfMaxM - 1) / kPfMaxM;
    if (passes > pf->host_slots)  // the caller keeps pos0 + n within max_ctx
        return set_error(ARC_ERR_INVALID_ARGUMENT, "prompt of %u tokens exceeds the session's %u positions", n,
                         S->max_ctx);
    hipStream_t st = S->stream;
    uint32_t nk = 0;
    auto chk = [&](hipError_t e, const char* what) {
        ++nk;
        return check_hip(e, what);
    };
    const float scale = 1.0f / std::sqrt(float(kHeadDim));
    for (uint32_t pass = 0; pass < passes; ++pass) {
        const uint32_t base = pass * kPfMaxM, M = std::min(uint32_t(kPfMaxM), n - base), p0 = pos0 + base;
        const uint32_t mb = m_blocks(M);
        uint32_t* ht = pf->host_tokens + size_t(pass) * kPfMaxM;
        std::memcpy(ht, tokens + base, M * sizeof(uint32_t));
        if ((rc = check_hip(hipMemcpyAsync(pf->tokens, ht, M * sizeof(uint32_t), hipMemcpyHostToDevice, st), "tokens")))
            return rc;
        // the LM head of the last row leaves position p0 + M in the control block
        S->host_ctl[1 + pass] = DecodeCtl{p0 + M - 1, 0u, 0u, 0u, 0u};
        if ((rc = check_hip(hipMemcpyAsync(S->ctl, &S->host_ctl[1 + pass], sizeof(DecodeCtl), hipMemcpyHostToDevice, st),
                            "ctl upload")))
            return rc;
        hipLaunchKernelGGL(k_pf_embed, dim3(H / kQK, M), dim3(kQK), 0, st, Mdl->emb, H / kQK, pf->tokens, pf->h);
        if ((rc = chk(hipGetLastError(), "prefill embed"))) return rc;
        for (uint32_t l = 0; l < d.layers; ++l) {
            const Layer& L = Mdl->layers[l];
            _Float16* kc = S->kcache + uint64_t(l) * S->max_ctx * kvd;
            _Float16* vc = S->vcache + uint64_t(l) * S->max_ctx * kvd;
            if (l == 0) {  // later layers: fused into the previous layer's down residual
                hipLaunchKernelGGL(k_pf_rmsnorm, dim3(M), dim3(256), 0, st, pf->h, H, L.attn_norm, d.rms_eps, pf->x, H);
                if ((rc = chk(hipGetLastError(), "attn norm"))) return rc;
            }

            PfGemm g{};
            g.M = M;
            g.mpad = kPfMaxM;
            g.x = pf->x;
            g.ldx = H;
            g.nb = H / kQK;
            g.out = pf->part;
            uint32_t gx, sp, bps;
            // q | k | v in one launch, partials [split][mpad][H | kvd | kvd]
            const uint32_t nqkv = H + 2 * kvd;
            g.w0 = L.q;
            g.w1 = L.k;
            g.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            g.ncol0 = H;
            g.N = H + kvd;
            g.ldo = nqkv;
            g.tiles = (g.N + 127) / 128;
            PfGemm gv = g;
            gv.w0 = gv.w1 = L.v;
            gv.row_bytes = uint64_t(g.nb) * (L.v_type == kFmtQ4 ? kQ4Bytes : kQ6PBytes);
            gv.ncol0 = kvd;
            gv.N = kvd;
            gv.out = pf->part + (H + kvd);
            gv.tiles = (kvd + 127) / 128;
            split_plan(g.tiles * 128 + gv.tiles * 128, g.nb, gx, sp, bps);
            g.bps = gv.bps = bps;
            if ((rc = chk(launch_qkv(g, gv, L.v_type, mb, sp, st), "q/k/v projection"))) return rc;
            hipLaunchKernelGGL(k_pf_qkv_epi, dim3((nqkv / 2 + 255) / 256, M), dim3(256), 0, st, pf->part, sp,
                               uint32_t(kPfMaxM), H, kvd, L.qb, L.kb, L.vb, S->rope, p0, pf->q, kc, vc);
            if ((rc = chk(hipGetLastError(), "q/k/v epilogue"))) return rc;
            // attention -> x
            if (g_pf_attn_mfma)
                hipLaunchKernelGGL(k_pf_attn_mf, dim3((M + 31) / 32, d.q_heads), dim3(256), 0, st, pf->q, kc, vc,
                                   d.kv_heads, hpk, p0, M, S->max_ctx, scale, pf->x, H);
            else
                launch_attn(hpk, dim3(M, d.kv_heads), st, pf->q, kc, vc, d.kv_heads, p0, scale, pf->x, H);
            if ((rc = chk(hipGetLastError(), "prefill attention"))) return rc;
            // o + residual + ffn norm
            g.w0 = g.w1 = L.o;
            g.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            g.ncol0 = H;
            g.N = H;
            g.ldo = H;
            split_plan(g.N, g.nb, gx, sp, bps);
            g.bps = bps;
            if ((rc = chk(launch_gemm_mb<kFmtQ4, 1, false>(g, mb, gx, sp, st), "o projection"))) return rc;
            launch_res_norm<true>(M, st, pf->part, sp, uint32_t(kPfMaxM), H, pf->h, L.ffn_norm, d.rms_eps, pf->x, H);
            if ((rc = chk(hipGetLastError(), "o residual + ffn norm"))) return rc;
            // gate/up + SwiGLU -> xs
            PfGemm u = g;
            u.w0 = L.gate;
            u.w1 = L.up;
            u.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            u.N = F;
            u.ncol0 = F;
            u.bps = g.nb;
            u.s = pf->xs;
            u.lds_out = F;
            if ((rc = chk(launch_gateup(u, mb, (F + 127) / 128, st), "gate/up"))) return rc;
            // down + residual (+ the next layer's attention norm)
            PfGemm dn = g;
            dn.x = pf->xs;
            dn.ldx = F;
            dn.nb = F / kQK;
            dn.w0 = dn.w1 = L.down;
            dn.row_bytes = uint64_t(dn.nb) * (L.down_type == kFmtQ4 ? kQ4Bytes : kQ6PBytes);
            dn.ncol0 = H;
            dn.N = H;
            dn.ldo = H;
            split_plan(dn.N, dn.nb, gx, sp, bps);
            dn.bps = bps;
            rc = chk(L.down_type == kFmtQ4 ? launch_gemm_mb<kFmtQ4, 1, false>(dn, mb, gx, sp, st)
                                           : launch_gemm_mb<kFmtQ6P, 1, false>(dn, mb, gx, sp, st),
                     "down projection");
            if (rc) return rc;
            if (l + 1 < d.layers) {
                launch_res_norm<true>(M, st, pf->part, sp, uint32_t(kPfMaxM), H, pf->h, Mdl->layers[l + 1].attn_norm,
                                      d.rms_eps, pf->x, H);
            } else {
                launch_res_norm<false>(M, st, pf->part, sp, uint32_t(kPfMaxM), H, pf->h, nullptr, 0.0f, nullptr, 0u);
            }
            if ((rc = chk(hipGetLastError(), "down residual"))) return rc;
        }
        if (pass + 1 == passes) {
            if ((rc = launch_lm_head(S, pf->h + uint64_t(M - 1) * H, logits, st))) return rc;
            nk += 1;
        }
    }
    S->prefill_kernels = nk;
    return ARC_OK;
}

}  // namespace arc

// ------------------------------------ standalone prompt-pass projections
namespace arc {
namespace {

struct PfWorkspace {
    size_t x, part, bytes;
};

// X staging (256 rows of K fp16: the GEMM tiles read up to 256 rows) and the
// split partials of the N x K projection's plan.
PfWorkspace pf_workspace(uint32_t N, uint32_t K)
{
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    uint32_t gx, sp, bps;
    split_plan(N, K / kQK, gx, sp, bps);
    PfWorkspace w{};
    w.x = 0;
    w.part = up(size_t(kPfMaxM) * K * sizeof(_Float16));
    w.bytes = w.part + up(size_t(sp) * kPfMaxM * N * sizeof(float));
    return w;
}

int pf_check(const void* w, uint32_t N, uint32_t K, const uint16_t* x, uint32_t M, const void* out, const void* ws)
{
    if (!w || !x || !out || !ws) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    if (N == 0 || K == 0 || K % kQK || M == 0 || M > uint32_t(kPfMaxM))
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad shape N=%u K=%u M=%u (K a multiple of 256, 1 <= M <= %d)", N, K,
                         M, kPfMaxM);
    if (N > uint32_t(kResCols) * 1024u) return set_error(ARC_ERR_UNSUPPORTED, "N must be <= %d", kResCols * 1024);
    if (reinterpret_cast<uintptr_t>(w) & 15u) return set_error(ARC_ERR_INVALID_ARGUMENT, "weights not 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(ws) & 255u)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    return ARC_OK;
}

// Copies the M given rows of X into the staging area and zeroes the rows the
// tiles read past them (up to the 32-row block count of M).
int pf_stage_x(uint8_t* ws, const PfWorkspace& w, const uint16_t* x, uint32_t M, uint32_t K, hipStream_t st)
{
    _Float16* xs = reinterpret_cast<_Float16*>(ws + w.x);
    const size_t row = size_t(K) * sizeof(_Float16), rows = size_t(m_blocks(M)) * 32;
    int rc = check_hip(hipMemcpyAsync(xs, x, M * row, hipMemcpyDeviceToDevice, st), "x staging");
    if (rc) return rc;
    if (rows > M) rc = check_hip(hipMemsetAsync(reinterpret_cast<uint8_t*>(xs) + M * row, 0, (rows - M) * row, st), "x pad");
    return rc;
}

// y[m][c] = sum over the splits of part[s][m][c], in split order.
int pf_reduce(const float* part, uint32_t splits, uint32_t M, uint32_t N, float* y, hipStream_t st)
{
    int rc = check_hip(hipMemsetAsync(y, 0, size_t(M) * N * sizeof(float), st), "y clear");
    if (rc) return rc;
    launch_res_norm<false>(M, st, part, splits, uint32_t(kPfMaxM), N, y, nullptr, 0.0f, nullptr, 0u);
    return check_hip(hipGetLastError(), "split reduction");
}

}  // namespace
}  // namespace arc

using namespace arc;

extern "C" {

int arc_tune_prefill_attention(int mfma)
{
    if (mfma != 0 && mfma != 1) return set_error(ARC_ERR_INVALID_ARGUMENT, "prefill attention: 0 (VALU) or 1 (MFMA)");
    g_pf_attn_mfma = mfma;
    return ARC_OK;
}

size_t arc_prefill_gemm_workspace_bytes(uint32_t N, uint32_t K)
{
    if (N == 0 || K == 0 || K % kQK) return 0;
    return pf_workspace(N, K).bytes;
}

int arc_prefill_gemm(int qtype, const void* w, uint32_t N, uint32_t K, const uint16_t* x, uint32_t M, float* y,
                     void* workspace, arc_stream_t stream)
{
    int rc = pf_check(w, N, K, x, M, y, workspace);
    if (rc) return rc;
    if (qtype != kFmtQ4 && qtype != kFmtQ6P)
        return set_error(ARC_ERR_UNSUPPORTED, "the prompt-pass GEMM takes Q4_K or padded Q6_K (qtype %d)", qtype);
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const PfWorkspace pw = pf_workspace(N, K);
    if ((rc = pf_stage_x(ws, pw, x, M, K, st))) return rc;
    PfGemm g{};
    g.M = M;
    g.mpad = kPfMaxM;
    g.x = reinterpret_cast<const _Float16*>(ws + pw.x);
    g.ldx = K;
    g.nb = K / kQK;
    g.out = reinterpret_cast<float*>(ws + pw.part);
    g.w0 = g.w1 = static_cast<const uint8_t*>(w);
    g.row_bytes = uint64_t(g.nb) * (qtype == kFmtQ4 ? kQ4Bytes : kQ6PBytes);
    g.ncol0 = N;
    g.N = N;
    g.ldo = N;
    uint32_t gx, sp, bps;
    split_plan(N, g.nb, gx, sp, bps);
    g.bps = bps;
    const uint32_t mb = m_blocks(M);
    rc = check_hip(qtype == kFmtQ4 ? launch_gemm_mb<kFmtQ4, 1, false>(g, mb, gx, sp, st)
                                   : launch_gemm_mb<kFmtQ6P, 1, false>(g, mb, gx, sp, st),
                   "prompt-pass GEMM");
    if (rc) return rc;
    return pf_reduce(g.out, sp, M, N, y, st);
}

int arc_prefill_gateup(const void* w_gate, const void* w_up, uint32_t N, uint32_t K, const uint16_t* x, uint32_t M,
                       uint16_t* s, void* workspace, arc_stream_t stream)
{
    int rc = pf_check(w_gate, N, K, x, M, s, workspace);
    if (rc) return rc;
    if (!w_up || (reinterpret_cast<uintptr_t>(w_up) & 15u))
        return set_error(ARC_ERR_INVALID_ARGUMENT, "up weights null or not 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const PfWorkspace pw = pf_workspace(N, K);
    if ((rc = pf_stage_x(ws, pw, x, M, K, st))) return rc;
    PfGemm u{};
    u.M = M;
    u.mpad = kPfMaxM;
    u.x = reinterpret_cast<const _Float16*>(ws + pw.x);
    u.ldx = K;
    u.nb = K / kQK;
    u.w0 = static_cast<const uint8_t*>(w_gate);
    u.w1 = static_cast<const uint8_t*>(w_up);
    u.row_bytes = uint64_t(u.nb) * kQ4Bytes;
    u.N = N;
    u.ncol0 = N;
    u.bps = u.nb;
    u.s = reinterpret_cast<_Float16*>(s);
    u.lds_out = N;
    return check_hip(launch_gateup(u, m_blocks(M), (N + 127) / 128, st), "prompt-pass gate/up");
}

int arc_prefill_attention(const float* q, const void* kc, const void* vc, uint32_t kv_heads, uint32_t hpk,
                          uint32_t max_ctx, uint32_t pos0, uint32_t M, uint16_t* x, uint32_t ldx, int mfma,
                          arc_stream_t stream)
{
    if (!q || !kc || !vc || !x) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    if (kv_heads == 0 || kv_heads > 64 || hpk == 0 || hpk > uint32_t(kMaxHpk))
        return set_error(ARC_ERR_UNSUPPORTED, "prefill attention supports 1..64 kv heads and 1..%d query heads per kv "
                         "head", kMaxHpk);
    if (M == 0 || max_ctx == 0 || max_ctx > uint32_t(kMaxChunks * kChunk) || uint64_t(pos0) + M > max_ctx)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad rows: pos0 %u + M %u > max_ctx %u (at most %d)", pos0, M,
                         max_ctx, kMaxChunks * kChunk);
    const uint32_t hidden = kv_heads * hpk * kHeadDim;
    if (ldx < hidden) return set_error(ARC_ERR_INVALID_ARGUMENT, "ldx %u < %u", ldx, hidden);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) |
                         reinterpret_cast<uintptr_t>(vc);
    if (al & 15u) return set_error(ARC_ERR_INVALID_ARGUMENT, "q, kc and vc must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const _Float16* k16 = static_cast<const _Float16*>(kc);
    const _Float16* v16 = static_cast<const _Float16*>(vc);
    _Float16* x16 = reinterpret_cast<_Float16*>(x);
    const float scale = 1.0f / std::sqrt(float(kHeadDim));
    if (mfma)
        hipLaunchKernelGGL(k_pf_attn_mf, dim3((M + 31) / 32, kv_heads * hpk), dim3(256), 0, st, q, k16, v16, kv_heads,
                           hpk, pos0, M, max_ctx, scale, x16, ldx);
    else
        launch_attn(hpk, dim3(M, kv_heads), st, q, k16, v16, kv_heads, pos0, scale, x16, ldx);
    return check_hip(hipGetLastError(), "prefill attention");
}

int arc_prefill_qkv(const void* wq, const void* wk, const void* wv, int v_qtype, uint32_t H, uint32_t kvd, uint32_t K,
                    const uint16_t* x, uint32_t M, float* y, void* workspace, arc_stream_t stream)
{
    const uint32_t N = H + 2 * kvd;
    int rc = pf_check(wq, N, K, x, M, y, workspace);
    if (rc) return rc;
    if (!wk || !wv || ((reinterpret_cast<uintptr_t>(wk) | reinterpret_cast<uintptr_t>(wv)) & 15u))
        return set_error(ARC_ERR_INVALID_ARGUMENT, "k or v weights null or not 16-byte aligned");
    if (v_qtype != kFmtQ4 && v_qtype != kFmtQ6P)
        return set_error(ARC_ERR_UNSUPPORTED, "v must be Q4_K or padded Q6_K (qtype %d)", v_qtype);
    if (H == 0 || kvd == 0 || H % 128 || kvd % 128)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "H and kvd must be nonzero multiples of 128");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const PfWorkspace pw = pf_workspace(N, K);
    if ((rc = pf_stage_x(ws, pw, x, M, K, st))) return rc;
    // as run_prefill: q|k one operand, v the other, partials [split][mpad][H | kvd | kvd]
    PfGemm g{};
    g.M = M;
    g.mpad = kPfMaxM;
    g.x = reinterpret_cast<const _Float16*>(ws + pw.x);
    g.ldx = K;
    g.nb = K / kQK;
    g.out = reinterpret_cast<float*>(ws + pw.part);
    g.w0 = static_cast<const uint8_t*>(wq);
    g.w1 = static_cast<const uint8_t*>(wk);
    g.row_bytes = uint64_t(g.nb) * kQ4Bytes;
    g.ncol0 = H;
    g.N = H + kvd;
    g.ldo = N;
    g.tiles = (g.N + 127) / 128;
    PfGemm gv = g;
    gv.w0 = gv.w1 = static_cast<const uint8_t*>(wv);
    gv.row_bytes = uint64_t(g.nb) * (v_qtype == kFmtQ4 ? kQ4Bytes : kQ6PBytes);
    gv.ncol0 = kvd;
    gv.N = kvd;
    gv.out = g.out + (H + kvd);
    gv.tiles = (kvd + 127) / 128;
    uint32_t gx, sp, bps;
    split_plan(g.tiles * 128 + gv.tiles * 128, g.nb, gx, sp, bps);
    g.bps = gv.bps = bps;
    // the partial buffer is sized by the plan of N columns; the q|k|v plan's
    // split count must fit it
    uint32_t gx2, sp2, bps2;
    split_plan(N, g.nb, gx2, sp2, bps2);
    if (sp > sp2) return set_error(ARC_ERR_UNSUPPORTED, "internal: q/k/v split plan %u > workspace plan %u", sp, sp2);
    if ((rc = check_hip(launch_qkv(g, gv, v_qtype, m_blocks(M), sp, st), "prompt-pass q/k/v"))) return rc;
    return pf_reduce(g.out, sp, M, N, y, st);
}

}  // extern "C"
