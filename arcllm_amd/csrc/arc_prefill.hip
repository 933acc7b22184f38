// arc_prefill.hip -- the batched prompt pass on gfx950 MFMA (the reference's
// build_prefill, src/arcllm_v1_runtime.cpp:340-369, which runs dequant-in-LDS
// fp32 tiles).
//
// A prompt of M <= 256 tokens at positions pos0 .. pos0+M-1 is processed as
// matrices: per layer
//   RMSNorm(H) -> X (fp16)                                    k_pf_rmsnorm
//   [q|k] = X Wqk^T  (split-K partials)                        k_pf_gemm<Q4>
//   + bias, RoPE, q -> fp32, k -> fp16 cache rows               k_pf_qk_epi
//   v = X Wv^T, + bias -> fp16 cache rows                       k_pf_gemm, k_pf_v_epi
//   causal GQA over the cache (positions <= own) -> X (fp16)    k_pf_attn
//   H += X Wo^T                                                 k_pf_gemm, k_pf_res_epi
//   RMSNorm(H) -> X; s = silu(X Wg^T) * (X Wu^T) -> X (fp16)    k_pf_rmsnorm, k_pf_gemm<SWIGLU>
//   H += s Wd^T                                                 k_pf_gemm, k_pf_res_epi
// then the output RMSNorm + LM head + argmax on the last row only (the
// decode step's kernels), leaving the argmax as the next token.
//
// GEMM (k_pf_gemm): Y[m][n] = sum_k X[m][k] W[n][k] with
// v_mfma_f32_32x32x16_f16.  A workgroup owns all M rows (MB blocks of 32) and
// 128 weight rows (4 waves x 32); X is staged through LDS in half-super-block
// tiles (double-buffered, rows padded by 8 halves so the 16-byte fragment
// reads are bank-conflict free); each lane dequantises its own B fragment
// (8 consecutive weights of one row per 16-wide K step) straight from the
// packed super-block into fp16 registers: w = (d*sc)*q - dmin*mn (Q4_K) or
// (d*sc)*q (Q6_K) in fp32, as the element decode, then rounded to fp16.
// Operands are fp16, accumulation fp32.
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

constexpr int kPfMaxM = 256;       // prompt rows per pass
constexpr int kPfKT = 128;         // K columns per LDS stage (half a super-block)
constexpr int kPfLd = kPfKT + 8;   // padded LDS row, in halves

struct PrefillBufs {
    float* h = nullptr;         // [256][hidden] residual stream
    _Float16* x = nullptr;      // [256][hidden] fp16 GEMM input (normed h, attention output)
    _Float16* xs = nullptr;     // [256][ffn] fp16 SwiGLU output (input of ffn_down)
    float* q = nullptr;         // [256][hidden] q after RoPE
    float* part = nullptr;      // split-K partials
    size_t part_elems = 0;
    uint32_t* tokens = nullptr; // [256] device
    uint32_t* host_tokens = nullptr;  // pinned staging, one slot of 256 per pass of a call
    uint32_t host_slots = 0;
    uint32_t kernels = 0;       // launches of the last prompt pass
    std::vector<void*> allocs;
};

void destroy_prefill(PrefillBufs* pf)
{
    if (!pf) return;
    for (void* p : pf->allocs) (void)hipFree(p);
    if (pf->host_tokens) (void)hipHostFree(pf->host_tokens);
    delete pf;
}

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
    float* out;          // PLAIN: [split][mpad][N]
    _Float16* s;         // SWIGLU: [M][lds_out]
    uint32_t lds_out;
};

// 8 bytes from a 2-byte-aligned address inside a Q6_K block, from dword
// loads at the dword-aligned floor, realigned in registers.  All dwords read
// lie inside the 210-byte block for the offsets used below.
__device__ __forceinline__ void ld8_2a(const uint8_t* p, uint32_t& lo, uint32_t& hi)
{
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p)) & 3u;
    const uint32_t* a = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t d0 = a[0], d1 = a[1];
    const uint32_t d2 = sh ? a[2] : 0u;
    lo = __builtin_amdgcn_alignbyte(d1, d0, sh);
    hi = __builtin_amdgcn_alignbyte(d2, d1, sh);
}

// Per-super-block factors of one row: Q4_K f[j] = d*sc_j, g[j] = dmin*mn_j
// (j = 0..7); Q6_K f[j] = d*sc_j (j = 0..15).
template <int FMT>
struct BlkScale {
    float f[FMT == kFmtQ4 ? 8 : 16];
    float g[FMT == kFmtQ4 ? 8 : 1];
};

template <int FMT>
__device__ __forceinline__ void load_scales(const uint8_t* blk, BlkScale<FMT>& s)
{
#pragma clang fp contract(off)
    if constexpr (FMT == kFmtQ4) {
        const uint4 h = *reinterpret_cast<const uint4*>(blk);
        const float d = f16_bits_to_f32(h.x), dmin = f16_bits_to_f32(h.x >> 16);
        const uint32_t b[3] = {h.y, h.z, h.w};
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
            s.f[j] = d * float(sc);
            s.g[j] = dmin * float(mn);
        }
    } else {
        uint32_t lo, hi, l2, h2;
        ld8_2a(blk + 192, lo, hi);
        ld8_2a(blk + 200, l2, h2);
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208));
        const uint32_t sw[4] = {lo, hi, l2, h2};
#pragma unroll
        for (int j = 0; j < 16; ++j) s.f[j] = d * float(int8_t(uint8_t(sw[j >> 2] >> (8 * (j & 3)))));
        s.g[0] = 0.0f;
    }
}

// The 8 weights at elements hb*128 + KS*16 + kh*8 .. +7 of one super-block
// row (hb: half block, KS: 16-wide K step, kh: lane half), as fp16, with the
// element decode's fp32 arithmetic.  a / c are the factors of the element's
// sub-block (Q4_K: d*sc, dmin*mn; Q6_K: d*sc), selected by the caller so no
// register array is indexed at run time.
template <int FMT, int KS>
__device__ __forceinline__ half8 dequant8(const uint8_t* blk, uint32_t hb, uint32_t kh, float a, float c)
{
#pragma clang fp contract(off)
    half8 w;
    if constexpr (FMT == kFmtQ4) {
        // element e = hb*128 + KS*16 + kh*8: chunk byte 16 + (e>>6)*32 + (e&31), high nibble when e&32
        const uint2 q = *reinterpret_cast<const uint2*>(blk + 16 + (hb * 2 + KS / 4) * 32 + (KS & 1) * 16 + kh * 8);
        constexpr uint32_t sh = ((KS >> 1) & 1) ? 4u : 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xffu;
            const float b = a * float((byte >> sh) & 15u);
            w[i] = _Float16(b - c);
        }
    } else {
        // half hb, quarter KS/2, l0 = (KS&1)*16 + kh*8
        constexpr uint32_t quarter = KS >> 1;
        const uint32_t l0 = (KS & 1) * 16 + kh * 8;
        uint32_t ql0, ql1, qh0, qh1;
        ld8_2a(blk + hb * 64 + l0 + 32 * (quarter & 1u), ql0, ql1);
        ld8_2a(blk + 128 + hb * 32 + l0, qh0, qh1);
        constexpr uint32_t lsh = (quarter >> 1) * 4u, hsh = quarter * 2u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lb = ((i < 4 ? ql0 : ql1) >> (8 * (i & 3))) & 0xffu;
            const uint32_t hbt = ((i < 4 ? qh0 : qh1) >> (8 * (i & 3))) & 0xffu;
            const int code = int(((lb >> lsh) & 15u) | (((hbt >> hsh) & 3u) << 4)) - 32;
            w[i] = _Float16(a * float(code));
        }
        (void)c;
    }
    return w;
}

// X staging of one LDS stage: K columns [k0, k0+128) of rows [0, MB*32),
// MB*32*16 pieces of 16 bytes, MB*2 per thread.
template <int MB>
__device__ __forceinline__ void x_fetch(const PfGemm& p, uint32_t k0, u32x4 (&reg)[MB * 2])
{
#pragma unroll
    for (int i = 0; i < MB * 2; ++i) {
        const uint32_t c = threadIdx.x + 256u * uint32_t(i);
        reg[i] = *reinterpret_cast<const u32x4*>(p.x + uint64_t(c >> 4) * p.ldx + k0 + (c & 15u) * 8);
    }
}

template <int MB>
__device__ __forceinline__ void x_store(_Float16* stage, const u32x4 (&reg)[MB * 2])
{
#pragma unroll
    for (int i = 0; i < MB * 2; ++i) {
        const uint32_t c = threadIdx.x + 256u * uint32_t(i);
        *reinterpret_cast<u32x4*>(stage + (c >> 4) * kPfLd + (c & 15u) * 8) = reg[i];
    }
}

// One 16-wide K step: this lane's B fragment, then MB MFMAs.
template <int FMT, int MB, int HB, int KS>
__device__ __forceinline__ void k_step(const uint8_t* blk, uint32_t kh, const BlkScale<FMT>& sc, const _Float16* a,
                                       f32x16 (&acc)[MB])
{
    // sub-block factors of elements HB*128 + KS*16 + kh*8 .. +7
    constexpr int F = FMT == kFmtQ4 ? HB * 4 + KS / 2 : HB * 8 + KS;
    const float fc = FMT == kFmtQ4 ? sc.g[F < 8 ? F : 0] : 0.0f;
    const half8 b = dequant8<FMT, KS>(blk, HB, kh, sc.f[F], fc);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const half8 av = *reinterpret_cast<const half8*>(a + mb * 32 * kPfLd + KS * 16);
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b, acc[mb], 0, 0, 0);
    }
}

template <int FMT, int MB, int HB>
__device__ __forceinline__ void half_block(const uint8_t* blk, uint32_t kh, const BlkScale<FMT>& sc, const _Float16* a,
                                           f32x16 (&acc)[MB])
{
    k_step<FMT, MB, HB, 0>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 1>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 2>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 3>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 4>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 5>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 6>(blk, kh, sc, a, acc);
    k_step<FMT, MB, HB, 7>(blk, kh, sc, a, acc);
}

template <int FMT, int MB, bool SWIGLU>
__global__ __launch_bounds__(256, 1) void k_pf_gemm(PfGemm p)
{
    extern __shared__ _Float16 ash[];  // [2][MB*32][kPfLd]
    constexpr int kRows = MB * 32;
    constexpr int kStage = kRows * kPfLd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // this lane's weight row (B column) and output column
    uint32_t col;
    const uint8_t* wrow;
    if constexpr (SWIGLU) {
        col = blockIdx.x * 64 + (wave & 1) * 32 + (lane & 31);
        const uint32_t r = min(col, p.N - 1);
        wrow = (wave < 2 ? p.w0 : p.w1) + uint64_t(r) * p.row_bytes;
    } else {
        col = blockIdx.x * 128 + wave * 32 + (lane & 31);
        const uint32_t r = min(col, p.N - 1);
        wrow = r < p.ncol0 ? p.w0 + uint64_t(r) * p.row_bytes : p.w1 + uint64_t(r - p.ncol0) * p.row_bytes;
    }
    constexpr int kBB = FMT == kFmtQ4 ? kQ4Bytes : kQ6Bytes;
    const uint32_t kb0 = blockIdx.y * p.bps, kb1 = min(p.nb, kb0 + p.bps);
    const uint32_t kh = uint32_t(lane) >> 5;

    f32x16 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;

    // stage 0 holds the first half of the current super-block, stage 1 the
    // second; each half's compute overlaps the fetch of the next half, whose
    // LDS store follows a barrier (the last fetch repeats the last half).
    u32x4 reg[MB * 2];
    x_fetch<MB>(p, kb0 * kQK, reg);
    x_store<MB>(ash, reg);
    __syncthreads();
    const _Float16* a0 = ash + (lane & 31) * kPfLd + kh * 8;
    const _Float16* a1 = a0 + kStage;
    for (uint32_t kb = kb0; kb < kb1; ++kb) {
        const uint8_t* blk = wrow + uint64_t(kb) * kBB;
        BlkScale<FMT> sc;
        load_scales<FMT>(blk, sc);
        x_fetch<MB>(p, kb * kQK + kPfKT, reg);
        half_block<FMT, MB, 0>(blk, kh, sc, a0, acc);
        x_store<MB>(ash + kStage, reg);
        __syncthreads();
        const uint32_t nk = kb + 1 < kb1 ? kb + 1 : kb;
        x_fetch<MB>(p, nk * kQK, reg);
        half_block<FMT, MB, 1>(blk, kh, sc, a1, acc);
        __syncthreads();
        x_store<MB>(ash, reg);
        __syncthreads();
    }

    // D[m][col]: register i of block mb holds row mb*32 + (i/4)*8 + (lane/32)*4 + i%4
    if constexpr (SWIGLU) {
        float* u = reinterpret_cast<float*>(ash);  // [kRows][64], after the last sync
        if (wave >= 2) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int m = mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                    u[m * 64 + (wave & 1) * 32 + (lane & 31)] = acc[mb][i];
                }
        }
        __syncthreads();
        if (wave < 2 && col < p.N) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t m = mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                    if (m < p.M) {
                        const float g = acc[mb][i], uv = u[m * 64 + (wave & 1) * 32 + (lane & 31)];
                        p.s[uint64_t(m) * p.lds_out + col] = _Float16((g / (1.0f + expf(-g))) * uv);
                    }
                }
        }
    } else {
        if (col < p.N) {
            float* o = p.out + uint64_t(blockIdx.y) * p.mpad * p.N + col;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t m = mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                    if (m < p.M) o[uint64_t(m) * p.N] = acc[mb][i];
                }
        }
    }
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

// q/k: per (m, column pair): fixed-order sum of the split partials + bias,
// RoPE on the pair, q -> fp32, k -> fp16 cache row pos0 + m.
__global__ __launch_bounds__(256) void k_pf_qk_epi(const float* __restrict__ part, uint32_t splits, uint32_t mpad,
                                                   uint32_t hidden, uint32_t kv_dim, const float* __restrict__ qb,
                                                   const float* __restrict__ kb, const float2* __restrict__ rope,
                                                   uint32_t pos0, float* __restrict__ q, _Float16* __restrict__ kc)
{
    const uint32_t N = hidden + kv_dim, m = blockIdx.y;
    const uint32_t c = 2 * (blockIdx.x * 256 + threadIdx.x);
    if (c >= N) return;
    float a = 0.0f, b = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) {
        const float2 v = *reinterpret_cast<const float2*>(part + (uint64_t(s) * mpad + m) * N + c);
        a += v.x;
        b += v.y;
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

// v: fixed-order split sum + bias -> fp16 cache row pos0 + m.
__global__ __launch_bounds__(256) void k_pf_v_epi(const float* __restrict__ part, uint32_t splits, uint32_t mpad,
                                                  uint32_t kv_dim, const float* __restrict__ vb, uint32_t pos0,
                                                  _Float16* __restrict__ vc)
{
    const uint32_t m = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (c >= kv_dim) return;
    float a = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) a += part[(uint64_t(s) * mpad + m) * kv_dim + c];
    vc[uint64_t(pos0 + m) * kv_dim + c] = _Float16(a + vb[c]);
}

// H[m][c] += fixed-order split sum.
__global__ __launch_bounds__(256) void k_pf_res_epi(const float* __restrict__ part, uint32_t splits, uint32_t mpad,
                                                    uint32_t n, float* __restrict__ h)
{
    const uint32_t m = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (c >= n) return;
    float a = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) a += part[(uint64_t(s) * mpad + m) * n + c];
    h[uint64_t(m) * n + c] = h[uint64_t(m) * n + c] + a;
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
        {   // scores of positions t0 + tk
            float s[HPK];
#pragma unroll
            for (int h = 0; h < HPK; ++h) s[h] = 0.0f;
            const uint4* kp = reinterpret_cast<const uint4*>(kc + uint64_t(t0 + min(tk, nt - 1)) * kvd + g * kHeadDim +
                                                             part * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 raw = kp[i];
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
            const _Float16* vb = vc + uint64_t(t0) * kvd + g * kHeadDim + 2 * vi;
#pragma unroll 4
            for (int tt = 0; tt < 16; ++tt) {
                const uint32_t t = pg * 16 + tt;
                const bool in = t < nt;
                const half2_t vv = *reinterpret_cast<const half2_t*>(vb + uint64_t(min(t, nt - 1)) * kvd);
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

// ------------------------------------------------------------------ host
namespace {

constexpr uint32_t kPfTargetWgs = 256;

template <int FMT, int MB, bool SW>
hipError_t launch_gemm_t(const PfGemm& p, uint32_t gx, uint32_t splits, hipStream_t st)
{
    const size_t lds = size_t(2) * MB * 32 * kPfLd * sizeof(_Float16);
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_pf_gemm<FMT, MB, SW>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((k_pf_gemm<FMT, MB, SW>), dim3(gx, splits), dim3(256), lds, st, p);
    return hipGetLastError();
}

template <int FMT, bool SW>
hipError_t launch_gemm_mb(const PfGemm& p, uint32_t mb, uint32_t gx, uint32_t splits, hipStream_t st)
{
    switch (mb) {
    case 1: return launch_gemm_t<FMT, 1, SW>(p, gx, splits, st);
    case 2: return launch_gemm_t<FMT, 2, SW>(p, gx, splits, st);
    case 4: return launch_gemm_t<FMT, 4, SW>(p, gx, splits, st);
    default: return launch_gemm_t<FMT, 8, SW>(p, gx, splits, st);
    }
}

uint32_t m_blocks(uint32_t M)
{
    const uint32_t b = (M + 31) / 32;
    return b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : 8;
}

// Split-K plan of a PLAIN projection: enough workgroups to cover the CUs.
void split_plan(uint32_t N, uint32_t nb, uint32_t& gx, uint32_t& splits, uint32_t& bps)
{
    gx = (N + 127) / 128;
    uint32_t want = (kPfTargetWgs + gx - 1) / gx;
    want = std::max(1u, std::min(want, nb));
    bps = (nb + want - 1) / want;
    splits = (nb + bps - 1) / bps;
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

int ensure_bufs(arc_session* S)
{
    if (S->pf) return ARC_OK;
    const arc_model_dims& d = S->model->dims;
    std::unique_ptr<PrefillBufs> pf(new (std::nothrow) PrefillBufs);
    if (!pf) return set_error(ARC_ERR_OUT_OF_MEMORY, "host allocation");
    auto alloc = [&](void** p, size_t bytes) {
        const int r = check_hip(hipMalloc(p, bytes), "hipMalloc prefill");
        if (!r) pf->allocs.push_back(*p);
        return r;
    };
    const uint32_t kvd = d.kv_heads * kHeadDim;
    size_t part = 0;
    const uint32_t shapes[3][2] = {{d.hidden + kvd, d.hidden / kQK}, {kvd, d.hidden / kQK}, {d.hidden, d.hidden / kQK}};
    for (const auto& sh : shapes) {
        uint32_t gx, sp, bps;
        split_plan(sh[0], sh[1], gx, sp, bps);
        part = std::max(part, size_t(sp) * kPfMaxM * sh[0]);
    }
    {
        uint32_t gx, sp, bps;
        split_plan(d.hidden, d.ffn / kQK, gx, sp, bps);
        part = std::max(part, size_t(sp) * kPfMaxM * d.hidden);
    }
    void* p = nullptr;
    int rc;
    if ((rc = alloc(&p, size_t(kPfMaxM) * d.hidden * sizeof(float)))) return rc;
    pf->h = static_cast<float*>(p);
    if ((rc = alloc(&p, size_t(kPfMaxM) * d.hidden * sizeof(_Float16)))) return rc;
    pf->x = static_cast<_Float16*>(p);
    if ((rc = alloc(&p, size_t(kPfMaxM) * d.ffn * sizeof(_Float16)))) return rc;
    pf->xs = static_cast<_Float16*>(p);
    if ((rc = alloc(&p, size_t(kPfMaxM) * d.hidden * sizeof(float)))) return rc;
    pf->q = static_cast<float*>(p);
    if ((rc = alloc(&p, part * sizeof(float)))) return rc;
    pf->part = static_cast<float*>(p);
    pf->part_elems = part;
    if ((rc = alloc(&p, kPfMaxM * sizeof(uint32_t)))) return rc;
    pf->tokens = static_cast<uint32_t*>(p);
    // rows past the prompt are read (never written) by the GEMM tiles
    if ((rc = check_hip(hipMemset(pf->x, 0, size_t(kPfMaxM) * d.hidden * sizeof(_Float16)), "prefill x"))) return rc;
    if ((rc = check_hip(hipMemset(pf->xs, 0, size_t(kPfMaxM) * d.ffn * sizeof(_Float16)), "prefill xs"))) return rc;
    S->pf = pf.release();
    return ARC_OK;
}

}  // namespace

int run_prefill(arc_session* S, const uint32_t* tokens, uint32_t n, uint32_t pos0, bool logits)
{
    int rc = ensure_bufs(S);
    if (rc) return rc;
    PrefillBufs* pf = S->pf;
    const arc_model* Mdl = S->model;
    const arc_model_dims& d = Mdl->dims;
    const uint32_t H = d.hidden, F = d.ffn, kvd = d.kv_heads * kHeadDim, hpk = d.q_heads / d.kv_heads;
    const uint32_t passes = (n + kPfMaxM - 1) / kPfMaxM;
    if (pf->host_slots < passes) {
        if (pf->host_tokens) (void)hipHostFree(pf->host_tokens);
        pf->host_tokens = nullptr;
        pf->host_slots = 0;
        if ((rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&pf->host_tokens),
                                          size_t(passes) * kPfMaxM * sizeof(uint32_t), hipHostMallocDefault),
                            "pinned prompt")))
            return rc;
        pf->host_slots = passes;
    }
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
        S->host_ctl[1 + pass] = DecodeCtl{p0 + M - 1, 0u, 0u, 0u};
        if ((rc = check_hip(hipMemcpyAsync(S->ctl, &S->host_ctl[1 + pass], sizeof(DecodeCtl), hipMemcpyHostToDevice, st),
                            "ctl upload")))
            return rc;
        hipLaunchKernelGGL(k_pf_embed, dim3(H / kQK, M), dim3(kQK), 0, st, Mdl->emb, H / kQK, pf->tokens, pf->h);
        if ((rc = chk(hipGetLastError(), "prefill embed"))) return rc;
        for (uint32_t l = 0; l < d.layers; ++l) {
            const Layer& L = Mdl->layers[l];
            _Float16* kc = S->kcache + uint64_t(l) * S->max_ctx * kvd;
            _Float16* vc = S->vcache + uint64_t(l) * S->max_ctx * kvd;
            hipLaunchKernelGGL(k_pf_rmsnorm, dim3(M), dim3(256), 0, st, pf->h, H, L.attn_norm, d.rms_eps, pf->x, H);
            if ((rc = chk(hipGetLastError(), "attn norm"))) return rc;

            PfGemm g{};
            g.M = M;
            g.mpad = kPfMaxM;
            g.x = pf->x;
            g.ldx = H;
            g.nb = H / kQK;
            g.out = pf->part;
            uint32_t gx, sp, bps;
            // q | k
            g.w0 = L.q;
            g.w1 = L.k;
            g.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            g.ncol0 = H;
            g.N = H + kvd;
            split_plan(g.N, g.nb, gx, sp, bps);
            g.bps = bps;
            if ((rc = chk(launch_gemm_mb<kFmtQ4, false>(g, mb, gx, sp, st), "q/k projection"))) return rc;
            hipLaunchKernelGGL(k_pf_qk_epi, dim3((g.N / 2 + 255) / 256, M), dim3(256), 0, st, pf->part, sp,
                               uint32_t(kPfMaxM), H, kvd, L.qb, L.kb, S->rope, p0, pf->q, kc);
            if ((rc = chk(hipGetLastError(), "q/k epilogue"))) return rc;
            // v
            g.w0 = g.w1 = L.v;
            g.row_bytes = uint64_t(g.nb) * (L.v_type == kFmtQ4 ? kQ4Bytes : kQ6Bytes);
            g.ncol0 = kvd;
            g.N = kvd;
            split_plan(g.N, g.nb, gx, sp, bps);
            g.bps = bps;
            rc = chk(L.v_type == kFmtQ4 ? launch_gemm_mb<kFmtQ4, false>(g, mb, gx, sp, st)
                                        : launch_gemm_mb<kFmtQ6, false>(g, mb, gx, sp, st),
                     "v projection");
            if (rc) return rc;
            hipLaunchKernelGGL(k_pf_v_epi, dim3((kvd + 255) / 256, M), dim3(256), 0, st, pf->part, sp,
                               uint32_t(kPfMaxM), kvd, L.vb, p0, vc);
            if ((rc = chk(hipGetLastError(), "v epilogue"))) return rc;
            // attention -> x
            launch_attn(hpk, dim3(M, d.kv_heads), st, pf->q, kc, vc, d.kv_heads, p0, scale, pf->x, H);
            if ((rc = chk(hipGetLastError(), "prefill attention"))) return rc;
            // o + residual
            g.w0 = g.w1 = L.o;
            g.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            g.ncol0 = H;
            g.N = H;
            split_plan(g.N, g.nb, gx, sp, bps);
            g.bps = bps;
            if ((rc = chk(launch_gemm_mb<kFmtQ4, false>(g, mb, gx, sp, st), "o projection"))) return rc;
            hipLaunchKernelGGL(k_pf_res_epi, dim3((H + 255) / 256, M), dim3(256), 0, st, pf->part, sp,
                               uint32_t(kPfMaxM), H, pf->h);
            if ((rc = chk(hipGetLastError(), "o residual"))) return rc;
            // ffn norm, gate/up + SwiGLU -> xs
            hipLaunchKernelGGL(k_pf_rmsnorm, dim3(M), dim3(256), 0, st, pf->h, H, L.ffn_norm, d.rms_eps, pf->x, H);
            if ((rc = chk(hipGetLastError(), "ffn norm"))) return rc;
            PfGemm u = g;
            u.w0 = L.gate;
            u.w1 = L.up;
            u.row_bytes = uint64_t(g.nb) * kQ4Bytes;
            u.N = F;
            u.ncol0 = F;
            u.bps = g.nb;
            u.s = pf->xs;
            u.lds_out = F;
            if ((rc = chk(launch_gemm_mb<kFmtQ4, true>(u, mb, (F + 63) / 64, 1, st), "gate/up"))) return rc;
            // down + residual
            PfGemm dn = g;
            dn.x = pf->xs;
            dn.ldx = F;
            dn.nb = F / kQK;
            dn.w0 = dn.w1 = L.down;
            dn.row_bytes = uint64_t(dn.nb) * (L.down_type == kFmtQ4 ? kQ4Bytes : kQ6Bytes);
            dn.ncol0 = H;
            dn.N = H;
            split_plan(dn.N, dn.nb, gx, sp, bps);
            dn.bps = bps;
            rc = chk(L.down_type == kFmtQ4 ? launch_gemm_mb<kFmtQ4, false>(dn, mb, gx, sp, st)
                                           : launch_gemm_mb<kFmtQ6, false>(dn, mb, gx, sp, st),
                     "down projection");
            if (rc) return rc;
            hipLaunchKernelGGL(k_pf_res_epi, dim3((H + 255) / 256, M), dim3(256), 0, st, pf->part, sp,
                               uint32_t(kPfMaxM), H, pf->h);
            if ((rc = chk(hipGetLastError(), "down residual"))) return rc;
        }
        if (pass + 1 == passes) {
            if ((rc = launch_lm_head(S, pf->h + uint64_t(M - 1) * H, logits, st))) return rc;
            nk += 2;
        }
    }
    pf->kernels = nk;
    S->prefill_kernels = nk;
    return ARC_OK;
}

}  // namespace arc
