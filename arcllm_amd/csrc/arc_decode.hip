// arc_decode.hip -- the single-token greedy decode step of a Qwen2.5-shaped
// model on gfx950, and its model/session C ABI (include/arcllm_hip.h).
//
// One decode step (src/arcllm_v1_runtime.cpp:371-421 restated as 4 launches
// per layer + 1 instead of 16 dispatches per layer + a host argmax):
//   per layer  [attn RMSNorm + q/k GEMV + bias + RoPE + k -> fp16 cache  k_qkv<v format>
//               and v GEMV + bias -> fp16 cache, one launch; layer 0
//               decodes the token's embedding row while staging x]
//              [cached GQA: chunk workgroups + last-arriver merge, and   k_attn_o
//               the o GEMV + residual, whose workgroups wait for the
//               attention's output (two launches, k_attn and
//               k_gemv<Q4,EPI_PLAIN>, when tuning asks for other shapes)]
//              [ffn RMSNorm + gate/up GEMV + SwiGLU]                     k_gemv<Q4,EPI_SWIGLU>
//              [down GEMV + residual]                                    k_gemv<down,EPI_PLAIN>
//   head       [output RMSNorm + LM head + argmax; the last workgroup
//               picks the token and advances the control block]         k_gemv<Q6,EPI_ARGMAX>
// The position and token live in a device control block, so the step is
// captured once as a hipGraph and replayed per token.
#include "arc_gemv.hpp"
#include "arc_session.hpp"

#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <vector>

namespace arc {

// ----------------------------------------------------------------- kernels
struct AttnParams {
    const float* q;           // [q_heads*128], RoPE applied
    const _Float16* kc;       // this layer's K cache [max_ctx][kv_heads*128]
    const _Float16* vc;       // this layer's V cache
    float* out;               // [q_heads*128]
    float* po;                // split partials o: [kv_heads][kMaxSplits][hpk][128]
    float* pml;               // split partials (m, l): [kv_heads][kMaxSplits][hpk][2]
    uint32_t* counter;        // [kv_heads] arrival counters, zero between launches
    const DecodeCtl* ctl;
    uint32_t kv_heads, hpk;
    uint32_t max_ctx;         // cache rows per layer (loads are clamped to it)
    uint32_t min_cps;         // chunks per split at least (>= 1)
    float scale;
    uint32_t* done;           // in the launch fused with the o projection: kDoneCopies copies of a
                              // counter raised once per kv head when its output is written (past the L2)
    uint32_t withhold;        // test of the bounded wait: nonzero = the attention never raises `done`
};

// Split plan of one decode position over T cached positions: chunks of
// `chunk` positions (16 per wave of the workgroup), each split (workgroup)
// taking a run of cps consecutive chunks in turn, at least min_cps and at
// most kMaxSplits splits per kv head.
struct AttnSplit {
    uint32_t nch, cps, nsplit;
};
__device__ __host__ inline AttnSplit attn_split(uint32_t T, uint32_t chunk, uint32_t min_cps)
{
    const uint32_t nch = (T + chunk - 1) / chunk;
    uint32_t cps = (nch + kMaxSplits - 1) / kMaxSplits;
    if (cps < min_cps) cps = min_cps;
    return AttnSplit{nch, cps, (nch + cps - 1) / cps};
}

// k_attn: W waves per workgroup; wave w takes positions 16w .. 16w+15 of
// every chunk of 16 W positions, with its own running softmax state.
constexpr int kAttnTile = 16;  // positions per wave and chunk (the MFMA rows)
static_assert(kChunk == 4 * kAttnTile, "the session's chunk: 4 waves of 16 positions");
static_assert(kHeadDim == 2 * kWave, "V sum: one dim pair per lane");
static_assert(kMaxSplits <= kWave, "the merge takes one split per lane");
constexpr int kAttnMergeBatch = 16;  // split outputs loaded per batch in the merge
constexpr int kCpolSc1 = 16;         // buffer-load cache policy bit sc1 (device-coherent read)
// Splits that load their first chunk before reading the position: with 4
// waves, splits 0..7 take part in every plan above 448 positions; with 8,
// splits 0..3 (plans above 384 positions).
template <int W>
constexpr uint32_t attn_early_splits() { return W == 4 ? 8u : 4u; }

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Cached GQA of one new position (flash decoding in one launch).  Workgroup
// (s, g) covers the chunks of split s for kv head g and all HPK query heads
// of that kv head.  Wave w owns positions 16w .. 16w+15 of each chunk and
// keeps its own running (max, sum, o) per head, so the chunk loop has no
// barrier:
//  scores  S^T = K Q^T on v_mfma_f32_16x16x32_f16.  A = K rows straight from
//          the cache (lane -> position lane%16; K slot (lane/16, j) of step
//          ks = dim 32*(lane/16) + 8*ks + j, so a lane's operand is 64
//          contiguous bytes of its row), B = Q^T (lane -> query head
//          lane%16, zero past HPK) split into fp16 hi + lo parts (q = hi + lo
//          to 2^-22 relative; the K*hi and K*lo products are exact in the
//          fp32 accumulator).  D: lane -> head lane%16, positions
//          4*(lane/16) + i.
//  softmax tile maximum per head (row exchanges), weights e^(x - max) to
//          the wave's LDS rows [position][head], read back by the same wave
//          (LDS operations of a wave complete in order).
//  V sum   lane -> dim pair (2 lane, 2 lane + 1), V read as fp16 straight
//          from the cache, one 256-byte row per load; o[head] += e * v on
//          v_fma_mix (fp32 weights, exact products).
// The next chunk's K and V loads are in flight while one is used (splits
// 0..7 issue their first chunk's before the position is read: rows clamped
// to the cache, masked later).  At the split's end the 4 waves' states are
// combined through LDS in wave order.  A single split writes the output;
// otherwise each split's (m, l, o) goes to memory past the L2 (st_agent) and
// the last workgroup of kv head g to arrive merges the splits in split order:
// M = max m_s, f_s = e^(m_s - M), L = sum l_s f_s, out = sum o_s (f_s / L).
// Every reduction has a fixed order, so the result does not depend on which
// workgroup arrives last.
// Semantics: src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1177-1212,
// shaders/p7_attention_kv_online.comp (kv head = q head / (q_heads/kv_heads)).
// Workgroup (s, g) of the attention; FUSED: the launch also runs the o
// projection, which waits for a.done to count every kv head.
template <int HPK, int W, bool FUSED>
__device__ __forceinline__ void attn_body(const AttnParams& a, const uint32_t s, const uint32_t g)
{
    constexpr int kC = W * kAttnTile;  // positions per chunk
    static_assert(W == 4 || W == 8, "4 or 8 waves per workgroup");
    __shared__ __align__(16) float pw[W][kAttnTile][8];  // per wave: weights [position][head]
    __shared__ __align__(16) float fow[W][8];            // per wave: rescale per head
    __shared__ float mw[W][8], lw[W][8];                 // split end: wave (max, sum) per head
    __shared__ __align__(16) float ow[W][HPK][kHeadDim];  // split end: rescaled wave o per head
    __shared__ float fw[kMaxSplits][HPK];                // merge: split weights
    __shared__ uint32_t flag;

    const uint64_t kvd = uint64_t(a.kv_heads) * kHeadDim;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r16 = lane & 15, grp = lane >> 4;  // scores: MFMA row/column, K-slot group

    const _Float16* kb = a.kc + g * kHeadDim + 32 * grp;
    const _Float16* vb = a.vc + g * kHeadDim + 2 * lane;
    uint4 kr[4];            // K row t0 + 16w + r16, dims 32grp .. 32grp+31
    uint32_t vr[kAttnTile];  // V rows t0 + 16w + j, dims 2 lane, 2 lane + 1
    auto load = [&](uint32_t t0, uint32_t tmax) {
        const uint32_t tw = t0 + kAttnTile * w;
        const uint4* kp = reinterpret_cast<const uint4*>(kb + uint64_t(min(tw + r16, tmax)) * kvd);
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = kp[i];
#pragma unroll
        for (int j = 0; j < kAttnTile; ++j)
            vr[j] = *reinterpret_cast<const uint32_t*>(vb + uint64_t(min(tw + j, tmax)) * kvd);
    };

    // Splits 0..7 take part in every plan above 448 positions: they issue
    // their first chunk's loads before the position is known.  The others
    // read the position first, so the splits a short context leaves idle
    // read nothing.
    const bool early = s < attn_early_splits<W>();
    if (early) load(s * kC, a.max_ctx - 1);  // chunk s: the first chunk of split s when cps = 1
    float4 qv[8];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + (uint64_t(g) * HPK + min(r16, HPK - 1)) * kHeadDim + 32 * grp);
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[i] = qp[i];
    }
    const uint32_t T = min(a.ctl->pos + 1u, a.max_ctx);  // device memory: never past the cache
    const AttnSplit sp = attn_split(T, kC, a.min_cps);
    if (s >= sp.nsplit) return;  // whole workgroup: not part of this position's plan
    const uint32_t c0 = s * sp.cps, c1 = min(c0 + sp.cps, sp.nch);
    if (sp.cps != 1 || !early) load(c0 * kC, T - 1);

    half8_t qh[4], ql[4];  // B operand: head r16 (zero past HPK), dims 32grp + 8ks .. +7
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const float f[8] = {qv[2 * ks].x, qv[2 * ks].y, qv[2 * ks].z, qv[2 * ks].w,
                            qv[2 * ks + 1].x, qv[2 * ks + 1].y, qv[2 * ks + 1].z, qv[2 * ks + 1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x = r16 < HPK ? f[j] : 0.0f;
            const _Float16 hi = static_cast<_Float16>(x);
            qh[ks][j] = hi;
            ql[ks][j] = static_cast<_Float16>(x - static_cast<float>(hi));
        }
    }

    float o0[HPK], o1[HPK];  // this wave's V sums: head h, dims 2 lane, 2 lane + 1
#pragma unroll
    for (int h = 0; h < HPK; ++h) o0[h] = o1[h] = 0.0f;
    float M = -INFINITY, Ls = 0.0f;  // head r16: running max, this lane's share of the running sum
    float (*pwr)[8] = pw[w];
    for (uint32_t c = c0; c < c1; ++c) {
        const uint32_t tw = c * kC + kAttnTile * w;
        uint4 kc[4];
        uint32_t vc[kAttnTile];
#pragma unroll
        for (int i = 0; i < 4; ++i) kc[i] = kr[i];
        // rows at or past T (clamped or early loads: stale or never written)
        // enter as zeros, so their weight 0 never multiplies an inf or NaN
#pragma unroll
        for (int j = 0; j < kAttnTile; ++j) vc[j] = tw + j < T ? vr[j] : 0u;
        if (c + 1 < c1) load((c + 1) * kC, T - 1);

        f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const half8_t kf = __builtin_bit_cast(half8_t, kc[ks]);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], d, 0, 0, 0);
        }
        float x[4], m = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = tw + 4u * grp + i < T ? d[i] * a.scale : -INFINITY;
            m = fmaxf(m, x[i]);
        }
        m = xor_max<16>(m);
        m = xor_max<32>(m);
        const float Mn = fmaxf(M, m);
        const float Mr = Mn == -INFINITY ? 0.0f : Mn;  // a wave may not have seen a position < T yet
        const float fo = expf(M - Mr);                 // M = -inf: 0
        float es = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e = expf(x[i] - Mr);  // masked: e^-inf = 0
            es += e;
            if (r16 < HPK) pwr[4 * grp + i][r16] = e;
        }
        Ls = Ls * fo + es;
        M = Mn;
        if (grp == 0 && r16 < HPK) fow[w][r16] = fo;

        const float4 f0 = *reinterpret_cast<const float4*>(fow[w]), f1 = *reinterpret_cast<const float4*>(fow[w] + 4);
        const float fh[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
        for (int h = 0; h < HPK; ++h) {
            o0[h] *= fh[h];
            o1[h] *= fh[h];
        }
#pragma unroll
        for (int j = 0; j < kAttnTile; ++j) {
            const float4 p0 = *reinterpret_cast<const float4*>(pwr[j]);
            const float4 p1 = *reinterpret_cast<const float4*>(pwr[j] + 4);
            const float ph[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int h = 0; h < HPK; ++h) {
                o0[h] = fmix(vc[j], false, ph[h], o0[h]);
                o1[h] = fmix(vc[j], true, ph[h], o1[h]);
            }
        }
    }

    // the waves' states combined in LDS: the split's max per head, each wave's
    // o rescaled by e^(m_w - M), then per (head, dim quad) the waves in order
    Ls = xor_sum<16>(Ls);
    Ls = xor_sum<32>(Ls);
    if (grp == 0 && r16 < HPK) {
        mw[w][r16] = M;
        lw[w][r16] = Ls;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < HPK; ++h) {
        float Mh = -INFINITY;
#pragma unroll
        for (int v = 0; v < W; ++v) Mh = fmaxf(Mh, mw[v][h]);  // finite: the split holds a position < T
        const float f = expf(mw[w][h] - Mh);                   // a wave without positions < T: e^-inf = 0
        o0[h] *= f;
        o1[h] *= f;
    }
#pragma unroll
    for (int h = 0; h < HPK; ++h) reinterpret_cast<float2*>(ow[w][h])[lane] = make_float2(o0[h], o1[h]);
    __syncthreads();

    const bool owner = tid < HPK * (kHeadDim / 4);  // thread -> head hh, dims 4 dq4 .. +3
    const uint32_t hh = min(uint32_t(tid) / (kHeadDim / 4), uint32_t(HPK - 1)), dq4 = uint32_t(tid) % (kHeadDim / 4);
    float Msp = -INFINITY, Lsp = 0.0f;
    float4 osp = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    {
#pragma unroll
        for (int v = 0; v < W; ++v) Msp = fmaxf(Msp, mw[v][hh]);
#pragma unroll
        for (int v = 0; v < W; ++v) Lsp = __builtin_fmaf(lw[v][hh], expf(mw[v][hh] - Msp), Lsp);
#pragma unroll
        for (int v = 0; v < W; ++v) {
            const float4 ov = reinterpret_cast<const float4*>(ow[v][hh])[dq4];
            osp.x += ov.x;
            osp.y += ov.y;
            osp.z += ov.z;
            osp.w += ov.w;
        }
    }

    float* out = a.out + uint64_t(g) * HPK * kHeadDim;
    // the kv head's output; fused: written past the L2 (sc1) for the o
    // projection's workgroups, then counted in
    auto store_out = [&](float4 r) {
        if constexpr (FUSED) {
            const __amdgpu_buffer_rsrc_t ors =
                __builtin_amdgcn_make_buffer_rsrc(out, 0, int(HPK * kHeadDim * 4), 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, r), ors, (hh * kHeadDim + 4 * dq4) * 4u,
                                                   0, kCpolSc1);
        } else {
            reinterpret_cast<float4*>(out + hh * kHeadDim)[dq4] = r;
        }
    };
    const uint64_t base = uint64_t(g) * kMaxSplits;
    if (sp.nsplit == 1) {
        if (owner) {
            const float li = 1.0f / Lsp;
            store_out(make_float4(osp.x * li, osp.y * li, osp.z * li, osp.w * li));
        }
        if constexpr (FUSED)
            if (!a.withhold) signal_done(a.done, kDoneCopies, kDoneStride);
        return;
    }
    // this split's partials, written past the L2 for the merging workgroup
    // (16-byte buffer stores with the cache policy of st_agent)
    if (owner) {
        const __amdgpu_buffer_rsrc_t pws = __builtin_amdgcn_make_buffer_rsrc(
            a.po + (base + s) * HPK * kHeadDim, 0, int(HPK * kHeadDim * 4), 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, osp), pws, (hh * kHeadDim + 4 * dq4) * 4u, 0,
                                               kCpolSc1);
        if (dq4 == 0) {
            st_agent(a.pml + ((base + s) * HPK + hh) * 2, Msp);
            st_agent(a.pml + ((base + s) * HPK + hh) * 2 + 1, Lsp);
        }
    }
    if (!arrive_last(a.counter + g, sp.nsplit, &flag)) return;

    // merge (last workgroup of kv head g).  Wave w, lane = split: the split
    // weights w_s = e^(m_s - M) / L of heads w, w + W (M and L by wave
    // reductions) into LDS; then thread -> (head hh, dims 4dq4 .. +3) sums
    // the splits' o weighted, in split order, loads in batches of kB, two
    // batches in flight (the first two are issued right after the (m, l)
    // loads).
    const bool in = uint32_t(lane) < sp.nsplit;
    const uint32_t ss = min(uint32_t(lane), sp.nsplit - 1);
    float2 ml[2];  // at most 2 heads per wave (W >= 4)
    constexpr int kMH = (kMaxHpk + W - 1) / W;  // heads per wave in the merge
#pragma unroll
    for (int k = 0; k < kMH; ++k) {
        const uint32_t h = min(uint32_t(w + W * k), uint32_t(HPK - 1));
        ml[k] = ld_agent2(a.pml + ((base + ss) * HPK + h) * 2);
    }
    // the kv head's partials as a buffer resource: 16-byte loads with the
    // device-coherence cache policy of ld_agent (sc1: not served from a
    // possibly stale cache line)
    const float* src = a.po + base * HPK * kHeadDim;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), 0, int(kMaxSplits * HPK * kHeadDim * 4), 0x00020000);
    const uint32_t off0 = (hh * kHeadDim + 4 * dq4) * 4u;
    constexpr int kB = kAttnMergeBatch;
    float4 ova[kB], ovb[kB];  // two batches: the next one's loads in flight while one is summed
    auto fetch = [&](float4 (&ov)[kB], uint32_t s0) {
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const uint32_t off = off0 + min(s0 + u, sp.nsplit - 1) * uint32_t(HPK * kHeadDim * 4);
            ov[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kCpolSc1));
        }
    };
    if (owner) {
        fetch(ova, 0);
        if (uint32_t(kB) < sp.nsplit) fetch(ovb, kB);
    }
#pragma unroll
    for (int k = 0; k < kMH; ++k) {
        const int h = w + W * k;
        if (h < HPK) {
            const float m = in ? ml[k].x : -INFINITY;
            const float Mx = wave_max(m);
            const float f = in ? expf(m - Mx) : 0.0f;
            const float Lsum = group_sum<kWave>(in ? ml[k].y * f : 0.0f);
            fw[lane][h] = f / Lsum;  // lane < kMaxSplits = kWave
        }
    }
    __syncthreads();
    if (owner) {
        float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        auto sum = [&](const float4 (&ov)[kB], uint32_t s0) {
#pragma unroll
            for (int u = 0; u < kB; ++u)
                if (s0 + u < sp.nsplit) {
                    const float f = fw[s0 + u][hh];
                    r.x = __builtin_fmaf(ov[u].x, f, r.x);
                    r.y = __builtin_fmaf(ov[u].y, f, r.y);
                    r.z = __builtin_fmaf(ov[u].z, f, r.z);
                    r.w = __builtin_fmaf(ov[u].w, f, r.w);
                }
        };
        // batches s0 (in ova) and s0 + kB (in ovb) are in flight on entry
        for (uint32_t s0 = 0; s0 < sp.nsplit; s0 += 2 * kB) {
            sum(ova, s0);
            if (s0 + 2 * kB < sp.nsplit) fetch(ova, s0 + 2 * kB);
            if (s0 + kB < sp.nsplit) {
                sum(ovb, s0 + kB);
                if (s0 + 3 * kB < sp.nsplit) fetch(ovb, s0 + 3 * kB);
            }
        }
        store_out(r);
    }
    if constexpr (FUSED)
        if (!a.withhold) signal_done(a.done, kDoneCopies, kDoneStride);
}

template <int HPK, int W>
__global__ __launch_bounds__(W * kWave) void k_attn(AttnParams a)
{
    attn_body<HPK, W, false>(a, blockIdx.x, blockIdx.y);
}

// Attention and the o projection in one launch.  Workgroups [0, n_attn) are
// the attention's (split b % kMaxSplits, kv head b / kMaxSplits), the rest
// the o GEMV's: those load their first weights, wait until every kv head's
// output is written (a.done = kv heads, each workgroup polling its own copy
// of the counter), then stage it as x.  The o workgroups come after every
// attention workgroup in dispatch order and the grid fits on the device at
// once, so a waiting workgroup never holds back one it waits for.  The next
// launch (the ffn gate/up) zeroes the done copies; a wait that gives up
// counts in ctl->waits_expired, which the host reports as an error.
struct AttnOWait {
    static constexpr bool kWaits = true;
    const uint32_t* done;
    uint32_t n;
    DecodeCtl* ctl;
    __device__ void operator()() const
    {
        __shared__ uint32_t flag;
        const bool ok = wait_count(done, n, &flag);
        if (threadIdx.x == 0 && !ok)
            __hip_atomic_fetch_add(&ctl->waits_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
};
constexpr int kAttnOBs = 8, kAttnORpl = 1;  // o projection layout in the fused launch (4 waves)

template <int HPK>
__global__ __launch_bounds__(4 * kWave) void k_attn_o(AttnParams a, GemvParams o, uint32_t n_attn)
{
    const uint32_t b = blockIdx.x;
    if (b < n_attn) {
        attn_body<HPK, 4, true>(a, b % kMaxSplits, b / kMaxSplits);
        return;
    }
    const AttnOWait hook{a.done + ((b - n_attn) % kDoneCopies) * kDoneStride, a.kv_heads, o.ctl};
    gemv_body<kFmtQ4, kAttnOBs, kAttnORpl, EPI_PLAIN, 4, AttnOWait>(o, b - n_attn, gridDim.x - n_attn, hook);
}

// Attention launch shape (tuning): waves per workgroup and the least chunks
// per split.  Measured on MI355X (7B shape, 28 q / 4 kv heads): 4 waves,
// one chunk per split 10.2 / 13.2 / 17.9 us at 512 / 2048 / 4096 positions,
// 8 waves 11.3 / 12.4 / 14.9 us, 16 waves 17.7 / 18.2 / 18.8 us, two or
// more chunks per split slower at every length; decode tokens/s with 8
// waves -1.8% at 512 positions, +1.1% at 2048, equal at 4096.  Automatic:
// 4 waves, one chunk per split.
inline thread_local int g_attn_waves = 0;    // 0: automatic
inline thread_local int g_attn_min_cps = 0;  // 0: automatic

// Per-launch layout overrides of the decode step's GEMVs (tuning), read when
// a step is captured: 0 the o projection, 1 the fused gate/up, 2 the down
// projection, 3 the LM head.  bs = 0 keeps the step's own layout, waves = 0
// its own waves per workgroup.
enum DecKind { kDecO = 0, kDecGateUp = 1, kDecDown = 2, kDecLmHead = 3, kDecKinds = 4 };
inline thread_local Cfg g_dec_cfg[kDecKinds] = {};

static Cfg dec_cfg(int kind, Cfg c)
{
    const Cfg& o = g_dec_cfg[kind];
    if (o.bs) {
        c.bs = o.bs;
        c.rpl = o.rpl;
    }
    if (o.waves) c.waves = o.waves;
    return c;
}

template <int HPK, int W>
static void launch_attn_hpk(const AttnParams& ap, uint32_t kv_heads, hipStream_t st)
{
    if (g_dry_run) return;
    hipLaunchKernelGGL((k_attn<HPK, W>), dim3(kMaxSplits, kv_heads), dim3(W * kWave), 0, st, ap);
}

template <int W>
static void launch_attn_w(const AttnParams& ap, uint32_t kv_heads, hipStream_t st)
{
    switch (ap.hpk) {
    case 1: launch_attn_hpk<1, W>(ap, kv_heads, st); break;
    case 2: launch_attn_hpk<2, W>(ap, kv_heads, st); break;
    case 3: launch_attn_hpk<3, W>(ap, kv_heads, st); break;
    case 4: launch_attn_hpk<4, W>(ap, kv_heads, st); break;
    case 5: launch_attn_hpk<5, W>(ap, kv_heads, st); break;
    case 6: launch_attn_hpk<6, W>(ap, kv_heads, st); break;
    case 7: launch_attn_hpk<7, W>(ap, kv_heads, st); break;
    default: launch_attn_hpk<8, W>(ap, kv_heads, st); break;
    }
}

// Sets ap.min_cps and launches (grid: kMaxSplits x kv heads; workgroups past
// the position's plan return at once).
static void launch_attn(AttnParams ap, uint32_t kv_heads, hipStream_t st)
{
    const int waves = g_attn_waves ? g_attn_waves : 4;
    ap.min_cps = g_attn_min_cps > 0 ? uint32_t(g_attn_min_cps) : 1u;
    if (waves == 8)
        launch_attn_w<8>(ap, kv_heads, st);
    else
        launch_attn_w<4>(ap, kv_heads, st);
}

// Attention + o projection in one launch (k_attn_o): 1 automatic, 0 two
// launches (tuning and comparison).
inline thread_local int g_fuse_attn_o = 1;  // 2: fused, the attention withholding its signal (test)

template <int HPK>
static hipError_t launch_attn_o_hpk(const AttnParams& ap, GemvParams o, hipStream_t st, bool* done)
{
    *done = false;
    const Cfg c{kAttnOBs, kAttnORpl, 4};
    o.ntiles = (o.rows + tile_rows(c) - 1) / tile_rows(c);
    const size_t lds = size_t(o.panel) * kXBlk * sizeof(float);
    static int occ[kPanel + 1] = {};
    if (!occ[o.panel]) {
        int nb = 0;
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_o<HPK>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_attn_o<HPK>, 4 * kWave, lds) != hipSuccess || nb < 1)
            nb = 1;
        occ[o.panel] = nb;
    }
    // every workgroup resident at once: the o part gets what the attention part leaves
    const uint64_t n_attn = uint64_t(kMaxSplits) * ap.kv_heads;
    const uint64_t resident = uint64_t(occ[o.panel]) * cu_count();
    if (resident <= n_attn) return hipSuccess;  // not done: the caller launches the two kernels
    const uint64_t n_o = std::min<uint64_t>(resident - n_attn, (o.ntiles + 3) / 4);
    *done = true;
    if (g_dry_run) return hipSuccess;
    hipLaunchKernelGGL(k_attn_o<HPK>, dim3(uint32_t(n_attn + n_o)), dim3(4 * kWave), lds, st, ap, o,
                       uint32_t(n_attn));
    return hipGetLastError();
}

// Launches attention + o fused when the step's automatic shapes allow it
// (4-wave attention, no layout override of the o projection); *done tells
// whether it did.  The launch after it must zero ap.done's copies
// (GemvParams::clear_done).
static hipError_t launch_attn_o(AttnParams ap, const GemvParams& o, hipStream_t st, bool* done)
{
    *done = false;
    if (!g_fuse_attn_o || (g_attn_waves && g_attn_waves != 4) || g_force_waves || g_force.bs ||
        g_dec_cfg[kDecO].bs || g_dec_cfg[kDecO].waves)
        return hipSuccess;
    ap.min_cps = g_attn_min_cps > 0 ? uint32_t(g_attn_min_cps) : 1u;
    ap.withhold = g_fuse_attn_o == 2 ? 1u : 0u;
    switch (ap.hpk) {
    case 1: return launch_attn_o_hpk<1>(ap, o, st, done);
    case 2: return launch_attn_o_hpk<2>(ap, o, st, done);
    case 3: return launch_attn_o_hpk<3>(ap, o, st, done);
    case 4: return launch_attn_o_hpk<4>(ap, o, st, done);
    case 5: return launch_attn_o_hpk<5>(ap, o, st, done);
    case 6: return launch_attn_o_hpk<6>(ap, o, st, done);
    case 7: return launch_attn_o_hpk<7>(ap, o, st, done);
    default: return launch_attn_o_hpk<8>(ap, o, st, done);
    }
}

static_assert(kMaxHpk == 8, "launch_attn instantiates 1..8");
static_assert(kMaxHpk <= 16, "query heads of a kv head fit the 16 MFMA columns");
static_assert(kMaxHpk * (kHeadDim / 4) <= 4 * kWave && kMaxHpk <= 2 * 4,
              "merge (4 waves): one thread per (head, dim quad); at most two heads per wave for the split weights");

}  // namespace arc

namespace arc {

// q/k and v projections in one launch: workgroups [0, gqk) run the q/k GEMV
// (bias, RoPE, K store), the others the v GEMV (bias, V store).  Both read
// the same attention-normed x and stage it in their own format's layout; the
// role is uniform per workgroup.  One launch instead of two saves the v
// projection's whole fixed cost (x staging, first-load latency, launch),
// which is most of its time: its weights are 1.5 MB.
// Quads per q/k row (2 rows per lane: RoPE pairs) and per v row.  8 and 8
// measured fastest in the decode step (7B shape, 564 tokens/s at T = 512;
// 16 and 16, tuned when q/k and v were separate launches, 541; 8 and 16, 562;
// 4 and 4, 546).
#ifndef ARC_QK_BS
#define ARC_QK_BS 8
#endif
#ifndef ARC_V_BS
#define ARC_V_BS 8
#endif
// Waves per workgroup: 4 (320 workgroups for the 7B shape, every CU busy)
// measured 0.3-0.5% more decode tokens/s than 8 (160 workgroups).
#ifndef ARC_QKV_WAVES
#define ARC_QKV_WAVES 4
#endif
constexpr int kQkvWaves = ARC_QKV_WAVES;  // waves per q/k/v workgroup

template <int VFMT>
__global__ __launch_bounds__(kQkvWaves * kWave) void k_qkv(GemvParams qk, GemvParams v, uint32_t gqk)
{
    if (blockIdx.x < gqk)
        gemv_body<kFmtQ4, ARC_QK_BS, 2, EPI_QKROPE, kQkvWaves>(qk, blockIdx.x, gqk);
    else
        gemv_body<VFMT, ARC_V_BS, 1, EPI_VSTORE, kQkvWaves>(v, blockIdx.x - gqk, gridDim.x - gqk);
}

template <int VFMT>
static hipError_t launch_qkv(GemvParams qk, GemvParams v, hipStream_t st)
{
    constexpr int W = kQkvWaves;
    const Cfg cqk{ARC_QK_BS, 2, W}, cv{ARC_V_BS, 1, W};
    qk.ntiles = (qk.rows + tile_rows(cqk) - 1) / tile_rows(cqk);
    v.ntiles = (v.rows + tile_rows(cv) - 1) / tile_rows(cv);
    const size_t lds = size_t(std::max(qk.panel, v.panel)) * kXBlk * sizeof(float);
    static int occ[kPanel + 1] = {};  // resident workgroups per CU, by panel (the hidden size in blocks)
    const uint32_t slot = std::max(qk.panel, v.panel);
    if (!occ[slot]) {
        int nb = 0;
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_qkv<VFMT>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_qkv<VFMT>, W * kWave, lds) != hipSuccess || nb < 1)
            nb = 1;
        occ[slot] = nb;
    }
    const uint64_t resident = uint64_t(occ[slot]) * cu_count();
    // each part gets at most one wave tile per wave and at most the resident count
    const uint32_t gqk = uint32_t(std::min<uint64_t>(resident, (qk.ntiles + W - 1) / W));
    const uint32_t gv = uint32_t(std::min<uint64_t>(resident, (v.ntiles + W - 1) / W));
    if (g_dry_run) return hipSuccess;
    hipLaunchKernelGGL(k_qkv<VFMT>, dim3(gqk + gv), dim3(W * kWave), lds, st, qk, v, gqk);
    return hipGetLastError();
}

static uint64_t packed_bytes(int qtype, uint32_t rows, uint32_t K)
{
    return uint64_t(rows) * (K / kQK) * (qtype == kFmtQ4 ? kQ4Bytes : kQ6Bytes);
}

static int dims_ok(const arc_model_dims& d)
{
    if (d.hidden == 0 || d.hidden % kQK || d.ffn == 0 || d.ffn % kQK || d.head_dim != kHeadDim || d.q_heads == 0 ||
        d.kv_heads == 0 || d.kv_heads > uint32_t(kCounterLmHead - kCounterAttn) || d.q_heads % d.kv_heads ||
        d.q_heads / d.kv_heads > kMaxHpk ||
        d.q_heads * kHeadDim != d.hidden || d.vocab == 0 || d.layers == 0 || d.layers > ARC_MAX_LAYERS)
        return set_error(ARC_ERR_UNSUPPORTED,
                         "unsupported model dims (hidden %u, heads %u/%u, head_dim %u, ffn %u, vocab %u, layers %u)",
                         d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.ffn, d.vocab, d.layers);
    if (d.hidden / kQK > uint32_t(kPanel) || d.ffn / kQK > uint32_t(kPanel))
        return set_error(ARC_ERR_UNSUPPORTED, "hidden and ffn must be <= %d", kPanel * kQK);
    // Q6_K tensors (held padded) are read through 32-bit byte offsets
    if (uint64_t(d.vocab) * (d.hidden / kQK) * kQ6PBytes > 0xfffffff0ull)
        return set_error(ARC_ERR_UNSUPPORTED, "output tensor of %u x %u exceeds 4 GiB", d.vocab, d.hidden);
    for (uint32_t l = 0; l < d.layers; ++l)
        if ((d.v_type[l] != kFmtQ4 && d.v_type[l] != kFmtQ6) || (d.down_type[l] != kFmtQ4 && d.down_type[l] != kFmtQ6))
            return set_error(ARC_ERR_UNSUPPORTED, "layer %u: attn_v / ffn_down must be Q4_K or Q6_K", l);
    return ARC_OK;
}

// Output RMSNorm + LM head + argmax of the hidden row x in one launch: the
// last workgroup to arrive picks the token and advances the control block.
int launch_lm_head(arc_session* S, const float* x, bool logits, hipStream_t st)
{
    const arc_model* M = S->model;
    const arc_model_dims& d = M->dims;
    const uint32_t H = d.hidden;
    GemvParams p = make_params(kFmtQ6P, M->out, nullptr, d.vocab, H, x);
    p.flags = F_NORM | F_ARGNEXT;
    p.normw = M->out_norm;
    p.eps = d.rms_eps;
    p.y = logits ? S->logits : nullptr;
    p.best = S->best;
    p.counter = S->counters + kCounterLmHead;
    p.ctl = S->ctl;
    p.out_tokens = S->out_tokens;
    p.out_cap = S->out_cap;
    const Cfg c = dec_cfg(kDecLmHead, choose_cfg(EPI_ARGMAX, d.vocab, H / kQK, 1));
    uint32_t gx = 0;
    const bool dry = g_dry_run;
    g_dry_run = true;  // size the grid first: every workgroup needs a partials slot
    int rc = check_hip(launch_gemv_epi(EPI_ARGMAX, kFmtQ6P, c, p, 1, st, &gx), "lm head");
    g_dry_run = dry;
    if (rc) return rc;
    if (gx > S->best_cap) return set_error(ARC_ERR_UNSUPPORTED, "internal: argmax grid %u > %u", gx, S->best_cap);
    return check_hip(launch_gemv_epi(EPI_ARGMAX, kFmtQ6P, c, p, 1, st, &gx), "lm head");
}

// Launch one decode step on the session stream (captured into a graph by the
// caller, or run eagerly).  Returns the number of kernels launched.
static int launch_step(arc_session* S, bool logits, uint32_t* nkernels)
{
    arc_model* M = S->model;
    const arc_model_dims& d = M->dims;
    hipStream_t st = S->stream;
    const uint32_t H = d.hidden, KVD = d.kv_heads * kHeadDim, F = d.ffn;
    uint32_t n = 0;
    int rc = 0;
    auto chk = [&](hipError_t e, const char* what) { ++n; return check_hip(e, what); };

    for (uint32_t l = 0; l < d.layers; ++l) {
        const Layer& L = M->layers[l];
        _Float16* kc = S->kcache + uint64_t(l) * S->max_ctx * KVD;
        _Float16* vc = S->vcache + uint64_t(l) * S->max_ctx * KVD;

        // q/k projection + RoPE + K store; layer 0 decodes the token's
        // embedding row as its x and writes it to h (the residual)
        GemvParams p = make_params(kFmtQ4, L.q, L.k, H + KVD, H, S->h);
        p.flags = F_NORM;
        p.normw = L.attn_norm;
        p.eps = d.rms_eps;
        p.bias = L.qb;
        p.bias2 = L.kb;
        p.row_split = H;
        p.kv_dim = KVD;
        p.cache = kc;
        p.rope = S->rope;
        p.ctl = S->ctl;
        p.ctx_rows = S->max_ctx;
        p.y = S->q;

        // v projection + V store, in the same launch
        GemvParams pv = make_params(L.v_type, L.v, nullptr, KVD, H, S->h);
        pv.flags = F_NORM;
        pv.normw = L.attn_norm;
        pv.eps = d.rms_eps;
        pv.bias = L.vb;
        pv.kv_dim = KVD;
        pv.cache = vc;
        pv.ctl = S->ctl;
        pv.ctx_rows = S->max_ctx;
        if (l == 0) {
            // x is the decoded embedding row; workgroup 0 writes it to h.  The
            // branch-free x pre-loads still read p.x: point it at a buffer
            // this launch does not write (the values are discarded).
            p.flags |= F_EMBED;
            p.emb = M->emb;
            p.emb_rows = d.vocab;
            p.h_out = S->h;
            p.x = L.attn_norm;
            pv.flags |= F_EMBED;
            pv.emb = M->emb;
            pv.emb_rows = d.vocab;
            pv.x = L.attn_norm;
        }
        hipError_t e = L.v_type == kFmtQ4 ? launch_qkv<kFmtQ4>(p, pv, st) : launch_qkv<kFmtQ6P>(p, pv, st);
        if ((rc = chk(e, "q/k/v projection"))) return rc;

        // attention
        AttnParams ap{};
        ap.q = S->q;
        ap.kc = kc;
        ap.vc = vc;
        ap.out = S->attn;
        ap.po = S->apo;
        ap.pml = S->apml;
        ap.counter = S->counters + kCounterAttn;
        ap.ctl = S->ctl;
        ap.kv_heads = d.kv_heads;
        ap.hpk = d.q_heads / d.kv_heads;
        ap.max_ctx = S->max_ctx;
        ap.scale = 1.0f / std::sqrt(float(kHeadDim));
        ap.done = S->done;

        // o projection + residual: h1 = h + Wo attn
        p = make_params(kFmtQ4, L.o, nullptr, H, H, S->attn);
        p.res = S->h;
        p.y = S->h1;
        p.ctl = S->ctl;
        bool fused = false;
        if ((rc = chk(launch_attn_o(ap, p, st, &fused), "attention + o projection")))
            return rc;
        if (!fused) {
            --n;
            launch_attn(ap, d.kv_heads, st);
            if ((rc = chk(hipGetLastError(), "attention"))) return rc;
            // 4-wave workgroups for the o projection in the step (7B shape: +0.8-1.1%
            // tokens/s over the 8 the standalone choice takes for 2048+ rows)
            Cfg ocfg = choose_cfg(EPI_PLAIN, H, H / kQK, 1);
            if (!g_force_waves) ocfg.waves = 4;
            ocfg = dec_cfg(kDecO, ocfg);
            if ((rc = chk(launch_gemv_epi(EPI_PLAIN, kFmtQ4, ocfg, p, 1, st), "o projection")))
                return rc;
        }

        // ffn RMSNorm + gate/up + SwiGLU
        p = make_params(kFmtQ4, L.gate, L.up, F, H, S->h1);
        p.flags = F_NORM;
        p.normw = L.ffn_norm;
        p.eps = d.rms_eps;
        p.y = S->s;
        p.clear_done = S->done;  // the attention + o launch's done counter, for the next layer
        if ((rc = chk(launch_gemv_epi(EPI_SWIGLU, kFmtQ4, dec_cfg(kDecGateUp, choose_cfg(EPI_SWIGLU, F, H / kQK, 1)), p,
                                      1, st),
                      "gate/up")))
            return rc;

        // down + residual: h = h1 + Wd s (route B: the layer's EXEC148 image)
        const uint8_t* e148 = l < S->down_e148.size() ? S->down_e148[l] : nullptr;
        const int dfmt = e148 ? int(kFmtE148) : L.down_type;
        p = make_params(dfmt, e148 ? e148 : L.down, nullptr, H, F, S->s);
        p.res = S->h1;
        p.y = S->h;
        // padded Q6_K down: 16 quads per row, 8 waves (measured on the 7B shape,
        // 3584 x 18944: 14.9 vs 15.2 us for the automatic (8, 1); decode
        // +0.3 .. 0.6% tokens/s)
        const Cfg dcfg = dec_cfg(kDecDown, (dfmt == int(kFmtQ6P) && !g_force.bs) ? Cfg{16, 1, 8}
                                                                                  : choose_cfg(EPI_PLAIN, H, F / kQK, 1));
        if ((rc = chk(launch_gemv_epi(EPI_PLAIN, dfmt, dcfg, p, 1, st), "down projection")))
            return rc;
    }

    // output RMSNorm + LM head + argmax + next token
    if ((rc = launch_lm_head(S, S->h, logits, st))) return rc;
    n += 1;
    if (nkernels) *nkernels = n;
    return ARC_OK;
}

}  // namespace arc

using namespace arc;

extern "C" {

int arc_tune_decode(int kind, int bs, int rpl, int waves)
{
    if (kind < 0 || kind >= kDecKinds) return set_error(ARC_ERR_INVALID_ARGUMENT, "decode launch kind must be 0..3");
    if (waves != 0 && waves != 4 && waves != 8)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "waves per workgroup must be 0 (the step's own), 4 or 8");
    static const int ok[][2] = {{1, 1}, {1, 2}, {1, 4}, {2, 1}, {2, 2}, {2, 4}, {4, 1}, {4, 2}, {8, 1}, {8, 2}, {16, 1}};
    bool found = bs == 0;
    for (const auto& c : ok) found = found || (c[0] == bs && c[1] == rpl);
    if (!found) return set_error(ARC_ERR_INVALID_ARGUMENT, "no kernel instance for bs=%d rpl=%d", bs, rpl);
    g_dec_cfg[kind] = Cfg{bs, bs ? rpl : 0, waves};
    return ARC_OK;
}

int arc_tune_fuse_attn_o(int on)
{
    if (on < 0 || on > 2) return set_error(ARC_ERR_INVALID_ARGUMENT, "fuse_attn_o must be 0, 1 or 2");
    g_fuse_attn_o = on;
    return ARC_OK;
}

int arc_tune_attention(int waves, int min_chunks_per_split)
{
    if (waves != 0 && waves != 4 && waves != 8)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "attention waves per workgroup must be 0 (automatic), 4 or 8");
    if (min_chunks_per_split < 0 || min_chunks_per_split > kMaxChunks)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "chunks per split must be 0 (automatic) .. %d", kMaxChunks);
    g_attn_waves = waves;
    g_attn_min_cps = min_chunks_per_split;
    return ARC_OK;
}

int arc_model_dims_qwen25_7b(arc_model_dims* d)
{
    if (!d) return set_error(ARC_ERR_INVALID_ARGUMENT, "null dims");
    std::memset(d, 0, sizeof(*d));
    d->hidden = 3584;
    d->q_heads = 28;
    d->kv_heads = 4;
    d->head_dim = 128;
    d->ffn = 18944;
    d->vocab = 152064;
    d->layers = 28;
    d->rms_eps = 1e-6f;
    d->rope_theta = 1e6f;
    for (uint32_t l = 0; l < ARC_MAX_LAYERS; ++l) {
        d->v_type[l] = ARC_Q6_K;
        d->down_type[l] = ARC_Q6_K;
    }
    return ARC_OK;
}

int arc_model_tensor_info(const arc_model_dims* d, int layer, int which, int* qtype, uint32_t* rows, uint32_t* K,
                          uint64_t* bytes)
{
    if (!d || !qtype || !rows || !K || !bytes) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    int rc = dims_ok(*d);
    if (rc) return rc;
    const uint32_t H = d->hidden, KVD = d->kv_heads * kHeadDim;
    int t = 0;
    uint32_t r = 0, k = 0;
    if (layer < 0) {
        switch (which) {
        case ARC_T_TOKEN_EMBD: t = ARC_Q4_K, r = d->vocab, k = H; break;
        case ARC_T_OUTPUT: t = ARC_Q6_K, r = d->vocab, k = H; break;
        case ARC_T_OUTPUT_NORM: t = 0, r = 1, k = H; break;
        default: return set_error(ARC_ERR_INVALID_ARGUMENT, "bad global tensor %d", which);
        }
    } else {
        if (uint32_t(layer) >= d->layers) return set_error(ARC_ERR_INVALID_ARGUMENT, "layer %d out of range", layer);
        switch (which) {
        case ARC_T_ATTN_NORM: case ARC_T_FFN_NORM: t = 0, r = 1, k = H; break;
        case ARC_T_ATTN_Q: case ARC_T_ATTN_O: t = ARC_Q4_K, r = H, k = H; break;
        case ARC_T_ATTN_K: t = ARC_Q4_K, r = KVD, k = H; break;
        case ARC_T_ATTN_V: t = d->v_type[layer], r = KVD, k = H; break;
        case ARC_T_ATTN_Q_BIAS: t = 0, r = 1, k = H; break;
        case ARC_T_ATTN_K_BIAS: case ARC_T_ATTN_V_BIAS: t = 0, r = 1, k = KVD; break;
        case ARC_T_FFN_GATE: case ARC_T_FFN_UP: t = ARC_Q4_K, r = d->ffn, k = H; break;
        case ARC_T_FFN_DOWN: t = d->down_type[layer], r = H, k = d->ffn; break;
        default: return set_error(ARC_ERR_INVALID_ARGUMENT, "bad layer tensor %d", which);
        }
    }
    *qtype = t;
    *rows = r;
    *K = k;
    *bytes = t == 0 ? uint64_t(k) * 4 : packed_bytes(t, r, k);
    return ARC_OK;
}

int arc_model_synth_tensor(const arc_model_dims* d, uint64_t seed, int layer, int which, void* out)
{
    int qtype;
    uint32_t rows, K;
    uint64_t bytes;
    int rc = arc_model_tensor_info(d, layer, which, &qtype, &rows, &K, &bytes);
    if (rc) return rc;
    const uint64_t stream = layer < 0 ? uint64_t(which) : 100ull + 16ull * uint64_t(layer) + uint64_t(which);
    // zero-mean, small-scale init: E[d*sc*q] = E[dmin*mn] for Q4_K, so rows
    // are centred and activations stay O(1) through the layers
    if (qtype != 0) return arc_synth_packed(qtype, seed, stream, rows, K, 1e-4f, 7.5e-4f, out);
    const bool norm = which == ARC_T_OUTPUT_NORM || which == ARC_T_ATTN_NORM || which == ARC_T_FFN_NORM;
    return arc_synth_normal(seed, stream, K, norm ? 1.0f : 0.0f, norm ? 0.05f : 0.1f, static_cast<float*>(out));
}

int arc_model_create(const arc_model_dims* dims, const void* const* tensors, arc_model** out)
{
    if (!dims || !tensors || !out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    int rc = dims_ok(*dims);
    if (rc) return rc;
    std::unique_ptr<arc_model> M(new (std::nothrow) arc_model);
    if (!M) return set_error(ARC_ERR_OUT_OF_MEMORY, "host allocation");
    M->dims = *dims;
    M->layers.resize(dims->layers);

    // The arena: every tensor in slot order (globals, then layer by layer),
    // 256 bytes of slack after the last (kernels read 16-byte vectors past a
    // row's end), then the EXEC148 reserve.
    // Q6_K tensors are held padded (212-byte blocks at dword boundaries, see
    // arc_q6_pad): every Q6_K GEMV of the decode step then reads its blocks
    // with aligned loads.
    struct Upload {
        const void* src;
        uint64_t bytes;          // as given (GGUF layout)
        uint64_t dev_bytes = 0;  // as held
        const void* dev = nullptr;
    };
    const size_t nt = size_t(ARC_T_GLOBAL_COUNT) + size_t(dims->layers) * ARC_T_LAYER_COUNT;
    std::vector<Upload> up(nt);
    ArenaPlan plan;
    for (size_t i = 0; i < nt; ++i) {
        const int layer = i < size_t(ARC_T_GLOBAL_COUNT) ? -1 : int((i - ARC_T_GLOBAL_COUNT) / ARC_T_LAYER_COUNT);
        const int which = i < size_t(ARC_T_GLOBAL_COUNT) ? int(i) : int((i - ARC_T_GLOBAL_COUNT) % ARC_T_LAYER_COUNT);
        int qtype;
        uint32_t rows, K;
        if ((rc = arc_model_tensor_info(dims, layer, which, &qtype, &rows, &K, &up[i].bytes))) return rc;
        if (!(up[i].src = tensors[i])) return set_error(ARC_ERR_INVALID_ARGUMENT, "tensor %zu is null", i);
        up[i].dev_bytes = qtype == kFmtQ6 ? up[i].bytes / kQ6Bytes * kQ6PBytes : up[i].bytes;
        plan.place(&up[i].dev, up[i].dev_bytes);
        M->weight_bytes += up[i].bytes;
    }
    plan.pad(256);
    for (uint32_t l = 0; l < dims->layers; ++l)
        if (dims->down_type[l] == ARC_Q4_K) ++M->e148_slots;
    if (M->e148_slots) {
        M->e148_stride = ArenaPlan::round_up(exec148_image_bytes(dims->hidden, dims->ffn));
        plan.place(&M->e148_base, M->e148_stride * M->e148_slots);
    }
    plan.pad(4096);  // nothing near the allocation's end is read past it
    M->arena_bytes = plan.bytes();
    if ((rc = plan.commit(&M->arena, "model arena"))) return rc;
    std::vector<uint8_t> padded;
    for (const Upload& u : up) {
        const void* src = u.src;
        if (u.dev_bytes != u.bytes) {
            const uint64_t blocks = u.bytes / kQ6Bytes;
            if (padded.size() < u.dev_bytes) {
                try {
                    padded.resize(u.dev_bytes);
                } catch (const std::bad_alloc&) {
                    return set_error(ARC_ERR_OUT_OF_MEMORY, "host staging for a padded Q6_K tensor");
                }
            }
            const uint8_t* s8 = static_cast<const uint8_t*>(u.src);
            for (uint64_t b = 0; b < blocks; ++b) {
                std::memcpy(padded.data() + b * kQ6PBytes, s8 + b * kQ6Bytes, kQ6Bytes);
                padded[b * kQ6PBytes + kQ6Bytes] = 0;
                padded[b * kQ6PBytes + kQ6Bytes + 1] = 0;
            }
            src = padded.data();
        }
        if ((rc = check_hip(hipMemcpy(const_cast<void*>(u.dev), src, u.dev_bytes, hipMemcpyHostToDevice),
                            "upload weights")))
            return rc;
    }

    auto at = [&](int layer, int which) { return up[size_t(ARC_T_GLOBAL_COUNT) + size_t(layer) * ARC_T_LAYER_COUNT + which].dev; };
    M->emb = static_cast<const uint8_t*>(up[ARC_T_TOKEN_EMBD].dev);
    M->out = static_cast<const uint8_t*>(up[ARC_T_OUTPUT].dev);
    M->out_norm = static_cast<const float*>(up[ARC_T_OUTPUT_NORM].dev);
    for (uint32_t l = 0; l < dims->layers; ++l) {
        Layer& L = M->layers[l];
        const int li = int(l);
        L.attn_norm = static_cast<const float*>(at(li, ARC_T_ATTN_NORM));
        L.q = static_cast<const uint8_t*>(at(li, ARC_T_ATTN_Q));
        L.k = static_cast<const uint8_t*>(at(li, ARC_T_ATTN_K));
        L.v = static_cast<const uint8_t*>(at(li, ARC_T_ATTN_V));
        L.qb = static_cast<const float*>(at(li, ARC_T_ATTN_Q_BIAS));
        L.kb = static_cast<const float*>(at(li, ARC_T_ATTN_K_BIAS));
        L.vb = static_cast<const float*>(at(li, ARC_T_ATTN_V_BIAS));
        L.o = static_cast<const uint8_t*>(at(li, ARC_T_ATTN_O));
        L.ffn_norm = static_cast<const float*>(at(li, ARC_T_FFN_NORM));
        L.gate = static_cast<const uint8_t*>(at(li, ARC_T_FFN_GATE));
        L.up = static_cast<const uint8_t*>(at(li, ARC_T_FFN_UP));
        L.down = static_cast<const uint8_t*>(at(li, ARC_T_FFN_DOWN));
        L.v_type = dims->v_type[l] == kFmtQ6 ? kFmtQ6P : kFmtQ4;
        L.down_type = dims->down_type[l] == kFmtQ6 ? kFmtQ6P : kFmtQ4;
    }
    *out = M.release();
    return ARC_OK;
}

int arc_model_create_synthetic(const arc_model_dims* dims, uint64_t seed, arc_model** out)
{
    if (!dims || !out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    int rc = dims_ok(*dims);
    if (rc) return rc;
    const size_t nt = size_t(ARC_T_GLOBAL_COUNT) + size_t(dims->layers) * ARC_T_LAYER_COUNT;
    std::vector<std::vector<uint8_t>> host(nt);
    std::vector<const void*> ptrs(nt, nullptr);
    // generate and upload tensor by tensor to bound host memory
    std::unique_ptr<arc_model> dummy;
    for (size_t i = 0; i < nt; ++i) {
        const int layer = i < size_t(ARC_T_GLOBAL_COUNT) ? -1 : int((i - ARC_T_GLOBAL_COUNT) / ARC_T_LAYER_COUNT);
        const int which = i < size_t(ARC_T_GLOBAL_COUNT) ? int(i) : int((i - ARC_T_GLOBAL_COUNT) % ARC_T_LAYER_COUNT);
        int qtype;
        uint32_t rows, K;
        uint64_t bytes;
        if ((rc = arc_model_tensor_info(dims, layer, which, &qtype, &rows, &K, &bytes))) return rc;
        host[i].resize(bytes);
        if ((rc = arc_model_synth_tensor(dims, seed, layer, which, host[i].data()))) return rc;
        ptrs[i] = host[i].data();
    }
    return arc_model_create(dims, ptrs.data(), out);
}

int arc_model_destroy(arc_model* m)
{
    delete m;
    return ARC_OK;
}

uint64_t arc_model_weight_bytes(const arc_model* m) { return m ? m->weight_bytes : 0; }

int arc_model_exec148_reserve(const arc_model* m, void** base, uint64_t* slot_stride, uint32_t* slots)
{
    if (!m || !base || !slot_stride || !slots) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    *base = m->e148_base;
    *slot_stride = m->e148_stride;
    *slots = m->e148_slots;
    return ARC_OK;
}

int arc_session_residency(const arc_session* s, arc_residency* out)
{
    if (!s || !out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    const arc_model* m = s->model;
    out->weight_bytes = m->weight_bytes;
    out->model_arena_bytes = m->arena_bytes;
    out->exec148_reserve_bytes = m->e148_stride * m->e148_slots;
    out->kv_bytes = s->kv_bytes;
    out->working_bytes = s->working_bytes;
    out->total_bytes = m->arena_bytes + s->kv_bytes + s->working_bytes;
    return ARC_OK;
}

int arc_session_create(arc_model* m, uint32_t max_ctx, arc_session** out)
{
    if (!m || !out || max_ctx == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad session arguments");
    if (max_ctx > uint32_t(kMaxChunks * kChunk))
        return set_error(ARC_ERR_UNSUPPORTED, "max_ctx %u exceeds the supported %d positions", max_ctx,
                         kMaxChunks * kChunk);
    *out = nullptr;
    std::unique_ptr<arc_session> S(new (std::nothrow) arc_session);
    if (!S) return set_error(ARC_ERR_OUT_OF_MEMORY, "host allocation");
    const arc_model_dims& d = m->dims;
    S->model = m;
    S->max_ctx = max_ctx;
    S->max_chunks = (max_ctx + kChunk - 1) / kChunk;
    S->out_cap = max_ctx;
    const uint32_t KVD = d.kv_heads * kHeadDim, H = d.hidden;
    int rc = check_hip(hipStreamCreateWithFlags(&S->stream, hipStreamNonBlocking), "stream");
    if (rc) return rc;
    S->best_cap = min((d.vocab + 3u) / 4u, 65536u);
    const uint64_t kv = uint64_t(d.layers) * max_ctx * KVD * sizeof(_Float16);
    const size_t fl = sizeof(float);
    const size_t heads_chunks = size_t(d.kv_heads) * kMaxSplits * (d.q_heads / d.kv_heads);
    PrefillBufs& pf = S->pf;
    pf.part_elems = prefill_part_elems(d);
    pf.host_slots = (max_ctx + kPfMaxM - 1) / kPfMaxM;

    // The session arena: KV cache, then the decode step's and the prompt
    // pass's working memory.  Nothing is allocated after this point.
    ArenaPlan plan;
    plan.place(&S->kcache, kv);
    plan.place(&S->vcache, kv);
    S->kv_bytes = plan.bytes();
    plan.place(&S->h, H * fl);
    plan.place(&S->h1, H * fl);
    plan.place(&S->q, H * fl);
    plan.place(&S->attn, H * fl);
    plan.place(&S->s, size_t(d.ffn) * fl);
    plan.place(&S->logits, size_t(d.vocab) * fl);
    plan.place(&S->apo, heads_chunks * kHeadDim * fl);
    plan.place(&S->apml, heads_chunks * 2 * fl);
    plan.place(&S->rope, size_t(max_ctx) * 64 * sizeof(float2));
    plan.place(&S->best, size_t(S->best_cap) * sizeof(ArgBest));
    plan.place(&S->ctl, sizeof(DecodeCtl));
    plan.place(&S->counters, kCounters * sizeof(uint32_t));
    plan.place(&S->done, kDoneCopies * kDoneStride * sizeof(uint32_t));
    plan.place(&S->out_tokens, size_t(S->out_cap) * sizeof(uint32_t));
    plan.place(&pf.h, size_t(kPfMaxM) * H * fl);
    plan.place(&pf.x, size_t(kPfMaxM) * H * sizeof(_Float16));
    plan.place(&pf.xs, size_t(kPfMaxM) * d.ffn * sizeof(_Float16));
    plan.place(&pf.q, size_t(kPfMaxM) * H * fl);
    plan.place(&pf.part, pf.part_elems * fl);
    plan.place(&pf.tokens, kPfMaxM * sizeof(uint32_t));
    plan.pad(4096);  // nothing near the allocation's end is read past it
    S->working_bytes = plan.bytes() - S->kv_bytes;
    if ((rc = plan.commit(&S->arena, "session arena"))) return rc;

    // Pinned host staging, one allocation: control-block uploads (slot 0 the
    // download), generated tokens, prompt tokens per pass.
    const size_t ctl_bytes = (size_t(max_ctx) + 1) * sizeof(DecodeCtl);
    const size_t tok_bytes = size_t(S->out_cap) * sizeof(uint32_t);
    const size_t prompt_bytes = size_t(pf.host_slots) * kPfMaxM * sizeof(uint32_t);
    if ((rc = check_hip(hipHostMalloc(&S->pinned, ctl_bytes + tok_bytes + prompt_bytes, hipHostMallocDefault),
                        "pinned staging")))
        return rc;
    S->host_ctl = static_cast<DecodeCtl*>(S->pinned);
    S->host_tokens = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(S->pinned) + ctl_bytes);
    pf.host_tokens = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(S->pinned) + ctl_bytes + tok_bytes);

    if ((rc = check_hip(hipMemset(S->counters, 0, kCounters * sizeof(uint32_t)), "counters"))) return rc;
    if ((rc = check_hip(hipMemset(S->done, 0, kDoneCopies * kDoneStride * sizeof(uint32_t)), "done counters")))
        return rc;
    // rows past a prompt are read (never written) by the prompt-pass GEMM tiles
    if ((rc = check_hip(hipMemset(pf.x, 0, size_t(kPfMaxM) * H * sizeof(_Float16)), "prefill x"))) return rc;
    if ((rc = check_hip(hipMemset(pf.xs, 0, size_t(kPfMaxM) * d.ffn * sizeof(_Float16)), "prefill xs"))) return rc;
    {   // RoPE factors: angle = pos * theta^(-2p/128) in fp64, cos and sin rounded to fp32
        double inv[64];
        for (int i = 0; i < 64; ++i) inv[i] = std::pow(double(d.rope_theta), -2.0 * double(i) / double(kHeadDim));
        std::vector<float2> tab(size_t(max_ctx) * 64);
        for (uint32_t t = 0; t < max_ctx; ++t)
            for (int i = 0; i < 64; ++i) {
                const double a = double(t) * inv[i];
                tab[size_t(t) * 64 + i] = make_float2(float(std::cos(a)), float(std::sin(a)));
            }
        if ((rc = check_hip(hipMemcpy(S->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice), "rope")))
            return rc;
    }
    if ((rc = check_hip(hipMemset(S->kcache, 0, kv), "kcache"))) return rc;
    if ((rc = check_hip(hipMemset(S->vcache, 0, kv), "vcache"))) return rc;
    *out = S.release();
    return ARC_OK;
}

int arc_session_destroy(arc_session* s)
{
    delete s;
    return ARC_OK;
}

int arc_session_kv(arc_session* s, uint32_t layer, void** k, void** v)
{
    if (!s || !k || !v || layer >= s->model->dims.layers) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad kv query");
    const uint64_t off = uint64_t(layer) * s->max_ctx * s->model->dims.kv_heads * kHeadDim;
    *k = s->kcache + off;
    *v = s->vcache + off;
    return ARC_OK;
}

int arc_session_fill_kv(arc_session* s, uint32_t ctx, uint64_t seed)
{
    if (!s || ctx > s->max_ctx) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad kv fill");
    const arc_model_dims& d = s->model->dims;
    const size_t row = size_t(d.kv_heads) * kHeadDim, n = size_t(ctx) * row;
    std::vector<float> f(n);
    std::vector<_Float16> hbuf(n);
    for (uint32_t l = 0; l < d.layers; ++l) {
        for (int kv = 0; kv < 2; ++kv) {
            int rc = arc_synth_normal(seed, 1000000ull + 2ull * l + uint64_t(kv), n, 0.0f, 1.0f, f.data());
            if (rc) return rc;
            for (size_t i = 0; i < n; ++i) hbuf[i] = static_cast<_Float16>(f[i]);
            _Float16* dst = (kv ? s->vcache : s->kcache) + uint64_t(l) * s->max_ctx * row;
            if ((rc = check_hip(hipMemcpy(dst, hbuf.data(), n * sizeof(_Float16), hipMemcpyHostToDevice), "kv fill")))
                return rc;
        }
    }
    return ARC_OK;
}

}  // extern "C"

namespace arc {

// Captures the decode step as a graph on first use (and when the logits
// flag changes).
static int ensure_graph(arc_session* s, bool logits)
{
    if (s->exec && s->graph_logits == logits) return ARC_OK;
    if (s->exec) {
        (void)hipGraphExecDestroy(s->exec);
        (void)hipGraphDestroy(s->graph);
        s->exec = nullptr;
        s->graph = nullptr;
    }
    // a dry run fills the launch helpers' occupancy caches (host-side
    // queries) before the capture starts
    g_dry_run = true;
    int rc = launch_step(s, logits, nullptr);
    g_dry_run = false;
    if (rc) return rc;
    if ((rc = check_hip(hipStreamSynchronize(s->stream), "sync"))) return rc;
    if ((rc = check_hip(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal), "begin capture"))) return rc;
    uint32_t nk = 0;
    rc = launch_step(s, logits, &nk);
    hipGraph_t g = nullptr;
    const int rc2 = check_hip(hipStreamEndCapture(s->stream, &g), "end capture");
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (rc2) return rc2;
    s->graph = g;
    if ((rc = check_hip(hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0), "instantiate"))) return rc;
    s->graph_logits = logits;
    s->kernels_per_step = nk;
    return ARC_OK;
}

static int run_step(arc_session* s, bool logits, bool use_graph)
{
    if (use_graph) return check_hip(hipGraphLaunch(s->exec, s->stream), "graph launch");
    uint32_t nk = 0;
    const int rc = launch_step(s, logits, &nk);
    if (!rc) s->kernels_per_step = nk;
    return rc;
}

// Stages step i's control block in pinned memory and queues its upload.  The
// staging slot stays untouched until the call's final synchronisation.
static int upload_ctl(arc_session* s, uint32_t i, uint32_t pos, uint32_t token)
{
    s->host_ctl[1 + i] = DecodeCtl{pos, token, 0u, 0u, 0u};
    return check_hip(hipMemcpyAsync(s->ctl, &s->host_ctl[1 + i], sizeof(DecodeCtl), hipMemcpyHostToDevice, s->stream),
                     "ctl upload");
}

// Downloads the control block after the last step and waits for the stream.
static int finish_call(arc_session* s, uint32_t* nonfinite, uint32_t* token)
{
    int rc = check_hip(hipMemcpyAsync(&s->host_ctl[0], s->ctl, sizeof(DecodeCtl), hipMemcpyDeviceToHost, s->stream),
                       "ctl download");
    if (rc) return rc;
    if ((rc = check_hip(hipStreamSynchronize(s->stream), "decode sync"))) return rc;
    if (s->host_ctl[0].waits_expired)
        return set_error(ARC_ERR_DEVICE, "%u cross-workgroup waits of the decode step gave up (results invalid)",
                         s->host_ctl[0].waits_expired);
    if (nonfinite) *nonfinite = s->host_ctl[0].nonfinite;
    if (token) *token = s->host_ctl[0].token;
    return ARC_OK;
}

}  // namespace arc

extern "C" {

int arc_session_decode(arc_session* s, uint32_t token, uint32_t pos, uint32_t n_steps, int flags, uint32_t* out_tokens,
                       uint32_t* nonfinite)
{
    if (!s || n_steps == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad decode arguments");
    const arc_model_dims& d = s->model->dims;
    if (token >= d.vocab) return set_error(ARC_ERR_INVALID_ARGUMENT, "token %u out of vocabulary", token);
    if (uint64_t(pos) + n_steps > s->max_ctx)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "positions %u..%u exceed the context %u", pos, pos + n_steps - 1,
                         s->max_ctx);
    const bool logits = (flags & ARC_DECODE_LOGITS) != 0;
    const bool use_graph = (flags & ARC_DECODE_NO_GRAPH) == 0;
    // the previous call ended with a stream synchronisation, so the pinned
    // staging is free to reuse
    int rc = upload_ctl(s, 0, pos, token);
    if (rc) return rc;
    if (use_graph && (rc = ensure_graph(s, logits))) return rc;
    for (uint32_t i = 0; i < n_steps; ++i)
        if ((rc = run_step(s, logits, use_graph))) return rc;
    if ((rc = check_hip(hipMemcpyAsync(s->host_tokens, s->out_tokens, n_steps * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                       s->stream),
                        "tokens download")))
        return rc;
    if ((rc = finish_call(s, nonfinite, nullptr))) return rc;
    if (out_tokens) std::memcpy(out_tokens, s->host_tokens, n_steps * sizeof(uint32_t));
    return ARC_OK;
}

int arc_session_prefill(arc_session* s, const uint32_t* tokens, uint32_t n, uint32_t pos0, int flags,
                        uint32_t* next_token, uint32_t* nonfinite)
{
    if (!s || !tokens || n == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad prefill arguments");
    const arc_model_dims& d = s->model->dims;
    if (uint64_t(pos0) + n > s->max_ctx)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "positions %u..%u exceed the context %u", pos0, pos0 + n - 1,
                         s->max_ctx);
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= d.vocab) return set_error(ARC_ERR_INVALID_ARGUMENT, "token %u out of vocabulary", tokens[i]);
    const bool logits = (flags & ARC_DECODE_LOGITS) != 0;
    const bool use_graph = (flags & ARC_DECODE_NO_GRAPH) == 0;
    int rc = 0;
    if (n > 1 && (flags & ARC_PREFILL_STEPWISE) == 0) {
        // batched MFMA prompt pass
        if ((rc = run_prefill(s, tokens, n, pos0, logits))) return rc;
        return finish_call(s, nonfinite, next_token);
    }
    if (use_graph && (rc = ensure_graph(s, logits))) return rc;
    s->prefill_kernels = 0;
    for (uint32_t i = 0; i < n; ++i) {
        // each step is fed the given token, not the previous step's argmax
        if ((rc = upload_ctl(s, i, pos0 + i, tokens[i]))) return rc;
        if ((rc = run_step(s, logits, use_graph))) return rc;
        s->prefill_kernels += s->kernels_per_step;
    }
    return finish_call(s, nonfinite, next_token);
}

int arc_session_logits(arc_session* s, float* host_logits)
{
    if (!s || !host_logits) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad logits query");
    return check_hip(hipMemcpy(host_logits, s->logits, size_t(s->model->dims.vocab) * sizeof(float), hipMemcpyDeviceToHost),
                     "logits download");
}

uint32_t arc_session_kernels_per_step(const arc_session* s) { return s ? s->kernels_per_step : 0; }

int arc_model_tensor_device(const arc_model* model, int layer, int which, const void** ptr)
{
    if (!model || !ptr) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    *ptr = nullptr;
    if (layer < 0) {
        switch (which) {
        case ARC_T_TOKEN_EMBD: *ptr = model->emb; break;
        case ARC_T_OUTPUT: *ptr = model->out; break;
        case ARC_T_OUTPUT_NORM: *ptr = model->out_norm; break;
        default: return set_error(ARC_ERR_INVALID_ARGUMENT, "bad global tensor %d", which);
        }
        return ARC_OK;
    }
    if (uint32_t(layer) >= model->layers.size()) return set_error(ARC_ERR_INVALID_ARGUMENT, "layer %d out of range", layer);
    if (which < 0 || which >= ARC_T_LAYER_COUNT) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad layer tensor %d", which);
    const arc::Layer& L = model->layers[layer];
    const void* const t[ARC_T_LAYER_COUNT] = {L.attn_norm, L.q, L.k, L.v, L.qb, L.kb, L.vb, L.o, L.ffn_norm, L.gate,
                                              L.up, L.down};
    *ptr = t[which];
    return ARC_OK;
}

int arc_session_route_down(arc_session* s, uint32_t layer, const void* exec148)
{
    if (!s) return set_error(ARC_ERR_INVALID_ARGUMENT, "null session");
    const arc_model* m = s->model;
    if (layer >= m->layers.size()) return set_error(ARC_ERR_INVALID_ARGUMENT, "layer %u out of range", layer);
    if (exec148 && m->layers[layer].down_type != kFmtQ4)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "layer %u: ffn_down is not Q4_K (no EXEC148 route)", layer);
    if (reinterpret_cast<uintptr_t>(exec148) & 15u)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "EXEC148 image not 16-byte aligned");
    if (s->down_e148.size() != m->layers.size()) s->down_e148.assign(m->layers.size(), nullptr);
    const uint8_t* e = static_cast<const uint8_t*>(exec148);
    if (s->down_e148[layer] == e) return ARC_OK;
    s->down_e148[layer] = e;
    // the captured step reads the old route: capture again on next use
    if (s->exec) (void)hipGraphExecDestroy(s->exec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    s->exec = nullptr;
    s->graph = nullptr;
    return ARC_OK;
}

uint32_t arc_session_prefill_kernels(const arc_session* s) { return s ? s->prefill_kernels : 0; }

}  // extern "C"

// --------------------------------------------- standalone decode attention
namespace arc {

// Zeroes the arrival counters and sets the control block's position for a
// standalone attention launch (kernels, not memsets: callers may capture).
__global__ void k_attn_setup(uint32_t* counters, uint32_t n, DecodeCtl* ctl, uint32_t pos)
{
    const uint32_t i = threadIdx.x;
    if (i < n) counters[i] = 0u;
    if (i == 0) *ctl = DecodeCtl{pos, 0u, 0u, 0u, 0u};
}

struct AttnWorkspace {
    size_t po, pml, counters, ctl, bytes;
};

static AttnWorkspace attn_workspace(uint32_t kv_heads, uint32_t hpk)
{
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    AttnWorkspace w{};
    const size_t parts = size_t(kv_heads) * kMaxSplits * hpk;
    w.po = 0;
    w.pml = up(parts * kHeadDim * sizeof(float));
    w.counters = w.pml + up(parts * 2 * sizeof(float));
    w.ctl = w.counters + up(kv_heads * sizeof(uint32_t));
    w.bytes = w.ctl + up(sizeof(DecodeCtl));
    return w;
}

}  // namespace arc

extern "C" {

size_t arc_attention_workspace_bytes(uint32_t kv_heads, uint32_t hpk)
{
    if (kv_heads == 0 || kv_heads > uint32_t(kCounterLmHead - kCounterAttn) || hpk == 0 || hpk > uint32_t(kMaxHpk))
        return 0;
    return attn_workspace(kv_heads, hpk).bytes;
}

int arc_attention_decode(const float* q, const void* kc, const void* vc, uint32_t kv_heads, uint32_t hpk,
                         uint32_t max_ctx, uint32_t T, float* out, void* workspace, arc_stream_t stream)
{
    if (!q || !kc || !vc || !out || !workspace) return set_error(ARC_ERR_INVALID_ARGUMENT, "null argument");
    if (kv_heads == 0 || kv_heads > uint32_t(kCounterLmHead - kCounterAttn) || hpk == 0 || hpk > uint32_t(kMaxHpk))
        return set_error(ARC_ERR_UNSUPPORTED, "attention supports 1..%d kv heads and 1..%d query heads per kv head",
                         kCounterLmHead - kCounterAttn, kMaxHpk);
    if (max_ctx == 0 || max_ctx > uint32_t(kMaxChunks * kChunk) || T == 0 || T > max_ctx)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "bad context: T %u, max_ctx %u (at most %d)", T, max_ctx,
                         kMaxChunks * kChunk);
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                         reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc);
    if (al & 15u) return set_error(ARC_ERR_INVALID_ARGUMENT, "q, out, kc and vc must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    const AttnWorkspace w = attn_workspace(kv_heads, hpk);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* counters = reinterpret_cast<uint32_t*>(ws + w.counters);
    DecodeCtl* ctl = reinterpret_cast<DecodeCtl*>(ws + w.ctl);
    hipLaunchKernelGGL(k_attn_setup, dim3(1), dim3(64), 0, st, counters, kv_heads, ctl, T - 1);
    int rc = check_hip(hipGetLastError(), "attention setup");
    if (rc) return rc;
    AttnParams ap{};
    ap.q = q;
    ap.kc = static_cast<const _Float16*>(kc);
    ap.vc = static_cast<const _Float16*>(vc);
    ap.out = out;
    ap.po = reinterpret_cast<float*>(ws + w.po);
    ap.pml = reinterpret_cast<float*>(ws + w.pml);
    ap.counter = counters;
    ap.ctl = ctl;
    ap.kv_heads = kv_heads;
    ap.hpk = hpk;
    ap.max_ctx = max_ctx;
    ap.scale = 1.0f / std::sqrt(float(kHeadDim));
    launch_attn(ap, kv_heads, st);
    return check_hip(hipGetLastError(), "attention");
}

}  // extern "C"
