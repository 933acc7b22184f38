// arc_kernels.hip -- standalone gfx950 kernels of the packed Q4_K/Q6_K decode
// hot path (GEMV, fused gate/up + SwiGLU, split-K, LM head + argmax,
// RMSNorm, dequant dump) and their C-ABI launchers (include/arcllm_hip.h).
// The GEMV core itself is in arc_gemv.hpp.
#include "arc_gemv.hpp"

#include <cstdio>
#include <cstring>
#include <mutex>

namespace arc {

// Argmax partials of arc_lmhead_argmax_noalloc: one ArgBest per workgroup of
// its LM-head launch, in a file-scope device array instead of a workspace.
// Each device holds its own copy at its own address; host code never passes
// the array's name to a kernel, only the address hipGetSymbolAddress returns
// for the current device (scratch_on_device).  Every workgroup of a launch
// writes its entry and the second stage reads exactly those entries, so
// nothing needs clearing between calls.
constexpr uint32_t kNoAllocBest = 8192;  // 128 KB per device
static __device__ __align__(256) ArgBest scratch[kNoAllocBest];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static ArgBest* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device with that device current.
static int scratch_on_device(ArgBest** out)
{
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "current device");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices) return set_error(ARC_ERR_UNSUPPORTED, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if ((rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "scratch address"))) return rc;
        if (!ptr) return set_error(ARC_ERR_DEVICE, "no device address for the argmax scratch");
        g_scratch_ptr[dev] = static_cast<ArgBest*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return ARC_OK;
}

// Fixed-order second pass of the split-K GEMV: y[r] = ((p0 + p1) + ...) + res,
// with the partials of row r contiguous at part[r*splits].  A workgroup
// covers 64 rows; per batch of up to 128 split columns its 256 threads read
// the rows' partials (contiguous when one batch holds every split) with all
// loads in flight, into LDS rows padded to 129 floats, and thread r then adds
// row r's partials in order.
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, uint32_t rows,
                                                       uint32_t splits, const float* __restrict__ residual,
                                                       float* __restrict__ y)
{
    constexpr uint32_t kRows = 64, kCols = 128, kStride = kCols + 1, kPer = kRows * kCols / 256;
    __shared__ float tile[kRows * kStride];
    const uint32_t r0 = blockIdx.x * kRows, tid = threadIdx.x;
    const uint32_t nr = min(kRows, rows - r0);
    float s = 0.0f;
    for (uint32_t j0 = 0; j0 < splits; j0 += kCols) {
        const uint32_t n = min(kCols, splits - j0), total = nr * n;
        float v[kPer];
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t e = tid + 256u * i;
            const uint32_t rr = e / n, j = e - rr * n;
            v[i] = e < total ? part[uint64_t(r0 + rr) * splits + j0 + j] : 0.0f;
        }
        __syncthreads();  // the previous batch has been added
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t e = tid + 256u * i;
            const uint32_t rr = e / n, j = e - rr * n;
            if (e < total) tile[rr * kStride + j] = v[i];
        }
        __syncthreads();
        if (tid < nr)
            for (uint32_t j = 0; j < n; ++j) s += tile[tid * kStride + j];
    }
    if (tid < nr) {
        const uint32_t r = r0 + tid;
        if (residual) s += residual[r];
        y[r] = s;
    }
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
    const ArgBest res = wg_argmax(bv, bi, nf);
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

// stride: kQ6Bytes, or kQ6PBytes for padded Q6_K
__global__ __launch_bounds__(256) void k_dequant_q6(const uint8_t* __restrict__ w, uint32_t stride,
                                                    float* __restrict__ out)
{
#pragma clang fp contract(off)
    const uint64_t blk = blockIdx.x;
    const uint32_t k = threadIdx.x;
    const uint8_t* b = w + blk * stride;
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

// Padded Q6_K: thread t writes dword t % 53 of block t / 53 (bytes 4j .. 4j+3
// of the 210-byte source block, read as two halves: the source is 2-byte
// aligned); dword 52 is bytes 208, 209 and two zero bytes.
constexpr uint32_t kQ6PDwords = kQ6PBytes / 4;
static_assert(kQ6PBytes == kQ6Bytes + 2 && kQ6PBytes % 4 == 0, "one 2-byte pad per block");
__global__ __launch_bounds__(256) void k_q6_pad(const uint16_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                uint64_t dwords)
{
    const uint64_t t = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (t >= dwords) return;
    const uint64_t blk = t / kQ6PDwords;
    const uint32_t j = uint32_t(t % kQ6PDwords);
    const uint16_t* b = src + blk * (kQ6Bytes / 2) + 2u * j;
    const uint32_t lo = b[0], hi = j + 1u < kQ6PDwords ? uint32_t(b[1]) : 0u;
    dst[t] = lo | (hi << 16);
}

}  // namespace arc

using namespace arc;

extern "C" {

int arc_tune_force(int bs, int rpl)
{
    if (bs == 0) {
        g_force = Cfg{0, 0, 0};
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
            g_force = Cfg{bs, rpl, 0};
            return ARC_OK;
        }
    return set_error(ARC_ERR_INVALID_ARGUMENT, "no kernel instance for bs=%d rpl=%d", bs, rpl);
}

int arc_tune_waves(int waves)
{
    if (waves != 0 && waves != 4 && waves != 8)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "waves per workgroup must be 0 (automatic), 4 or 8");
    g_force_waves = waves;
    return ARC_OK;
}

int arc_tune_rowstream(int mode)
{
    if (mode < -1 || mode > 1)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "row-stream mode must be -1 (automatic), 0 (off) or 1 (on)");
    g_rowstream = mode;
    return ARC_OK;
}

int arc_dequant(int qtype, const void* w, uint32_t rows, uint32_t K, float* out, arc_stream_t stream)
{
    if (qtype == kFmtE148) return set_error(ARC_ERR_UNSUPPORTED, "arc_dequant takes Q4_K or Q6_K");
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if (!out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    const uint64_t blocks = uint64_t(rows) * (K / kQK);
    if (blocks > 0x7fffffffull) return set_error(ARC_ERR_UNSUPPORTED, "tensor too large for one dequant launch");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (qtype == kFmtQ4)
        hipLaunchKernelGGL(k_dequant_q4, dim3(uint32_t(blocks)), dim3(256), 0, s, static_cast<const uint8_t*>(w), out);
    else
        hipLaunchKernelGGL(k_dequant_q6, dim3(uint32_t(blocks)), dim3(256), 0, s, static_cast<const uint8_t*>(w),
                           uint32_t(qtype == kFmtQ6P ? kQ6PBytes : kQ6Bytes), out);
    return check_hip(hipGetLastError(), "dequant launch");
}

int arc_q6_pad(const void* q6, uint32_t rows, uint32_t K, void* padded, arc_stream_t stream)
{
    int rc = check_shape(kFmtQ6, q6, rows, K);
    if (rc) return rc;
    if ((rc = check_shape(kFmtQ6P, padded, rows, K))) return rc;
    const uint64_t blocks = uint64_t(rows) * (K / kQK);
    const uint8_t* a = static_cast<const uint8_t*>(q6);
    const uint8_t* b = static_cast<const uint8_t*>(padded);
    if (b < a + blocks * kQ6Bytes && a < b + blocks * kQ6PBytes)
        return set_error(ARC_ERR_INVALID_ARGUMENT, "padded image overlaps its source");
    const uint64_t dwords = blocks * kQ6PDwords;
    hipLaunchKernelGGL(k_q6_pad, dim3(uint32_t((dwords + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(q6), static_cast<uint32_t*>(padded), dwords);
    return check_hip(hipGetLastError(), "Q6_K pad launch");
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
    if (qtype == kFmtE148) return set_error(ARC_ERR_UNSUPPORTED, "fused gate/up takes Q4_K or Q6_K");
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
        // one column per split, all columns in one launch: the wave owning a
        // row computes its partials (one per quad and column) and then adds
        // them in column order, so both passes run in this launch
        p.split_bps = nb;
        p.panel = nb;
        p.y2 = y;
        p.res = residual;
        Cfg c = choose_cfg(EPI_PLAIN, rows, nb, 1);
        if (c.bs < 8 || c.rpl > 2) c = Cfg{8, 1, c.waves};  // <= 4 rows per wave tile in LDS
        return check_hip(launch_gemv_epi(EPI_COLPART, qtype, c, p, 1, s), "split-K");
    }
    rc = run_paneled(EPI_PARTIAL, qtype, p, used, s, "split-K pass 1");
    if (rc) return rc;
    hipLaunchKernelGGL(k_splitk_reduce, dim3((rows + 63) / 64), dim3(256), 0, s, partials, rows, used, residual, y);
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
    if ((qtype != kFmtQ4 && qtype != kFmtQ6 && qtype != kFmtQ6P) || rows == 0 || K == 0 || K % kQK) return 0;
    return size_t(lm_max_wgs(rows)) * sizeof(ArgBest);
}

int arc_lmhead_argmax(int qtype, const void* w, uint32_t rows, uint32_t K, const float* h, const float* normw,
                      float eps, float* logits, void* workspace, uint32_t* out, arc_stream_t stream)
{
    if (qtype == kFmtE148) return set_error(ARC_ERR_UNSUPPORTED, "the LM head takes Q4_K or Q6_K");
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

int arc_lmhead_argmax_noalloc(int qtype, const void* w, uint32_t rows, uint32_t K, const float* h,
                              const float* normw, float eps, float* logits, uint32_t* out, arc_stream_t stream)
{
    if (qtype == kFmtE148) return set_error(ARC_ERR_UNSUPPORTED, "the LM head takes Q4_K or Q6_K");
    int rc = check_shape(qtype, w, rows, K);
    if (rc) return rc;
    if ((rc = check_vec(h, "h"))) return rc;
    if (normw && (rc = check_vec(normw, "normw"))) return rc;
    if (!out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null out");
    if (K / kQK > uint32_t(kPanel)) return set_error(ARC_ERR_UNSUPPORTED, "LM head supports K <= %d", kPanel * kQK);
    ArgBest* best = nullptr;
    if ((rc = scratch_on_device(&best))) return rc;
    GemvParams p = make_params(qtype, w, nullptr, rows, K, h);
    p.flags = normw ? F_NORM : 0u;
    p.normw = normw;
    p.eps = eps;
    p.y = logits;
    p.best = best;
    const Cfg c = choose_cfg(EPI_ARGMAX, rows, p.nb, 1);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // size the grid first (host-side only): its workgroups must fit the scratch
    uint32_t gx = 0;
    const bool dry = g_dry_run;
    g_dry_run = true;
    const hipError_t e = launch_gemv_epi(EPI_ARGMAX, qtype, c, p, 1, s, &gx);
    g_dry_run = dry;
    if ((rc = check_hip(e, "lm-head sizing"))) return rc;
    if (gx > kNoAllocBest)
        return set_error(ARC_ERR_UNSUPPORTED, "LM-head launch needs %u workgroup results, the scratch holds %u", gx,
                         kNoAllocBest);
    uint32_t gx2 = 0;
    rc = check_hip(launch_gemv_epi(EPI_ARGMAX, qtype, c, p, 1, s, &gx2), "lm-head launch");
    if (rc) return rc;
    if (gx2 != gx) return set_error(ARC_ERR_DEVICE, "internal: LM-head grid changed (%u vs %u)", gx2, gx);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, s, best, gx, out);
    return check_hip(hipGetLastError(), "argmax launch");
}

}  // extern "C"
