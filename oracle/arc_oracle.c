/*
 * arc_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see arc_oracle.h).
 *
 * Plain-C restatement of the reference's CPU arithmetic for the packed
 * Q4_K/Q6_K decode path.  Citations are to the reference tree
 * (minhtri22/ArcLLM).  Compiled with -ffp-contract=off so every float
 * expression rounds exactly as written, as under MSVC /fp:precise.
 */
#include "arc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary16 -> binary32.  src/q6cb_q6_reference.hpp:20-36 and
 * src/sa1_component_benchmark.cpp:84-94: subnormals via ldexp(frac, -24),
 * +-inf, any NaN payload -> the canonical quiet NaN. */
float orc_half_to_float(uint16_t h)
{
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 31u, frac = h & 1023u;
    float v;
    if (ex == 0u) {
        if (frac == 0u) return sign ? -0.0f : 0.0f;
        v = ldexpf((float)frac, -24);
        return sign ? -v : v;
    }
    if (ex == 31u) {
        if (frac) return NAN;
        return sign ? -INFINITY : INFINITY;
    }
    v = ldexpf(1.0f + (float)frac / 1024.0f, (int)ex - 15);
    return sign ? -v : v;
}

/* binary32 -> binary16, round to nearest even (overflow -> inf, NaN kept
 * quiet).  Used where the reference path stores a value as fp16 (the KV
 * cache of the MI355X runtime). */
uint16_t orc_float_to_half_rne(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or NaN */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* result is subnormal or zero: value = ax * 2^24 in units of 2^-24 */
        const uint32_t e = ax >> 23;
        if (e < 102u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e; /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

static uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q4_K 6-bit scale/min of sub-block j (0..7) from the 12 packed bytes at
 * block offset 4.  src/sa1_component_benchmark.cpp:97-104,
 * src/arcllm_v1_i001r_p8c_profile_runtime.cpp:563-572. */
void orc_q4k_scale_min(const uint8_t *blk, uint32_t j, uint32_t *sc, uint32_t *mn)
{
    const uint8_t *s = blk + 4;
    if (j < 4u) {
        *sc = s[j] & 63u;
        *mn = s[j + 4] & 63u;
    } else {
        *sc = (uint32_t)(s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
        *mn = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

/* 4-bit code of element k (0..255): byte 16 + (k>>6)*32 + (k&31), low
 * nibble when (k&63) < 32.  src/sa1_component_benchmark.cpp:113-114. */
uint32_t orc_q4k_code(const uint8_t *blk, uint32_t k)
{
    const uint32_t local64 = k & 63u;
    const uint8_t qb = blk[16u + (k >> 6) * 32u + (local64 & 31u)];
    return local64 < 32u ? (qb & 15u) : (qb >> 4u);
}

/* w = d*sc*q - dmin*mn, evaluated left to right in fp32 without
 * contraction.  src/sa1_component_benchmark.cpp:105-116,
 * shaders/sa1_q4k_subgroup_splitk.comp:48-61. */
float orc_q4k_weight(const uint8_t *blk, uint32_t k)
{
    const float d = orc_half_to_float(ld16(blk));
    const float dmin = orc_half_to_float(ld16(blk + 2));
    uint32_t sc, mn;
    orc_q4k_scale_min(blk, k >> 5, &sc, &mn);
    const uint32_t q = orc_q4k_code(blk, k);
    const float a = d * (float)sc;
    const float b = a * (float)q;
    const float c = dmin * (float)mn;
    return b - c;
}

/* Q6_K code and scale of element k.  src/q6cb_q6_reference.hpp:49-91,
 * src/sa1_component_benchmark.cpp:118-130. */
int orc_q6k_code(const uint8_t *blk, uint32_t k, int *scale)
{
    const uint32_t half = k >> 7, kk = k & 127u, l = kk & 31u, quarter = kk >> 5;
    const uint8_t *ql = blk + half * 64u;
    const uint8_t *qh = blk + 128u + half * 32u;
    const uint8_t *sc = blk + 192u + half * 8u;
    const uint32_t is = l >> 4;
    uint32_t low, high, si;
    switch (quarter) {
    case 0: low = ql[l] & 15u; high = qh[l] & 3u; si = is; break;
    case 1: low = ql[l + 32u] & 15u; high = (qh[l] >> 2) & 3u; si = is + 2u; break;
    case 2: low = ql[l] >> 4; high = (qh[l] >> 4) & 3u; si = is + 4u; break;
    default: low = ql[l + 32u] >> 4; high = (qh[l] >> 6) & 3u; si = is + 6u; break;
    }
    *scale = (int)(int8_t)sc[si];
    return (int)(low | (high << 4)) - 32;
}

/* w = d*scale*q in fp32, left to right.  src/q6cb_q6_reference.hpp:86-89. */
float orc_q6k_weight(const uint8_t *blk, uint32_t k)
{
    int scale;
    const int q = orc_q6k_code(blk, k, &scale);
    const float d = orc_half_to_float(ld16(blk + 208));
    const float a = d * (float)scale;
    return a * (float)q;
}

/* ---- EXEC148: the Q4_K down-projection's route-B representation ----
 * src/q4_down_exec148_materializer.h:14-17 (materialize_block),
 * shaders/b1_2_exec148_gpu_materialize.comp:44-75.  A 148-byte block holds
 * the Q4_K block's d and dmin bytes verbatim (0..3), the eight unpacked 6-bit
 * (sc, mn) pairs as bytes 4 + 2j, 5 + 2j, and the 256 codes in element order,
 * two per byte from byte 20: element k in byte 20 + k/2, low nibble for even
 * k. */
void orc_exec148_block(const uint8_t *q4, uint8_t *e)
{
    memcpy(e, q4, 4);
    for (uint32_t j = 0; j < 8u; ++j) {
        uint32_t sc, mn;
        orc_q4k_scale_min(q4, j, &sc, &mn);
        e[4u + 2u * j] = (uint8_t)sc;
        e[5u + 2u * j] = (uint8_t)mn;
    }
    for (uint32_t p = 0; p < 128u; ++p)
        e[20u + p] = (uint8_t)(orc_q4k_code(q4, 2u * p) | (orc_q4k_code(q4, 2u * p + 1u) << 4));
}

int orc_exec148_tensor(const uint8_t *q4, uint32_t rows, uint32_t K, uint8_t *e)
{
    if (K == 0u || (K % ORC_QK) != 0u) return -1;
    const size_t nb = (size_t)rows * (K / ORC_QK);
    for (size_t b = 0; b < nb; ++b) orc_exec148_block(q4 + b * ORC_Q4K_BLOCK_BYTES, e + b * ORC_EXEC148_BLOCK_BYTES);
    return 0;
}

/* The validator's canonical 276-byte tuple (d, dmin bytes; (sc, mn) x 8;
 * 256 codes) of a Q4_K block and of an EXEC148 block
 * (src/q4_down_exec148_materializer.h:18-19, validator_source_tuple /
 * validator_exec_tuple); a correct EXEC148 block has the same tuple as its
 * source. */
void orc_q4k_canon(const uint8_t *q4, uint8_t *t)
{
    memcpy(t, q4, 4);
    for (uint32_t j = 0; j < 8u; ++j) {
        uint32_t sc, mn;
        orc_q4k_scale_min(q4, j, &sc, &mn);
        t[4u + 2u * j] = (uint8_t)sc;
        t[5u + 2u * j] = (uint8_t)mn;
    }
    for (uint32_t k = 0; k < 256u; ++k) t[20u + k] = (uint8_t)orc_q4k_code(q4, k);
}

void orc_exec148_canon(const uint8_t *e, uint8_t *t)
{
    memcpy(t, e, 20);
    for (uint32_t k = 0; k < 256u; ++k) {
        const uint8_t b = e[20u + (k >> 1)];
        t[20u + k] = (uint8_t)((k & 1u) ? (b >> 4) : (b & 15u));
    }
}

/* Element k of an EXEC148 block: d*sc*q - dmin*mn, the Q4_K element formula
 * on the unpacked fields (shaders/q4_down_exec148_serial.comp). */
float orc_exec148_weight(const uint8_t *e, uint32_t k)
{
    const float d = orc_half_to_float(ld16(e));
    const float dmin = orc_half_to_float(ld16(e + 2));
    const uint32_t j = k >> 5;
    const uint8_t b = e[20u + (k >> 1)];
    const uint32_t q = (k & 1u) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15u);
    const float a = d * (float)e[4u + 2u * j];
    const float bq = a * (float)q;
    const float c = dmin * (float)e[5u + 2u * j];
    return bq - c;
}

/* ---- SHA-256 (FIPS 180-4) ----
 * The round constants and initial hash are the first 32 fractional bits of
 * the cube roots of the first 64 primes and of the square roots of the first
 * 8 primes; they are computed here with exact integer roots. */
static uint64_t iroot_u128(unsigned __int128 n, int cube)
{
    uint64_t x = (uint64_t)(cube ? cbrtl((long double)n) : sqrtl((long double)n));
#define POW(v) (cube ? (unsigned __int128)(v) * (v) * (v) : (unsigned __int128)(v) * (v))
    while (x > 0 && POW(x) > n) --x;
    while (POW(x + 1) <= n) ++x;
#undef POW
    return x;
}

static void sha256_constants(uint32_t k[64], uint32_t h0[8])
{
    uint32_t primes[64], n = 0;
    for (uint32_t c = 2; n < 64u; ++c) {
        int is_p = 1;
        for (uint32_t i = 0; i < n && primes[i] * primes[i] <= c; ++i)
            if (c % primes[i] == 0u) { is_p = 0; break; }
        if (is_p) primes[n++] = c;
    }
    for (uint32_t i = 0; i < 64u; ++i) k[i] = (uint32_t)iroot_u128((unsigned __int128)primes[i] << 96, 1);
    for (uint32_t i = 0; i < 8u; ++i) h0[i] = (uint32_t)iroot_u128((unsigned __int128)primes[i] << 64, 0);
}

static uint32_t ror32(uint32_t x, uint32_t r) { return (x >> r) | (x << (32u - r)); }

static void sha256_block(uint32_t st[8], const uint32_t k[64], const uint8_t *blk)
{
    uint32_t w[64];
    for (uint32_t i = 0; i < 16u; ++i)
        w[i] = ((uint32_t)blk[4 * i] << 24) | ((uint32_t)blk[4 * i + 1] << 16) | ((uint32_t)blk[4 * i + 2] << 8) |
               (uint32_t)blk[4 * i + 3];
    for (uint32_t i = 16; i < 64u; ++i) {
        const uint32_t s0 = ror32(w[i - 15], 7) ^ ror32(w[i - 15], 18) ^ (w[i - 15] >> 3);
        const uint32_t s1 = ror32(w[i - 2], 17) ^ ror32(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t v[8];
    memcpy(v, st, sizeof(v));
    for (uint32_t i = 0; i < 64u; ++i) {
        const uint32_t e = v[4], a = v[0];
        const uint32_t t1 = v[7] + (ror32(e, 6) ^ ror32(e, 11) ^ ror32(e, 25)) + ((e & v[5]) ^ (~e & v[6])) + k[i] + w[i];
        const uint32_t t2 = (ror32(a, 2) ^ ror32(a, 13) ^ ror32(a, 22)) + ((a & v[1]) ^ (a & v[2]) ^ (v[1] & v[2]));
        memmove(v + 1, v, 7 * sizeof(uint32_t));
        v[4] += t1;
        v[0] = t1 + t2;
    }
    for (uint32_t i = 0; i < 8u; ++i) st[i] += v[i];
}

void orc_sha256(const uint8_t *p, size_t n, uint8_t out[32])
{
    uint32_t k[64], st[8];
    sha256_constants(k, st);
    size_t i = 0;
    for (; i + 64 <= n; i += 64) sha256_block(st, k, p + i);
    uint8_t tail[128];
    const size_t r = n - i, tl = r < 56 ? 64 : 128;
    memset(tail, 0, sizeof(tail));
    if (r) memcpy(tail, p + i, r);
    tail[r] = 0x80;
    const uint64_t bits = (uint64_t)n * 8u;
    for (int b = 0; b < 8; ++b) tail[tl - 1 - b] = (uint8_t)(bits >> (8 * b));
    sha256_block(st, k, tail);
    if (tl == 128) sha256_block(st, k, tail + 64);
    for (uint32_t j = 0; j < 8u; ++j) {
        out[4 * j] = (uint8_t)(st[j] >> 24);
        out[4 * j + 1] = (uint8_t)(st[j] >> 16);
        out[4 * j + 2] = (uint8_t)(st[j] >> 8);
        out[4 * j + 3] = (uint8_t)st[j];
    }
}

static int row_bytes(int qtype, uint32_t K, size_t *rb, size_t *bb)
{
    if (K == 0u || (K % ORC_QK) != 0u) return -1;
    if (qtype == ORC_Q4_K) *bb = ORC_Q4K_BLOCK_BYTES;
    else if (qtype == ORC_Q6_K) *bb = ORC_Q6K_BLOCK_BYTES;
    else return -1;
    *rb = (size_t)(K / ORC_QK) * *bb;
    return 0;
}

static float weight_at(int qtype, const uint8_t *blk, uint32_t k)
{
    return qtype == ORC_Q4_K ? orc_q4k_weight(blk, k) : orc_q6k_weight(blk, k);
}

/* All 256 weights of one block, each with exactly the operations and operand
 * order of orc_q4k_weight / orc_q6k_weight (the per-block factors d, dmin,
 * d*sc and dmin*mn are the same fp32 values those compute per element), so
 * w[k] == weight_at(qtype, blk, k) bit for bit; it only hoists the repeated
 * half and scale decodes out of the element loop. */
static void decode_block(int qtype, const uint8_t *blk, float *w)
{
    if (qtype == ORC_Q4_K) {
        const float d = orc_half_to_float(ld16(blk));
        const float dmin = orc_half_to_float(ld16(blk + 2));
        for (uint32_t j = 0; j < 8u; ++j) {
            uint32_t sc, mn;
            orc_q4k_scale_min(blk, j, &sc, &mn);
            const float a = d * (float)sc;
            const float c = dmin * (float)mn;
            /* sub-block j holds the low (j even) or high (j odd) nibbles of
             * bytes 16 + 32*(j/2) .. +31, as orc_q4k_code reads them */
            const uint8_t *qs = blk + 16u + 32u * (j >> 1);
            const uint32_t sh = (j & 1u) * 4u;
            for (uint32_t i = 0; i < 32u; ++i) {
                const float b = a * (float)((qs[i] >> sh) & 15u);
                w[32u * j + i] = b - c;
            }
        }
    } else {
        const float d = orc_half_to_float(ld16(blk + 208));
        /* the element order of orc_q6k_code: half h, quarter t, lane l */
        for (uint32_t h = 0; h < 2u; ++h) {
            const uint8_t *ql = blk + 64u * h, *qh = blk + 128u + 32u * h;
            const int8_t *sc = (const int8_t *)(blk + 192u + 8u * h);
            for (uint32_t t = 0; t < 4u; ++t)
                for (uint32_t l = 0; l < 32u; ++l) {
                    const uint32_t lo = (ql[l + 32u * (t & 1u)] >> (4u * (t >> 1))) & 15u;
                    const uint32_t hi = (qh[l] >> (2u * t)) & 3u;
                    const int q = (int)(lo | (hi << 4)) - 32;
                    const float a = d * (float)sc[(l >> 4) + 2u * t];
                    w[128u * h + 32u * t + l] = a * (float)q;
                }
        }
    }
}

int orc_dequant(int qtype, const uint8_t *w, uint32_t rows, uint32_t K, float *out)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t k = 0; k < K; k += ORC_QK)
            decode_block(qtype, w + r * rb + (k / ORC_QK) * bb, out + (size_t)r * K + k);
    return 0;
}

/* Serial fp32 dot, sum initialised with the bias: shaders/p7_q4k_gemm_2d.comp:13,
 * shaders/p7_q6k_gemm_2d.comp, src/sa1_component_benchmark.cpp:165-173. */
static float dot_r0(int qtype, const uint8_t *row, size_t bb, uint32_t K, const float *x, float init)
{
    float sum = init;
    for (uint32_t k = 0; k < K; ++k) {
        const float p = weight_at(qtype, row + (k / ORC_QK) * bb, k % ORC_QK) * x[k];
        sum = sum + p;
    }
    return sum;
}

int orc_gemv_r0(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                const float *x, const float *bias, float *y)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    for (uint32_t r = 0; r < rows; ++r)
        y[r] = dot_r0(qtype, w + r * rb, bb, K, x, bias ? bias[r] : 0.0f);
    return 0;
}

int orc_gemv_r0_mt(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                   const float *x, const float *bias, float *y, int nthreads)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (r = 0; r < (long)rows; ++r)
        y[r] = dot_r0(qtype, w + (size_t)r * rb, bb, K, x, bias ? bias[r] : 0.0f);
    (void)nthreads;
    return 0;
}

/* fp64 accumulation over fp32-decoded weights: src/q6cb_q6_reference.hpp:118-132. */
int orc_gemv_r64(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                 const float *x, const float *bias, double *y)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (r = 0; r < (long)rows; ++r) {
        const uint8_t *row = w + (size_t)r * rb;
        float wb[ORC_QK];
        double sum = 0.0;
        for (uint32_t k0 = 0; k0 < K; k0 += ORC_QK) {
            decode_block(qtype, row + (k0 / ORC_QK) * bb, wb);
            for (uint32_t k = 0; k < ORC_QK; ++k)
                sum += (double)wb[k] * (double)x[k0 + k];
        }
        y[r] = sum + (bias ? (double)bias[r] : 0.0);
    }
    return 0;
}

int orc_gemv_r64_xd(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                    const double *x, double *y)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (r = 0; r < (long)rows; ++r) {
        const uint8_t *row = w + (size_t)r * rb;
        float wb[ORC_QK];
        double sum = 0.0;
        for (uint32_t k0 = 0; k0 < K; k0 += ORC_QK) {
            decode_block(qtype, row + (k0 / ORC_QK) * bb, wb);
            for (uint32_t k = 0; k < ORC_QK; ++k)
                sum += (double)wb[k] * x[k0 + k];
        }
        y[r] = sum;
    }
    return 0;
}

/* R64 with both operands rounded to binary16 first (RNE from fp32: the
 * decoded weight, and the input element rounded to fp32): the arithmetic of
 * an fp16-operand matrix unit with exact products and fp64 accumulation. */
int orc_gemv_r64_f16(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                     const double *x, double *y)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    float *x16 = malloc(sizeof(float) * K);
    if (!x16) return -2;
    for (uint32_t k = 0; k < K; ++k) x16[k] = orc_half_to_float(orc_float_to_half_rne((float)x[k]));
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (r = 0; r < (long)rows; ++r) {
        const uint8_t *row = w + (size_t)r * rb;
        float wb[ORC_QK];
        double sum = 0.0;
        for (uint32_t k0 = 0; k0 < K; k0 += ORC_QK) {
            decode_block(qtype, row + (k0 / ORC_QK) * bb, wb);
            for (uint32_t k = 0; k < ORC_QK; ++k)
                sum += (double)orc_half_to_float(orc_float_to_half_rne(wb[k])) * (double)x16[k0 + k];
        }
        y[r] = sum;
    }
    free(x16);
    return 0;
}

int orc_gemv_splitk_r64(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                        uint32_t splits, const float *x, double *part)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb) || splits == 0u) return -1;
    const uint32_t nb = K / ORC_QK;
    const uint32_t bps = (nb + splits - 1u) / splits;
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (r = 0; r < (long)rows; ++r) {
        const uint8_t *row = w + (size_t)r * rb;
        for (uint32_t s = 0; s < splits; ++s) {
            double sum = 0.0;
            const uint32_t b0 = s * bps, b1 = (s + 1u) * bps < nb ? (s + 1u) * bps : nb;
            float wb[ORC_QK];
            for (uint32_t b = b0; b < b1; ++b) {
                decode_block(qtype, row + b * bb, wb);
                for (uint32_t k = 0; k < ORC_QK; ++k)
                    sum += (double)wb[k] * (double)x[b * ORC_QK + k];
            }
            part[(size_t)s * rows + (size_t)r] = sum;
        }
    }
    return 0;
}

/* RMSNorm: fp64 sum of squares, float rsqrt, y = x*inv*w.
 * src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1115-1126. */
void orc_rmsnorm_f32(const float *x, const float *w, uint32_t n, float eps, float *y)
{
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float mean = (float)(ss / (double)n);
    const float inv = 1.0f / sqrtf(mean + eps);
    for (uint32_t i = 0; i < n; ++i) {
        const float t = x[i] * inv;
        y[i] = t * w[i];
    }
}

void orc_rmsnorm_f64(const double *x, const float *w, uint32_t n, double eps, double *y)
{
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const double inv = 1.0 / sqrt(ss / (double)n + eps);
    for (uint32_t i = 0; i < n; ++i) y[i] = x[i] * inv * (double)w[i];
}

/* s = (g / (1 + exp(-g))) * u.  src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1221-1230,
 * shaders/p7_swiglu.comp:7-12. */
void orc_swiglu_f32(const float *g, const float *u, uint32_t n, float *s)
{
    for (uint32_t i = 0; i < n; ++i) {
        const float d = 1.0f + expf(-g[i]);
        const float a = g[i] / d;
        s[i] = a * u[i];
    }
}

void orc_swiglu_f64(const double *g, const double *u, uint32_t n, double *s)
{
    for (uint32_t i = 0; i < n; ++i) s[i] = (g[i] / (1.0 + exp(-g[i]))) * u[i];
}

/* RoPE on ADJACENT pairs (2p, 2p+1) of each head, angle = pos * theta^(-2p/dim).
 * src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1158-1175, shaders/p7_rope_seq.comp:27-37. */
void orc_rope_f32(float *x, uint32_t heads, uint32_t dim, uint32_t pos, float theta)
{
    for (uint32_t h = 0; h < heads; ++h) {
        float *base = x + (size_t)h * dim;
        for (uint32_t p = 0; p < dim / 2u; ++p) {
            const float ex = -2.0f * (float)p / (float)dim;
            const float angle = (float)pos * powf(theta, ex);
            const float c = cosf(angle), s = sinf(angle);
            const float a = base[2 * p], b = base[2 * p + 1];
            const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
            base[2 * p] = ac - bs;
            base[2 * p + 1] = as + bc;
        }
    }
}

void orc_rope_f64(double *x, uint32_t heads, uint32_t dim, uint32_t pos, double theta)
{
    for (uint32_t h = 0; h < heads; ++h) {
        double *base = x + (size_t)h * dim;
        for (uint32_t p = 0; p < dim / 2u; ++p) {
            const double angle = (double)pos * pow(theta, -2.0 * (double)p / (double)dim);
            const double c = cos(angle), s = sin(angle);
            const double a = base[2 * p], b = base[2 * p + 1];
            base[2 * p] = a * c - b * s;
            base[2 * p + 1] = a * s + b * c;
        }
    }
}

/* Top-1/top-2 with strict '>' (ties go to the lowest index); non-finite
 * logits are skipped and clear the finite flag.  src/arcllm_v1_runtime.cpp:132-148. */
void orc_top2(const float *p, uint32_t n, orc_top2_t *r)
{
    r->top1 = r->top2 = 0;
    r->logit1 = r->logit2 = -INFINITY;
    r->finite = 1;
    for (uint32_t i = 0; i < n; ++i) {
        const float v = p[i];
        if (!isfinite(v)) { r->finite = 0; continue; }
        if (v > r->logit1) {
            r->logit2 = r->logit1; r->top2 = r->top1;
            r->logit1 = v; r->top1 = i;
        } else if (v > r->logit2) {
            r->logit2 = v; r->top2 = i;
        }
    }
    if (!isfinite(r->logit1) || !isfinite(r->logit2)) r->finite = 0;
}

void orc_top2_f64(const double *p, uint32_t n, uint32_t *t1, uint32_t *t2, double *l1, double *l2)
{
    *t1 = *t2 = 0;
    *l1 = *l2 = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) {
        const double v = p[i];
        if (!isfinite(v)) continue;
        if (v > *l1) { *l2 = *l1; *t2 = *t1; *l1 = v; *t1 = i; }
        else if (v > *l2) { *l2 = v; *t2 = i; }
    }
}

/* Cached GQA for one query position: fp64 dot products and softmax over
 * positions 0..pos, kv head = q head / (qh/kvh).
 * src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1177-1212 (causal row t = pos),
 * cache addressing shaders/p7_attention_kv_online.comp (layer slice
 * [ctx][kvh][dim]).  Keys and values are the fp16 cache contents. */
void orc_attention_decode_f64(const double *q, const uint16_t *kc, const uint16_t *vc,
                              uint32_t pos, uint32_t qh, uint32_t kvh, uint32_t dim,
                              double *out)
{
    const uint32_t hpk = qh / kvh;
    const double scale = 1.0 / sqrt((double)dim);
    const uint32_t T = pos + 1u;
    long hh;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (hh = 0; hh < (long)qh; ++hh) {
        const uint32_t h = (uint32_t)hh;
        const uint32_t kh = h / hpk;
        double mx = -INFINITY, sum = 0.0;
        /* two passes over the keys: max, then exp-sum and weighted values */
        for (uint32_t t = 0; t < T; ++t) {
            const uint16_t *k = kc + ((size_t)t * kvh + kh) * dim;
            double dot = 0.0;
            for (uint32_t d = 0; d < dim; ++d) dot += q[h * dim + d] * (double)orc_half_to_float(k[d]);
            const double z = dot * scale;
            if (z > mx) mx = z;
        }
        for (uint32_t d = 0; d < dim; ++d) out[h * dim + d] = 0.0;
        for (uint32_t t = 0; t < T; ++t) {
            const uint16_t *k = kc + ((size_t)t * kvh + kh) * dim;
            const uint16_t *v = vc + ((size_t)t * kvh + kh) * dim;
            double dot = 0.0;
            for (uint32_t d = 0; d < dim; ++d) dot += q[h * dim + d] * (double)orc_half_to_float(k[d]);
            const double e = exp(dot * scale - mx);
            sum += e;
            for (uint32_t d = 0; d < dim; ++d) out[h * dim + d] += e * (double)orc_half_to_float(v[d]);
        }
        for (uint32_t d = 0; d < dim; ++d) out[h * dim + d] /= sum;
    }
}

/* One decode step, restating the reference's per-token chain
 * (src/arcllm_v1_runtime.cpp:371-421; CPU helpers
 * src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1115-1230): embedding row
 * (Q4_K decode), then per layer attn RMSNorm, q/k/v GEMV + bias, RoPE on
 * adjacent pairs, K/V stored as fp16 at `pos`, cached GQA over 0..pos,
 * o GEMV + residual, ffn RMSNorm, SwiGLU(gate, up), down GEMV + residual;
 * final RMSNorm and the LM head.  Everything after the decoded weights is
 * fp64; the cache holds fp16(float(value)). */
int orc_decode_step(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos,
                    uint32_t token, double *logits)
{
    return orc_decode_step_ex(m, kc, vc, max_ctx, pos, token, 0, logits);
}

typedef int (*orc_layer_gemv)(int, const uint8_t *, uint32_t, uint32_t, const double *, double *);

int orc_decode_step_ex(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos,
                       uint32_t token, int f16_operands, double *logits)
{
    /* the layer GEMVs (not the LM head) optionally with fp16 operands */
    const orc_layer_gemv lg = f16_operands ? orc_gemv_r64_f16 : orc_gemv_r64_xd;
    const uint32_t H = m->hidden, KVD = m->kv_heads * m->head_dim, F = m->ffn;
    if (pos >= max_ctx || token >= m->vocab || m->layers > ORC_MAX_LAYERS) return -1;
    double *h = malloc(sizeof(double) * H), *xn = malloc(sizeof(double) * H), *q = malloc(sizeof(double) * H);
    double *kk = malloc(sizeof(double) * KVD), *vv = malloc(sizeof(double) * KVD), *at = malloc(sizeof(double) * H);
    double *o = malloc(sizeof(double) * H), *g = malloc(sizeof(double) * F), *u = malloc(sizeof(double) * F);
    double *sw = malloc(sizeof(double) * F);
    if (!h || !xn || !q || !kk || !vv || !at || !o || !g || !u || !sw) return -2;
    const size_t erow = (size_t)(H / ORC_QK) * ORC_Q4K_BLOCK_BYTES;
    for (uint32_t e = 0; e < H; ++e)
        h[e] = (double)orc_q4k_weight(m->emb + (size_t)token * erow + (e / ORC_QK) * ORC_Q4K_BLOCK_BYTES, e % ORC_QK);
    for (uint32_t l = 0; l < m->layers; ++l) {
        uint16_t *kl = kc + (size_t)l * max_ctx * KVD, *vl = vc + (size_t)l * max_ctx * KVD;
        orc_rmsnorm_f64(h, m->attn_norm[l], H, m->eps, xn);
        lg(ORC_Q4_K, m->q[l], H, H, xn, q);
        lg(ORC_Q4_K, m->k[l], KVD, H, xn, kk);
        lg(m->v_type[l], m->v[l], KVD, H, xn, vv);
        for (uint32_t i = 0; i < H; ++i) q[i] += (double)m->qb[l][i];
        for (uint32_t i = 0; i < KVD; ++i) {
            kk[i] += (double)m->kb[l][i];
            vv[i] += (double)m->vb[l][i];
        }
        orc_rope_f64(q, m->q_heads, m->head_dim, pos, m->theta);
        orc_rope_f64(kk, m->kv_heads, m->head_dim, pos, m->theta);
        for (uint32_t i = 0; i < KVD; ++i) {
            kl[(size_t)pos * KVD + i] = orc_float_to_half_rne((float)kk[i]);
            vl[(size_t)pos * KVD + i] = orc_float_to_half_rne((float)vv[i]);
        }
        orc_attention_decode_f64(q, kl, vl, pos, m->q_heads, m->kv_heads, m->head_dim, at);
        lg(ORC_Q4_K, m->o[l], H, H, at, o);
        for (uint32_t i = 0; i < H; ++i) h[i] += o[i];
        orc_rmsnorm_f64(h, m->ffn_norm[l], H, m->eps, xn);
        lg(ORC_Q4_K, m->gate[l], F, H, xn, g);
        lg(ORC_Q4_K, m->up[l], F, H, xn, u);
        orc_swiglu_f64(g, u, F, sw);
        lg(m->down_type[l], m->down[l], H, F, sw, o);
        for (uint32_t i = 0; i < H; ++i) h[i] += o[i];
    }
    orc_rmsnorm_f64(h, m->out_norm, H, m->eps, xn);
    orc_gemv_r64_xd(ORC_Q6_K, m->out, m->vocab, H, xn, logits);
    free(h); free(xn); free(q); free(kk); free(vv); free(at); free(o); free(g); free(u); free(sw);
    return 0;
}


/* ---- the prompt pass batched over n positions ---- */

/* Y[i][r] = sum_k w[r][k] * X[i][k] for i < n, each sum in the order of
 * orc_gemv_r64_xd (f16 = 0) or orc_gemv_r64_f16 (f16 != 0): every weight row
 * is decoded once and applied to all n rows, the n sums of a row advance
 * together over k (independent accumulators, so the order within each sum is
 * unchanged and the results are bit-identical to n single GEMVs). */
static int gemm_rows(int qtype, const uint8_t *w, uint32_t rows, uint32_t K, uint32_t n,
                     const double *X, int f16, double *Y)
{
    size_t rb, bb;
    if (row_bytes(qtype, K, &rb, &bb)) return -1;
    double *XT = malloc(sizeof(double) * (size_t)K * n);
    if (!XT) return -2;
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t k = 0; k < K; ++k) {
            const double x = X[(size_t)i * K + k];
            XT[(size_t)k * n + i] = f16 ? (double)orc_half_to_float(orc_float_to_half_rne((float)x)) : x;
        }
    int fail = 0;
    long r;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16)
#endif
    for (r = 0; r < (long)rows; ++r) {
        double *acc = malloc(sizeof(double) * n);
        if (!acc) { fail = 1; continue; }
        for (uint32_t i = 0; i < n; ++i) acc[i] = 0.0;
        const uint8_t *row = w + (size_t)r * rb;
        float wb[ORC_QK];
        for (uint32_t k0 = 0; k0 < K; k0 += ORC_QK) {
            decode_block(qtype, row + (k0 / ORC_QK) * bb, wb);
            for (uint32_t k = 0; k < ORC_QK; ++k) {
                const double wk = f16 ? (double)orc_half_to_float(orc_float_to_half_rne(wb[k])) : (double)wb[k];
                const double *xt = XT + (size_t)(k0 + k) * n;
                for (uint32_t i = 0; i < n; ++i) acc[i] += wk * xt[i];
            }
        }
        for (uint32_t i = 0; i < n; ++i) Y[(size_t)i * rows + r] = acc[i];
        free(acc);
    }
    free(XT);
    return fail ? -2 : 0;
}

/* n calls of orc_decode_step_ex with teacher forcing (tokens[i] at position
 * pos0 + i), restated layer by layer over all n positions at once: position
 * i's attention reads cache rows 0 .. pos0 + i of the layer, all written
 * before it, so every value equals the stepwise oracle's bit for bit.
 * src/arcllm_v1_runtime.cpp:340-369 (build_prefill, last-token LM head).
 * Returns the logits of the last position. */
int orc_prompt_pass(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos0, uint32_t n,
                    const uint32_t *tokens, int f16_operands, double *logits)
{
    const uint32_t H = m->hidden, KVD = m->kv_heads * m->head_dim, F = m->ffn;
    if (n == 0u || (uint64_t)pos0 + n > max_ctx || m->layers > ORC_MAX_LAYERS) return -1;
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= m->vocab) return -1;
    const size_t nH = (size_t)n * H, nK = (size_t)n * KVD, nF = (size_t)n * F;
    double *h = malloc(sizeof(double) * nH), *xn = malloc(sizeof(double) * nH), *q = malloc(sizeof(double) * nH);
    double *kk = malloc(sizeof(double) * nK), *vv = malloc(sizeof(double) * nK), *at = malloc(sizeof(double) * nH);
    double *o = malloc(sizeof(double) * nH), *g = malloc(sizeof(double) * nF), *u = malloc(sizeof(double) * nF);
    double *sw = malloc(sizeof(double) * nF);
    int rc = 0;
    if (!h || !xn || !q || !kk || !vv || !at || !o || !g || !u || !sw) { rc = -2; goto done; }
    const size_t erow = (size_t)(H / ORC_QK) * ORC_Q4K_BLOCK_BYTES;
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t e = 0; e < H; ++e)
            h[(size_t)i * H + e] = (double)orc_q4k_weight(m->emb + (size_t)tokens[i] * erow + (e / ORC_QK) * ORC_Q4K_BLOCK_BYTES,
                                                          e % ORC_QK);
    for (uint32_t l = 0; l < m->layers; ++l) {
        uint16_t *kl = kc + (size_t)l * max_ctx * KVD, *vl = vc + (size_t)l * max_ctx * KVD;
        for (uint32_t i = 0; i < n; ++i) orc_rmsnorm_f64(h + (size_t)i * H, m->attn_norm[l], H, m->eps, xn + (size_t)i * H);
        if ((rc = gemm_rows(ORC_Q4_K, m->q[l], H, H, n, xn, f16_operands, q))) goto done;
        if ((rc = gemm_rows(ORC_Q4_K, m->k[l], KVD, H, n, xn, f16_operands, kk))) goto done;
        if ((rc = gemm_rows(m->v_type[l], m->v[l], KVD, H, n, xn, f16_operands, vv))) goto done;
        for (uint32_t i = 0; i < n; ++i) {
            double *qi = q + (size_t)i * H, *ki = kk + (size_t)i * KVD, *vi = vv + (size_t)i * KVD;
            const uint32_t pos = pos0 + i;
            for (uint32_t e = 0; e < H; ++e) qi[e] += (double)m->qb[l][e];
            for (uint32_t e = 0; e < KVD; ++e) {
                ki[e] += (double)m->kb[l][e];
                vi[e] += (double)m->vb[l][e];
            }
            orc_rope_f64(qi, m->q_heads, m->head_dim, pos, m->theta);
            orc_rope_f64(ki, m->kv_heads, m->head_dim, pos, m->theta);
            for (uint32_t e = 0; e < KVD; ++e) {
                kl[(size_t)pos * KVD + e] = orc_float_to_half_rne((float)ki[e]);
                vl[(size_t)pos * KVD + e] = orc_float_to_half_rne((float)vi[e]);
            }
        }
        for (uint32_t i = 0; i < n; ++i)
            orc_attention_decode_f64(q + (size_t)i * H, kl, vl, pos0 + i, m->q_heads, m->kv_heads, m->head_dim,
                                     at + (size_t)i * H);
        if ((rc = gemm_rows(ORC_Q4_K, m->o[l], H, H, n, at, f16_operands, o))) goto done;
        for (size_t e = 0; e < nH; ++e) h[e] += o[e];
        for (uint32_t i = 0; i < n; ++i) orc_rmsnorm_f64(h + (size_t)i * H, m->ffn_norm[l], H, m->eps, xn + (size_t)i * H);
        if ((rc = gemm_rows(ORC_Q4_K, m->gate[l], F, H, n, xn, f16_operands, g))) goto done;
        if ((rc = gemm_rows(ORC_Q4_K, m->up[l], F, H, n, xn, f16_operands, u))) goto done;
        for (uint32_t i = 0; i < n; ++i) orc_swiglu_f64(g + (size_t)i * F, u + (size_t)i * F, F, sw + (size_t)i * F);
        if ((rc = gemm_rows(m->down_type[l], m->down[l], H, F, n, sw, f16_operands, o))) goto done;
        for (size_t e = 0; e < nH; ++e) h[e] += o[e];
    }
    orc_rmsnorm_f64(h + (size_t)(n - 1) * H, m->out_norm, H, m->eps, xn);
    rc = orc_gemv_r64_xd(ORC_Q6_K, m->out, m->vocab, H, xn, logits);
done:
    free(h); free(xn); free(q); free(kk); free(vv); free(at); free(o); free(g); free(u); free(sw);
    return rc;
}
