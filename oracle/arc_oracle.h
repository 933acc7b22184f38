/*
 * arc_oracle.h -- CPU oracle for the packed Q4_K/Q6_K decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * runtime's CPU arithmetic for the decode path.  It is the checker the HIP
 * library is compared against; nothing in the product links or loads it.
 * Only tests/, the smoke check and bench.py's CPU-baseline leg use it.
 *
 * Every function names the reference file:line whose behaviour it restates.
 * Build (see oracle/Makefile): gcc -O2 -std=c11 -ffp-contract=off, matching
 * the reference's MSVC /O2 /fp:precise (no FMA contraction).
 */
#ifndef ARC_ORACLE_H
#define ARC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_Q4_K = 12, ORC_Q6_K = 14 };
enum { ORC_Q4K_BLOCK_BYTES = 144, ORC_Q6K_BLOCK_BYTES = 210, ORC_EXEC148_BLOCK_BYTES = 148, ORC_QK = 256 };

/* ---- element decode (bit-exact fp32) ---- */
float orc_half_to_float(uint16_t h);
void orc_q4k_scale_min(const uint8_t *blk, uint32_t j, uint32_t *sc, uint32_t *mn);
uint32_t orc_q4k_code(const uint8_t *blk, uint32_t k);
float orc_q4k_weight(const uint8_t *blk, uint32_t k);
int orc_q6k_code(const uint8_t *blk, uint32_t k, int *scale);
float orc_q6k_weight(const uint8_t *blk, uint32_t k);
/* Dequantise rows x K (K a multiple of 256) of a packed row-major tensor. */
int orc_dequant(int qtype, const uint8_t *w, uint32_t rows, uint32_t K, float *out);

/* ---- EXEC148 (Q4_K route-B representation) ---- */
void orc_exec148_block(const uint8_t *q4, uint8_t *e);
int orc_exec148_tensor(const uint8_t *q4, uint32_t rows, uint32_t K, uint8_t *e);
void orc_q4k_canon(const uint8_t *q4, uint8_t *t);        /* 276-byte canonical tuple */
void orc_exec148_canon(const uint8_t *e, uint8_t *t);
float orc_exec148_weight(const uint8_t *e, uint32_t k);
void orc_sha256(const uint8_t *p, size_t n, uint8_t out[32]);

/* ---- GEMV ---- */
/* R0: serial fp32 per row, per-element decode, sum starts at bias[r] (or 0). */
int orc_gemv_r0(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                const float *x, const float *bias, float *y);
/* Same, rows split over nthreads OpenMP threads (row partition). */
int orc_gemv_r0_mt(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                   const float *x, const float *bias, float *y, int nthreads);
/* R64: fp64 accumulation of fp32-decoded weights times fp32 x, plus bias. */
int orc_gemv_r64(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                 const float *x, const float *bias, double *y);
/* R64 with an fp64 input vector (for inputs produced by the fp64 chain). */
int orc_gemv_r64_xd(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                    const double *x, double *y);
/* R64 with fp16 operands: each decoded weight and each input element
 * (rounded to fp32) rounded to binary16 (RNE), exact products, fp64 sum. */
int orc_gemv_r64_f16(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                     const double *x, double *y);
/* Split-K partials in fp64: part[s*rows + r] = sum over blocks
 * [s*bps, min((s+1)*bps, nb)) of row r. */
int orc_gemv_splitk_r64(int qtype, const uint8_t *w, uint32_t rows, uint32_t K,
                        uint32_t splits, const float *x, double *part);

/* ---- elementwise / normalisation ---- */
void orc_rmsnorm_f32(const float *x, const float *w, uint32_t n, float eps, float *y);
void orc_rmsnorm_f64(const double *x, const float *w, uint32_t n, double eps, double *y);
void orc_swiglu_f32(const float *g, const float *u, uint32_t n, float *s);
void orc_swiglu_f64(const double *g, const double *u, uint32_t n, double *s);
void orc_rope_f32(float *x, uint32_t heads, uint32_t dim, uint32_t pos, float theta);
void orc_rope_f64(double *x, uint32_t heads, uint32_t dim, uint32_t pos, double theta);

/* ---- argmax ---- */
typedef struct {
    uint32_t top1, top2;
    float logit1, logit2;
    int finite;
} orc_top2_t;
void orc_top2(const float *logits, uint32_t n, orc_top2_t *out);
void orc_top2_f64(const double *logits, uint32_t n, uint32_t *top1, uint32_t *top2,
                  double *l1, double *l2);

/* ---- cached GQA attention for one query position (fp64 softmax) ---- */
/* q: [qh*dim]; kc/vc: fp16 bits laid out [ctx][kvh][dim]; attends to
 * positions 0..pos inclusive; out: [qh*dim]. */
void orc_attention_decode_f64(const double *q, const uint16_t *kc, const uint16_t *vc,
                              uint32_t pos, uint32_t qh, uint32_t kvh, uint32_t dim,
                              double *out);
uint16_t orc_float_to_half_rne(float f);

/* ---- one greedy decode step of a Qwen2.5-shaped model, fp64 chain ---- */
#define ORC_MAX_LAYERS 64
typedef struct {
    uint32_t hidden, q_heads, kv_heads, head_dim, ffn, vocab, layers;
    double eps, theta;
    const uint8_t *emb, *out;
    const float *out_norm;
    const float *attn_norm[ORC_MAX_LAYERS], *ffn_norm[ORC_MAX_LAYERS];
    const uint8_t *q[ORC_MAX_LAYERS], *k[ORC_MAX_LAYERS], *v[ORC_MAX_LAYERS], *o[ORC_MAX_LAYERS];
    const float *qb[ORC_MAX_LAYERS], *kb[ORC_MAX_LAYERS], *vb[ORC_MAX_LAYERS];
    const uint8_t *gate[ORC_MAX_LAYERS], *up[ORC_MAX_LAYERS], *down[ORC_MAX_LAYERS];
    int v_type[ORC_MAX_LAYERS], down_type[ORC_MAX_LAYERS];
} orc_model;
/* Feeds `token` at position `pos`: writes this position's K and V (fp16 bits
 * of the fp32-rounded values) into kc/vc ([layer][max_ctx][kv_heads*head_dim])
 * and returns the logits.  Returns 0 on success. */
int orc_decode_step(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos,
                    uint32_t token, double *logits);
/* The same with f16_operands != 0: every layer GEMV (q, k, v, o, gate, up,
 * down; not the LM head) uses orc_gemv_r64_f16 -- the arithmetic of the
 * batched MFMA prompt pass. */
int orc_decode_step_ex(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos,
                       uint32_t token, int f16_operands, double *logits);
/* The same as n calls of orc_decode_step_ex with tokens[i] at position
 * pos0 + i (teacher forcing), computed layer by layer over all n positions
 * (each weight row decoded once per layer); bit-identical results.  Returns
 * the logits of the last position. */
int orc_prompt_pass(const orc_model *m, uint16_t *kc, uint16_t *vc, uint32_t max_ctx, uint32_t pos0, uint32_t n,
                    const uint32_t *tokens, int f16_operands, double *logits);

#ifdef __cplusplus
}
#endif
#endif
