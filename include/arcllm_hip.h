/*
 * arcllm_hip.h -- C ABI of the MI355X (gfx950) backend for ArcLLM's packed
 * Q4_K/Q6_K decode hot path.
 *
 * Plain C: pointers, sizes and int status codes.  No exception and no C++
 * or torch type crosses this boundary.  Every call returns ARC_OK (0) or an
 * arc_status code; arc_last_error() then holds a thread-local message.
 *
 * Device pointers come from arc_malloc (or any hipMalloc'd memory of the same
 * process).  Kernel entry points are asynchronous on the given stream (NULL =
 * the default stream); results are visible after arc_stream_synchronize /
 * arc_synchronize.  A stream (and everything launched on it) is used by one
 * host thread at a time.
 *
 * Packed tensors are GGUF row-major: a weight of rows x K (K a multiple of
 * 256) is rows * (K/256) super-blocks, 144 bytes each for Q4_K
 *   (d f16 @0, dmin f16 @2, 12 bytes 6-bit scales/mins @4, 128 bytes nibbles @16)
 * and 210 bytes each for Q6_K
 *   (ql[128] @0, qh[64] @128, int8 scales[16] @192, d f16 @208).
 * Q4_K tensors must start 16-byte aligned, Q6_K tensors 2-byte aligned (GGUF
 * data is 32-byte aligned).  fp32 vectors must be 16-byte aligned.
 *
 * Reference interfaces replaced (minhtri22/ArcLLM):
 *   device runtime   VkRuntime::{init,make_buffer,execute_prepared}
 *                    src/arcllm_v1_vulkan_runtime_support.h:498-704
 *   kernel contract  PCGemm{n,rows,batch,row_bytes,add_bias,w_base_bytes,bias_base}
 *                    src/arcllm_v1_runtime.cpp:268-277, dispatches :371-421
 */
#ifndef ARCLLM_HIP_H
#define ARCLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum arc_status {
    ARC_OK = 0,
    ARC_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size or alignment */
    ARC_ERR_UNSUPPORTED = 2,      /* shape or type outside what the kernels implement */
    ARC_ERR_DEVICE = 3,           /* HIP runtime error (message in arc_last_error) */
    ARC_ERR_OUT_OF_MEMORY = 4,
    ARC_ERR_NO_DEVICE = 5
} arc_status;

typedef enum arc_qtype {
    ARC_Q4_K = 12,     /* ggml type id of Q4_K (src/arcllm_v1_runtime.cpp:168) */
    ARC_Q6_K = 14,     /* ggml type id of Q6_K */
    ARC_EXEC148 = 148, /* Q4_K repacked as EXEC148 (src/q4_down_exec148_materializer.h:14-17):
                          accepted by arc_gemv and arc_gemv_splitk */
    ARC_Q6_K_PADDED = 214 /* Q6_K with 2 zero bytes after each 210-byte block, so every
                             block starts at a dword boundary (written by arc_q6_pad; the
                             model arena holds its Q6_K tensors this way).  Accepted by
                             arc_dequant, arc_gemv, arc_gemv_splitk and arc_lmhead_argmax.
                             No counterpart in the reference: a device-side layout of
                             the same blocks, for dword-aligned loads. */
} arc_qtype;

typedef void *arc_stream_t; /* a hipStream_t; NULL is the default stream */
typedef void *arc_event_t;  /* a hipEvent_t */

/* ---------------------------------------------------------------- runtime */
const char *arc_last_error(void);
const char *arc_version(void);
/* Number of HIP devices visible (0 without a GPU; never an error then). */
int arc_device_count(int *count);
int arc_set_device(int device);
/* Device name and gfx architecture string of the current device. */
int arc_device_info(char *name, size_t name_len, char *arch, size_t arch_len);

int arc_malloc(void **ptr, size_t bytes);
int arc_free(void *ptr);
/* Device allocations the library has made in this process (model and
 * session arenas, arc_malloc).  No counterpart in the reference: lets a
 * caller check that decoding, the prompt pass and route changes allocate
 * nothing once a session exists. */
int arc_device_allocations(uint64_t *count);
int arc_memcpy_htod(void *dst, const void *src, size_t bytes, arc_stream_t stream);
int arc_memcpy_dtoh(void *dst, const void *src, size_t bytes, arc_stream_t stream);
int arc_memcpy_dtod(void *dst, const void *src, size_t bytes, arc_stream_t stream);
int arc_memset(void *dst, int value, size_t bytes, arc_stream_t stream);
int arc_synchronize(void);

int arc_stream_create(arc_stream_t *stream);
int arc_stream_destroy(arc_stream_t stream);
int arc_stream_synchronize(arc_stream_t stream);
int arc_event_create(arc_event_t *event);
int arc_event_destroy(arc_event_t event);
int arc_event_record(arc_event_t event, arc_stream_t stream);
int arc_event_elapsed_ms(arc_event_t start, arc_event_t stop, float *ms);

/* ------------------------------------------------------- element decode */
/* out[r*K + k] = fp32 weight, bit-exact with the reference CPU decode:
 * Q4_K  w = d*sc*q - dmin*mn   (src/sa1_component_benchmark.cpp:105-116)
 * Q6_K  w = d*scale*q          (src/q6cb_q6_reference.hpp:49-91)
 * each product/difference rounded separately, left to right. */
int arc_dequant(int qtype, const void *w, uint32_t rows, uint32_t K, float *out,
                arc_stream_t stream);

/* Padded image of a Q6_K tensor (rows x K; device pointers, q6 2-byte and
 * padded 4-byte aligned, not overlapping): rows*(K/256) blocks of 212 bytes,
 * each the 210-byte block followed by two zero bytes.  No counterpart in the
 * reference (it reads GGUF blocks in place): the loads of a padded block
 * are dword-aligned, which the Q6_K GEMVs run faster on. */
int arc_q6_pad(const void *q6, uint32_t rows, uint32_t K, void *padded, arc_stream_t stream);

/* ------------------------------------------------------------------ GEMV */
/* y[r] = sum_k w[r,k] * x[k] (+ bias[r] when bias != NULL), fp32 accumulate.
 * Replaces the decode q/k/v/o, gate/up and Q6 down dispatches of
 * shaders/p7_q4k_gemm_2d.comp, shaders/sa1_q4k_subgroup_splitk.comp and
 * shaders/p7_q6k_gemm_2d.comp (src/arcllm_v1_runtime.cpp:380-413). */
int arc_gemv(int qtype, const void *w, uint32_t rows, uint32_t K, const float *x,
             const float *bias, float *y, arc_stream_t stream);

/* Fused FFN gate/up + SwiGLU on Q4_K: s[r] = silu(gate[r].x) * (up[r].x),
 * silu(g) = g / (1 + exp(-g)).  Replaces the ffn_gate + ffn_up + swiglu
 * dispatches (src/arcllm_v1_runtime.cpp:390-409, shaders/p7_swiglu.comp). */
int arc_gateup_swiglu(int qtype, const void *w_gate, const void *w_up, uint32_t rows,
                      uint32_t K, const float *x, float *s, arc_stream_t stream);

/* Split-K GEMV with a deterministic two-pass reduction.  Pass 1 writes
 * partials[r*used + j] for split j over super-block columns
 * [j*bps, min((j+1)*bps, K/256)), bps = ceil((K/256)/splits); pass 2 sums
 * the partials of each row in order j = 0..used-1 (no atomics), and adds
 * residual[r] last when residual != NULL.  used = ceil((K/256)/bps) (splits
 * that would own no column are dropped).  partials holds splits*rows floats.
 * With one column per split (bps = 1, K/256 <= 80) both passes run in one
 * launch: the wave that computes a row's partials stores them and adds them
 * in the same order; otherwise pass 2 is a second launch.  Results are
 * identical either way.
 * Replaces the ffn_down dispatch and the Q4 down backend route
 * (src/arcllm_v1_runtime.cpp:405-413,
 *  src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:347-386). */
int arc_gemv_splitk(int qtype, const void *w, uint32_t rows, uint32_t K, uint32_t splits,
                    const float *x, float *partials, const float *residual, float *y,
                    arc_stream_t stream);

/* ---------------------------------------------------------------- EXEC148 */
/* EXEC148 image of a Q4_K tensor (rows x K, device pointers, both 16-byte
 * aligned): rows*(K/256) blocks of 148 bytes, d and dmin bytes, the eight
 * unpacked (sc, mn) byte pairs, then the 256 codes two per byte in element
 * order.  Replaces the P1 acquisition path of the Q4-down backend
 * (shaders/b1_2_exec148_gpu_materialize.comp,
 * src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:120-141, 218-224) and
 * materialize_tensor (src/q4_down_exec148_materializer.h:17). */
int arc_exec148_materialize(const void *q4, uint32_t rows, uint32_t K, void *exec, arc_stream_t stream);

/* *mismatched = number of EXEC148 blocks whose canonical tuple (d, dmin,
 * (sc, mn) x 8, 256 codes) differs from their Q4_K source block's: 0 means
 * the image is exact.  The per-block check of validate_tensor
 * (src/q4_down_exec148_materializer.h:21-22); synchronous on `stream`. */
int arc_exec148_validate(const void *q4, const void *exec, uint32_t rows, uint32_t K, uint64_t *mismatched,
                         arc_stream_t stream);
/* The same check over `count` tensor pairs of one shape (q4[i] against
 * exec[i]) with one result: *mismatched = mismatched blocks over all pairs;
 * one synchronization (the whole family of a model in one call, as
 * validate_image does for its 14 layers,
 * src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:97-119). */
int arc_exec148_validate_many(const void *const *q4, const void *const *exec, uint32_t count, uint32_t rows,
                              uint32_t K, uint64_t *mismatched, arc_stream_t stream);

/* ------------------------------------------------------- norm / LM head */
/* y = x * rsqrt(mean(x^2) + eps) * w over n elements (shaders/p7_rmsnorm_seq.comp). */
int arc_rmsnorm(const float *x, const float *w, uint32_t n, float eps, float *y,
                arc_stream_t stream);

/* Bytes of device workspace arc_lmhead_argmax needs for `rows` vocabulary
 * rows; 0 for a qtype or shape the LM head does not take. */
size_t arc_lmhead_workspace_bytes(int qtype, uint32_t rows, uint32_t K);

/* Greedy LM-head step on the GPU: x = RMSNorm(h; normw, eps), logits =
 * W.x, out[0] = argmax with ties to the LOWEST index over finite logits,
 * out[1] = number of non-finite logits (0 when all are finite).
 * logits may be NULL (not materialised).  workspace: device memory of
 * arc_lmhead_workspace_bytes() bytes.  normw == NULL skips the norm.
 * Replaces append_lm (src/arcllm_v1_runtime.cpp:285-291,
 * shaders/p8q1_lmhead_q6k_segmented_chunk.comp) plus the host argmax
 * runtime_top2 (src/arcllm_v1_runtime.cpp:132-148,499-504). */
int arc_lmhead_argmax(int qtype, const void *w, uint32_t rows, uint32_t K, const float *h,
                      const float *normw, float eps, float *logits, void *workspace,
                      uint32_t *out, arc_stream_t stream);

/* arc_lmhead_argmax without a workspace, for callers that cannot allocate
 * device memory (code under stream/graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, kernels and results as arc_lmhead_argmax; the per-workgroup
 * argmax partials live in a static device array of 8192 entries (128 KB,
 * held by each GPU the library runs on until the process ends).  Calls no
 * allocator.  A launch that would need more than 8192 workgroup results is
 * rejected with ARC_ERR_UNSUPPORTED (the grid never exceeds the resident
 * workgroup count, at most 8192 on MI355X).  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (concurrent streams or threads)
 * race and must be serialised by the caller. */
int arc_lmhead_argmax_noalloc(int qtype, const void *w, uint32_t rows, uint32_t K, const float *h,
                              const float *normw, float eps, float *logits, uint32_t *out,
                              arc_stream_t stream);

/* Bytes of device workspace arc_attention_decode needs (split partials,
 * arrival counters, control block); 0 for unsupported head counts. */
size_t arc_attention_workspace_bytes(uint32_t kv_heads, uint32_t hpk);

/* Cached GQA attention of one decode position, with the decode step's kernel
 * and split plan: out[h*128 + d] = sum_t softmax_t(q_h . k_t / sqrt(128))
 * v_t[d] over positions t < T, query head h reading kv head h / hpk.
 * q, out: fp32 [kv_heads*hpk*128] (16-byte aligned); kc, vc: fp16
 * [max_ctx][kv_heads*128] (16-byte aligned); 1 <= T <= max_ctx <= 32768;
 * hpk 1..8.  workspace: arc_attention_workspace_bytes() bytes of device
 * memory (256-byte aligned), owned by the caller and reset by the call.
 * Replaces the decode attention dispatch of build_decode
 * (src/arcllm_v1_runtime.cpp:371-421, shaders/p7_attention_kv_online.comp;
 * semantics src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1177-1212). */
int arc_attention_decode(const float *q, const void *kc, const void *vc, uint32_t kv_heads, uint32_t hpk,
                         uint32_t max_ctx, uint32_t T, float *out, void *workspace, arc_stream_t stream);

/* Bytes of device workspace the prompt-pass projection entry points need for
 * an N x K weight (fp16 X staging of 256 rows and the split-K partials). */
size_t arc_prefill_gemm_workspace_bytes(uint32_t N, uint32_t K);

/* The prompt pass's projection GEMM, with its kernel and split-K plan:
 * y[m][n] = sum_k x[m][k] w[n][k] for m < M <= 256, fp16 operands (each
 * weight decoded in fp32 and rounded to fp16), fp32 accumulation, the split
 * partials added in split order.  x: fp16 bits [M][K]; w: [N x K] Q4_K or
 * ARC_Q6_K_PADDED; y: fp32 [M][N].  Replaces the p7c/p7g tiled GEMM
 * dispatches of build_prefill (src/arcllm_v1_runtime.cpp:340-369). */
int arc_prefill_gemm(int qtype, const void *w, uint32_t N, uint32_t K, const uint16_t *x, uint32_t M, float *y,
                     void *workspace, arc_stream_t stream);

/* The prompt pass's fused gate/up + SwiGLU GEMM (Q4_K gate and up):
 * s[m][n] = fp16(silu(g) * u), g = x w_gate^T, u = x w_up^T, for m < M <= 256.
 * x: fp16 bits [M][K]; s: fp16 bits [M][N].  workspace as for
 * arc_prefill_gemm.  Replaces p7l (src/arcllm_v1_runtime.cpp:340-369). */
int arc_prefill_gateup(const void *w_gate, const void *w_up, uint32_t N, uint32_t K, const uint16_t *x, uint32_t M,
                       uint16_t *s, void *workspace, arc_stream_t stream);

/* The prompt pass's q|k|v launch (Q4_K q and k, v Q4_K or ARC_Q6_K_PADDED):
 * y[m][0..H) = x wq^T, y[m][H..H+kvd) = x wk^T, y[m][H+kvd..H+2kvd) = x wv^T
 * (before bias and RoPE), fp32 [M][H + 2*kvd].  workspace:
 * arc_prefill_gemm_workspace_bytes(H + 2*kvd, K). */
int arc_prefill_qkv(const void *wq, const void *wk, const void *wv, int v_qtype, uint32_t H, uint32_t kvd, uint32_t K,
                    const uint16_t *x, uint32_t M, float *y, void *workspace, arc_stream_t stream);

/* The prompt pass's causal GQA, with its kernel: prompt row m (position
 * pos0 + m, m < M) attends to cache positions 0 .. pos0 + m.  q: fp32
 * [M][kv_heads * hpk * 128] (RoPE applied); kc, vc: fp16 bits
 * [max_ctx][kv_heads * 128], rows 0 .. pos0 + M - 1 written; x: fp16 bits,
 * row m at x + m * ldx (ldx >= kv_heads * hpk * 128).  mfma = 1: the MFMA
 * kernel the prompt pass runs, 0: the VALU kernel.  Replaces the per-row
 * attention of build_prefill (src/arcllm_v1_runtime.cpp:340-369, with the
 * semantics of src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1177-1212). */
int arc_prefill_attention(const float *q, const void *kc, const void *vc, uint32_t kv_heads, uint32_t hpk,
                          uint32_t max_ctx, uint32_t pos0, uint32_t M, uint16_t *x, uint32_t ldx, int mfma,
                          arc_stream_t stream);

/* Tuning hook: force the GEMV lane layout for later launches on this host
 * thread (bs = super-block quads per row: 1,2,4,8,16; rpl = rows per lane:
 * 1,2,4).  bs = 0 restores the automatic choice. */
int arc_tune_force(int bs, int rpl);
/* Tuning hook: waves per GEMV workgroup (4 or 8) for later launches on this
 * host thread; 0 restores the automatic choice. */
int arc_tune_waves(int waves);
/* Tuning hook for whole-row Q4_K GEMVs (plain, gate/up; K <= 3584)
 * launched or captured later on this host thread: -1 (default) automatic,
 * 0 keeps every Q4_K launch on the quad layout, 1 takes the row-stream
 * kernel. */
int arc_tune_rowstream(int mode);
/* Tuning hook for decode attention launched or captured later on this host
 * thread: waves per workgroup (4 or 8; a chunk is 16 positions per wave)
 * and the least chunks one split (workgroup) covers; 0 = automatic. */
int arc_tune_attention(int waves, int min_chunks_per_split);
/* Tuning hook: the lane layout (bs quads per row, rpl rows per lane; bs = 0
 * keeps the step's own) and waves per workgroup (0 = the step's own) of one
 * GEMV of decode steps captured later on this host thread: kind 0 the o
 * projection, 1 the fused gate/up, 2 the down projection, 3 the LM head. */
int arc_tune_decode(int kind, int bs, int rpl, int waves);
/* Tuning hook: the prompt pass's attention kernel for passes run later on
 * this host thread: 1 (default) on MFMA (query blocks of 32 rows per q
 * head, key chunks over 4 waves), 0 the VALU kernel (one query row per
 * workgroup and kv head). */
int arc_tune_prefill_attention(int mfma);
/* Tuning hook: 1 (default) runs each layer's attention and o projection of
 * decode steps captured later on this host thread as one launch, whose o
 * workgroups wait (bounded) for the attention's output; 0 as two launches;
 * 2 (test of the bounded wait) as one launch whose attention never signals:
 * every wait gives up and the decode call returns ARC_ERR_DEVICE. */
int arc_tune_fuse_attn_o(int on);

/* Diagnostic: streaming read of `bytes` (16-byte aligned) with `grid`
 * workgroups of 256 lanes, 16 bytes per lane access, xor-folded into
 * out[grid*256] (device).  Measures the practical HBM read ceiling. */
int arc_probe_read(const void *p, size_t bytes, uint32_t *out, uint32_t grid, arc_stream_t stream);
/* The same probe with `loads` (1, 2, 4 or 8) independent 16-byte loads per
 * lane in flight per iteration.  No counterpart in the reference: a
 * measurement aid of this build. */
int arc_probe_read_unrolled(const void *p, size_t bytes, uint32_t *out, uint32_t grid, int loads,
                            arc_stream_t stream);
/* The one-load probe with the non-temporal cache policy on its loads (the
 * same chunks folded into the same outputs as arc_probe_read).  No
 * counterpart in the reference: a measurement aid of this build. */
int arc_probe_read_nt(const void *p, size_t bytes, uint32_t *out, uint32_t grid, arc_stream_t stream);

/* ------------------------------------------------------ synthetic inputs */
/* Host-side, deterministic generators for seeded synthetic packed tensors
 * (no GPU needed).  Each super-block draws from splitmix64 seeded by
 * (seed, stream, block index), so any slice can be regenerated alone.
 * Q4_K: d = f16(|N(0, d_sigma)|), dmin = f16(|N(0, dmin_sigma)|), the 140
 *       scale/min and nibble bytes uniform.
 * Q6_K: ql/qh uniform bits, int8 scales uniform in [-32, 31],
 *       d = f16(|N(0, d_sigma)|).
 * `out` is host memory of rows*(K/256)*block_bytes bytes. */
int arc_synth_packed(int qtype, uint64_t seed, uint64_t stream, uint32_t rows, uint32_t K,
                     float d_sigma, float dmin_sigma, void *out);
/* out[i] = float(mean + sigma * N(0,1)), element i drawn from (seed, stream, i). */
int arc_synth_normal(uint64_t seed, uint64_t stream, size_t n, float mean, float sigma,
                     float *out);

/* ------------------------------------------------------- decode runtime */
/* A Qwen2.5-shaped model (the reference's only model family,
 * src/arcllm_v1_runtime.cpp:164-211): per layer attn_norm, attn_q/k (Q4_K),
 * attn_v (Q4_K or Q6_K), q/k/v biases, attn_output (Q4_K), ffn_norm,
 * ffn_gate/up (Q4_K), ffn_down (Q4_K or Q6_K); token_embd (Q4_K),
 * output_norm, output (Q6_K).  Norm weights and biases are fp32. */
#define ARC_MAX_LAYERS 64

typedef struct arc_model_dims {
    uint32_t hidden, q_heads, kv_heads, head_dim, ffn, vocab, layers;
    float rms_eps, rope_theta;
    int32_t v_type[ARC_MAX_LAYERS];    /* ARC_Q4_K or ARC_Q6_K per layer */
    int32_t down_type[ARC_MAX_LAYERS];
} arc_model_dims;

/* Tensor slots: global tensors (layer = -1) and per-layer tensors. */
enum { ARC_T_TOKEN_EMBD = 0, ARC_T_OUTPUT = 1, ARC_T_OUTPUT_NORM = 2, ARC_T_GLOBAL_COUNT = 3 };
enum {
    ARC_T_ATTN_NORM = 0, ARC_T_ATTN_Q = 1, ARC_T_ATTN_K = 2, ARC_T_ATTN_V = 3,
    ARC_T_ATTN_Q_BIAS = 4, ARC_T_ATTN_K_BIAS = 5, ARC_T_ATTN_V_BIAS = 6, ARC_T_ATTN_O = 7,
    ARC_T_FFN_NORM = 8, ARC_T_FFN_GATE = 9, ARC_T_FFN_UP = 10, ARC_T_FFN_DOWN = 11,
    ARC_T_LAYER_COUNT = 12
};

typedef struct arc_model arc_model;
typedef struct arc_session arc_session;

/* Qwen2.5-7B dims: hidden 3584, 28/4 heads of 128, ffn 18944, vocab 152064,
 * 28 layers, eps 1e-6, theta 1e6, attn_v and ffn_down Q6_K. */
int arc_model_dims_qwen25_7b(arc_model_dims *dims);
/* qtype (ARC_Q4_K, ARC_Q6_K, or 0 for an fp32 vector of K floats), shape
 * and byte size of one tensor slot (layer -1 for the global tensors). */
int arc_model_tensor_info(const arc_model_dims *dims, int layer, int which, int *qtype, uint32_t *rows,
                          uint32_t *K, uint64_t *bytes);
/* Random-init contents of one tensor slot, host memory: packed tensors as
 * arc_synth_packed with d_sigma 1e-4, dmin_sigma 7.5e-4 (zero-mean Q4_K rows,
 * weight std ~0.03), norm weights N(1, 0.05), biases N(0, 0.1);
 * stream = slot for globals, 100 + 16*layer + slot. */
int arc_model_synth_tensor(const arc_model_dims *dims, uint64_t seed, int layer, int which, void *out);
/* Upload a model: tensors[ARC_T_GLOBAL_COUNT + layer*ARC_T_LAYER_COUNT + slot]
 * (globals first) are host pointers to each slot's bytes (GGUF layout). */
int arc_model_create(const arc_model_dims *dims, const void *const *tensors, arc_model **out);
int arc_model_create_synthetic(const arc_model_dims *dims, uint64_t seed, arc_model **out);
int arc_model_destroy(arc_model *model);
uint64_t arc_model_weight_bytes(const arc_model *model);
/* A model is one device allocation (its arena): every tensor at a 256-byte
 * aligned offset in slot order, then, when some ffn_down is Q4_K, a reserve
 * for the EXEC148 image of every Q4_K ffn_down (slot i = the i-th such layer
 * in layer order, at base + i * slot_stride).  The Q4_K FFN-down backend
 * builds its representation there instead of allocating at acquisition
 * (the reference allocates it then, src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:238).
 * slots = 0 and base = NULL when no ffn_down is Q4_K. */
int arc_model_exec148_reserve(const arc_model *model, void **base, uint64_t *slot_stride, uint32_t *slots);

/* A decode session: fp16 KV cache [layer][max_ctx][kv_heads*128] for K and
 * V (GPU-resident across steps), working buffers and the captured step.
 * max_ctx is 1..32768 (ARC_ERR_UNSUPPORTED above). */
int arc_session_create(arc_model *model, uint32_t max_ctx, arc_session **out);
int arc_session_destroy(arc_session *session);

/* Residency plan of a session and its model, in bytes: the reference's
 * weight / KV / working accounting and its budget check
 * (src/arcllm_v1_runtime.cpp:227-266).  A session is one device allocation
 * (the KV cache, then the decode step's and the prompt pass's working
 * memory) planned in full at arc_session_create; nothing is allocated on the
 * device after that.  arc_model_create and arc_session_create each refuse,
 * with ARC_ERR_OUT_OF_MEMORY, a plan that does not fit the free device
 * memory less a 512 MiB headroom. */
typedef struct arc_residency {
    uint64_t weight_bytes;          /* tensor bytes of the model */
    uint64_t model_arena_bytes;     /* the model's allocation: tensors, alignment, EXEC148 reserve */
    uint64_t exec148_reserve_bytes; /* of which the EXEC148 reserve */
    uint64_t kv_bytes;              /* fp16 K and V cache */
    uint64_t working_bytes;         /* the rest of the session's allocation */
    uint64_t total_bytes;           /* model arena + kv + working */
} arc_residency;
int arc_session_residency(const arc_session *session, arc_residency *out);
/* Device pointers of one layer's K and V cache. */
int arc_session_kv(arc_session *session, uint32_t layer, void **k, void **v);
/* Positions [0, ctx) of every layer's K and V := fp16(N(0, 1)), drawn from
 * (seed, stream 1000000 + 2*layer + {0: K, 1: V}). */
int arc_session_fill_kv(arc_session *session, uint32_t ctx, uint64_t seed);

#define ARC_DECODE_LOGITS 1   /* keep the last step's logits (arc_session_logits) */
#define ARC_DECODE_NO_GRAPH 2 /* launch kernels one by one instead of the captured graph */
/* Greedy decode of n_steps tokens: step i feeds the current token at
 * position pos + i and writes the argmax (ties to the lowest id) to
 * out_tokens[i] (host, may be NULL); the next step feeds that token.
 * *nonfinite = number of non-finite logits seen.  Synchronous. */
int arc_session_decode(arc_session *session, uint32_t token, uint32_t pos, uint32_t n_steps, int flags,
                       uint32_t *out_tokens, uint32_t *nonfinite);
/* Prompt processing: tokens[i] at position pos0 + i for i < n, writing every
 * position's K and V; *next_token = the argmax after the last prompt token,
 * *nonfinite = non-finite logits at that last position.  n >= 2 runs the
 * batched prompt pass (src/arcllm_v1_runtime.cpp:340-369): MFMA GEMMs over
 * all prompt rows (fp16 operands: X and the dequantised weights, fp32
 * accumulation), causal GQA, the LM head on the last row only; passes of 256
 * rows.  n = 1 or ARC_PREFILL_STEPWISE replays the decode step per token
 * with teacher forcing instead.  Synchronous. */
#define ARC_PREFILL_STEPWISE 4
int arc_session_prefill(arc_session *session, const uint32_t *tokens, uint32_t n, uint32_t pos0, int flags,
                        uint32_t *next_token, uint32_t *nonfinite);
/* Logits of the last step run with ARC_DECODE_LOGITS (host, vocab floats). */
int arc_session_logits(arc_session *session, float *host_logits);
uint32_t arc_session_kernels_per_step(const arc_session *session);

/* Device pointer of a model tensor (layer < 0: the global tensors
 * ARC_T_TOKEN_EMBD .. ARC_T_OUTPUT_NORM; otherwise slot `which` of `layer`),
 * in the layout of arc_model_create, except that Q6_K tensors are held as
 * ARC_Q6_K_PADDED.  Used by the Q4_K FFN-down backend to build the EXEC148
 * representation on the GPU. */
int arc_model_tensor_device(const arc_model *model, int layer, int which, const void **ptr);

/* Route B of the Q4_K FFN-down capability for one decode layer: the decode
 * step of this session multiplies by `exec148` (the EXEC148 image of that
 * layer's Q4_K ffn_down, see arc_exec148_materialize; 16-byte aligned, kept
 * alive by the caller while routed) instead of the packed tensor; NULL
 * returns the layer to route A.  A change takes effect at the next decode
 * call (the captured step is rebuilt).  The reference's route selection,
 * src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:347-386 (append_ffn_down_op). */
int arc_session_route_down(arc_session *session, uint32_t layer, const void *exec148);
/* Kernel launches of the last arc_session_prefill call. */
uint32_t arc_session_prefill_kernels(const arc_session *session);

#ifdef __cplusplus
}
#endif
#endif /* ARCLLM_HIP_H */
