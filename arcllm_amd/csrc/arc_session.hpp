// arc_session.hpp -- host objects of the decode runtime: the uploaded model
// and a decode session (KV cache, working buffers, captured step), shared by
// the decode step (arc_decode.hip) and the batched prompt pass
// (arc_prefill.hip).
#pragma once

#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <vector>

namespace arc {

constexpr int kHeadDim = 128;
constexpr int kChunk = 64;       // positions per attention chunk
constexpr int kMaxHpk = 8;       // q heads per kv head
constexpr int kMaxChunks = 512;  // contexts up to 32768 positions
constexpr int kMaxSplits = 64;   // attention workgroups per kv head
// Arrival counters of the decode step's last-arriver hand-offs (session
// memory, zero between launches): one per kv head for attention, one for
// the LM-head argmax.
constexpr int kCounterAttn = 0;
constexpr int kCounterLmHead = 64;
constexpr int kCounters = 65;

struct PrefillBufs;                  // arc_prefill.hip
void destroy_prefill(PrefillBufs*);  // arc_prefill.hip

struct Layer {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm, *qb, *kb, *vb;
    int v_type, down_type;
};

}  // namespace arc

struct arc_model {
    arc_model_dims dims{};
    std::vector<void*> allocations;  // device memory owned by the model
    const uint8_t* emb = nullptr;
    const uint8_t* out = nullptr;
    const float* out_norm = nullptr;
    std::vector<arc::Layer> layers;
    uint64_t weight_bytes = 0;

    ~arc_model()
    {
        for (void* p : allocations) (void)hipFree(p);
    }
};

struct arc_session {
    arc_model* model = nullptr;
    uint32_t max_ctx = 0;
    uint32_t max_chunks = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> allocations;
    _Float16* kcache = nullptr;  // [layers][max_ctx][kv_dim]
    _Float16* vcache = nullptr;
    float *h = nullptr, *h1 = nullptr, *q = nullptr, *attn = nullptr, *s = nullptr, *logits = nullptr;
    float *apo = nullptr, *apml = nullptr;  // attention split partials [kv_heads][kMaxSplits][hpk][...]
    uint32_t* counters = nullptr;            // kCounters arrival counters
    float2* rope = nullptr;  // [max_ctx][64] (cos, sin) of pos * theta^(-2p/128)
    arc::ArgBest* best = nullptr;
    uint32_t best_cap = 0;
    arc::DecodeCtl* ctl = nullptr;
    uint32_t* out_tokens = nullptr;
    uint32_t out_cap = 0;
    arc::DecodeCtl* host_ctl = nullptr;  // pinned staging: [0] download, [1 + i] upload of step i
    uint32_t* host_tokens = nullptr;     // pinned staging, out_cap entries
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool graph_logits = false;
    uint32_t kernels_per_step = 0;
    arc::PrefillBufs* pf = nullptr;  // batched prompt-pass buffers, made on first use
    uint32_t prefill_kernels = 0;    // launches of the last arc_session_prefill call
    // per layer: EXEC148 image of a Q4_K ffn_down the decode step reads
    // instead of the packed tensor (route B), or null (route A)
    std::vector<const uint8_t*> down_e148;

    ~arc_session()
    {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (stream) (void)hipStreamDestroy(stream);
        for (void* p : allocations) (void)hipFree(p);
        if (host_ctl) (void)hipHostFree(host_ctl);
        if (host_tokens) (void)hipHostFree(host_tokens);
        arc::destroy_prefill(pf);
    }
};

namespace arc {

// Output RMSNorm + LM head + argmax of the hidden row x, then the next-token
// kernel (token, position + 1, non-finite count into the control block).
// arc_decode.hip.
int launch_lm_head(arc_session* S, const float* x, bool logits, hipStream_t st);

// The batched prompt pass: tokens (host) at positions pos0 .. pos0+n-1, the
// control block left as after the last prompt token.  arc_prefill.hip.
int run_prefill(arc_session* S, const uint32_t* tokens, uint32_t n, uint32_t pos0, bool logits);

}  // namespace arc
