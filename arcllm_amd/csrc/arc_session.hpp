// arc_session.hpp -- host objects of the decode runtime: the uploaded model
// and a decode session (KV cache, working buffers, captured step), shared by
// the decode step (arc_decode.hip) and the batched prompt pass
// (arc_prefill.hip).
#pragma once

#include "arc_device.hpp"
#include "../../include/arcllm_hip.h"

#include <functional>
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

// ------------------------------------------------------------------ arenas
// One device allocation carved into 256-byte aligned pieces.  While planning,
// place() reserves a piece and remembers where its address goes; commit()
// checks the total against the free device memory, makes the one allocation
// and hands every piece its address.
class ArenaPlan {
public:
    static constexpr uint64_t kAlign = 256;

    template <typename T>
    void place(T** slot, uint64_t bytes)
    {
        pieces_.push_back(Piece{offset_, [slot](uint8_t* at) { *slot = reinterpret_cast<T*>(at); }});
        offset_ += round_up(bytes);
    }
    void pad(uint64_t bytes) { offset_ += round_up(bytes); }
    uint64_t bytes() const { return offset_; }

    // `what` names the arena in errors; on success *base owns the memory.
    int commit(void** base, const char* what) const
    {
        int rc = residency_fits(offset_, what);
        if (rc) return rc;
        if ((rc = device_alloc(base, offset_, what))) return rc;
        for (const Piece& p : pieces_) p.bind(static_cast<uint8_t*>(*base) + p.offset);
        return ARC_OK;
    }

    static uint64_t round_up(uint64_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

private:
    struct Piece {
        uint64_t offset;
        std::function<void(uint8_t*)> bind;
    };
    std::vector<Piece> pieces_;
    uint64_t offset_ = 0;
};

// ------------------------------------------------------------ prompt pass
constexpr int kPfMaxM = 256;  // prompt rows per pass of the batched prompt pass

// Device buffers of the batched prompt pass (arc_prefill.hip), carved from
// the session arena.
struct PrefillBufs {
    float* h = nullptr;         // [256][hidden] residual stream
    _Float16* x = nullptr;      // [256][hidden] fp16 GEMM input (normed h, attention output)
    _Float16* xs = nullptr;     // [256][ffn] fp16 SwiGLU output (input of ffn_down)
    float* q = nullptr;         // [256][hidden] q after RoPE
    float* part = nullptr;      // split-K partials
    uint64_t part_elems = 0;
    uint32_t* tokens = nullptr;       // [256] device
    uint32_t* host_tokens = nullptr;  // pinned staging, one slot of 256 per pass
    uint32_t host_slots = 0;
};

// Floats of split-K partials the prompt pass needs for these dims.
// arc_prefill.hip.
uint64_t prefill_part_elems(const arc_model_dims& d);

// Bytes of the EXEC148 image of a rows x K Q4_K tensor (148 bytes per
// 256-weight block).
inline uint64_t exec148_image_bytes(uint32_t rows, uint32_t K) { return uint64_t(rows) * (K / kQK) * kE148Bytes; }

struct Layer {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm, *qb, *kb, *vb;
    int v_type, down_type;  // kFmtQ4, or kFmtQ6P: the model holds Q6_K tensors padded
};

}  // namespace arc

struct arc_model {
    arc_model_dims dims{};
    void* arena = nullptr;  // the model's one device allocation
    uint64_t arena_bytes = 0;
    const uint8_t* emb = nullptr;
    const uint8_t* out = nullptr;
    const float* out_norm = nullptr;
    std::vector<arc::Layer> layers;
    uint64_t weight_bytes = 0;
    // Reserve for the EXEC148 image of every Q4_K ffn_down (layer order):
    // slot i at e148_base + i * e148_stride.
    uint8_t* e148_base = nullptr;
    uint64_t e148_stride = 0;
    uint32_t e148_slots = 0;

    ~arc_model()
    {
        if (arena) (void)hipFree(arena);
    }
};

struct arc_session {
    arc_model* model = nullptr;
    uint32_t max_ctx = 0;
    uint32_t max_chunks = 0;
    hipStream_t stream = nullptr;
    void* arena = nullptr;   // the session's one device allocation
    void* pinned = nullptr;  // the session's one pinned host allocation
    uint64_t kv_bytes = 0, working_bytes = 0;
    _Float16* kcache = nullptr;  // [layers][max_ctx][kv_dim]
    _Float16* vcache = nullptr;
    float *h = nullptr, *h1 = nullptr, *q = nullptr, *attn = nullptr, *s = nullptr, *logits = nullptr;
    float *apo = nullptr, *apml = nullptr;  // attention split partials [kv_heads][kMaxSplits][hpk][...]
    uint32_t* counters = nullptr;            // kCounters arrival counters
    uint32_t* done = nullptr;                // kDoneCopies copies of the attention + o done counter
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
    arc::PrefillBufs pf;             // batched prompt-pass buffers
    uint32_t prefill_kernels = 0;    // launches of the last arc_session_prefill call
    // per layer: EXEC148 image of a Q4_K ffn_down the decode step reads
    // instead of the packed tensor (route B), or null (route A)
    std::vector<const uint8_t*> down_e148;

    ~arc_session()
    {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (stream) (void)hipStreamDestroy(stream);
        if (arena) (void)hipFree(arena);
        if (pinned) (void)hipHostFree(pinned);
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
