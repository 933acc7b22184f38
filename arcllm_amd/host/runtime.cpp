// runtime.cpp -- arcllm::v1::runtime::generate over the gfx950 C ABI.
//
// Flow (the reference's generate, src/arcllm_v1_runtime.cpp:149-535):
//   request checks -> GGUF map + tensor-table checks -> Qwen2 model binding
//   (tensor census, shapes, quant types) -> upload of the packed tensors to
//   HBM (arc_model_create) -> session with an fp16 KV cache for
//   prompt + max_new positions -> prompt pass (arc_session_prefill: the
//   argmax after the last prompt token is the first generated token) ->
//   max_new - 1 greedy decode steps (arc_session_decode, one captured-graph
//   launch per token, argmax on the GPU) -> stats.
// Every C-ABI status other than ARC_OK becomes std::runtime_error carrying
// arc_last_error(); handles are released on every path.
#include "../../include/arcllm/v1/runtime.h"
#include "../../include/arcllm_hip.h"
#include "gguf.h"

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

namespace arcllm::v1::runtime {

namespace {

// The reference's validated request domain (src/arcllm_v1_runtime.cpp:164,
// 246-252): prompts of at most 256 tokens and at most 4096 positions.
constexpr uint32_t kMaxPrompt = 256;
constexpr uint32_t kMaxContext = 4096;

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error("ArcLLM runtime: " + what); }

void check(int rc, const char* what)
{
    if (rc != ARC_OK) fail(std::string(what) + ": " + arc_last_error());
}

struct ModelDeleter {
    void operator()(arc_model* m) const { (void)arc_model_destroy(m); }
};
struct SessionDeleter {
    void operator()(arc_session* s) const { (void)arc_session_destroy(s); }
};

uint32_t meta_u32(const gguf::File& f, const std::string& key, uint32_t fallback)
{
    const gguf::Value* v = f.find_value(key);
    if (!v) return fallback;
    const uint64_t x = v->as_u64();
    if (x > 0xffffffffull) fail("metadata " + key + " out of range");
    return uint32_t(x);
}

float meta_f32(const gguf::File& f, const std::string& key, float fallback)
{
    const gguf::Value* v = f.find_value(key);
    return v ? float(v->as_f64()) : fallback;
}

const gguf::Tensor& need(const gguf::File& f, const std::string& name)
{
    const gguf::Tensor* t = f.find_tensor(name);
    if (!t) fail("missing tensor " + name);
    return *t;
}

std::string layer_name(uint32_t l, const char* suffix) { return "blk." + std::to_string(l) + "." + suffix; }

// The GGUF -> slot binding of a Qwen2-architecture model: dims from the
// metadata (with the reference's eps/theta defaults), each tensor checked
// against the slot's expected type and shape (arc_model_tensor_info).
struct Binding {
    arc_model_dims dims{};
    std::vector<const void*> ptrs;
};

Binding bind_qwen2(const gguf::File& f)
{
    Binding b;
    arc_model_dims& d = b.dims;
    const gguf::Value* arch = f.find_value("general.architecture");
    if (arch && arch->type == gguf::kString && arch->s != "qwen2") fail("unsupported architecture " + arch->s);
    d.layers = meta_u32(f, "qwen2.block_count", 0);
    if (d.layers == 0 || d.layers > ARC_MAX_LAYERS) fail("block count mismatch");
    const gguf::Tensor& emb = need(f, "token_embd.weight");
    if (emb.dims.size() != 2) fail("token_embd.weight must be 2-D");
    d.hidden = meta_u32(f, "qwen2.embedding_length", uint32_t(emb.dims[0]));
    d.vocab = uint32_t(emb.dims[1]);
    d.q_heads = meta_u32(f, "qwen2.attention.head_count", 0);
    d.kv_heads = meta_u32(f, "qwen2.attention.head_count_kv", d.q_heads);
    d.head_dim = d.q_heads ? d.hidden / d.q_heads : 0;
    d.ffn = meta_u32(f, "qwen2.feed_forward_length", 0);
    d.rms_eps = meta_f32(f, "qwen2.attention.layer_norm_rms_epsilon", 1e-6f);
    d.rope_theta = meta_f32(f, "qwen2.rope.freq_base", 1000000.0f);
    const size_t expect = 3 + size_t(d.layers) * 12;
    if (f.tensors().size() != expect)
        fail("tensor census mismatch: " + std::to_string(f.tensors().size()) + " tensors, expected " +
             std::to_string(expect));
    for (uint32_t l = 0; l < d.layers; ++l) {
        const gguf::Tensor& v = need(f, layer_name(l, "attn_v.weight"));
        const gguf::Tensor& dn = need(f, layer_name(l, "ffn_down.weight"));
        if ((v.type != gguf::kTypeQ4K && v.type != gguf::kTypeQ6K) ||
            (dn.type != gguf::kTypeQ4K && dn.type != gguf::kTypeQ6K))
            fail("mixed-quant layer obstruction: " + std::to_string(l));
        d.v_type[l] = int32_t(v.type);
        d.down_type[l] = int32_t(dn.type);
    }

    static const char* const kGlobal[ARC_T_GLOBAL_COUNT] = {"token_embd.weight", "output.weight",
                                                             "output_norm.weight"};
    static const char* const kLayer[ARC_T_LAYER_COUNT] = {
        "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q.bias",     "attn_k.bias",
        "attn_v.bias",      "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
        "ffn_down.weight"};
    auto bind_one = [&](int layer, int slot, const std::string& name) {
        int qtype = 0;
        uint32_t rows = 0, K = 0;
        uint64_t bytes = 0;
        check(arc_model_tensor_info(&d, layer, slot, &qtype, &rows, &K, &bytes), "model dims");
        const gguf::Tensor& t = need(f, name);
        const bool vec = qtype == 0;
        const uint32_t want_type = vec ? gguf::kTypeF32 : uint32_t(qtype);
        const bool shape_ok = vec ? (t.dims.size() == 1 && t.dims[0] == K)
                                  : (t.dims.size() == 2 && t.dims[0] == K && t.dims[1] == rows);
        if (t.type != want_type || !shape_ok || t.nbytes != bytes) fail("tensor " + name + " has an unexpected type or shape");
        b.ptrs.push_back(t.data);
    };
    for (int s = 0; s < ARC_T_GLOBAL_COUNT; ++s) bind_one(-1, s, kGlobal[s]);
    for (uint32_t l = 0; l < d.layers; ++l)
        for (int s = 0; s < ARC_T_LAYER_COUNT; ++s) bind_one(int(l), s, layer_name(l, kLayer[s]));
    return b;
}

}  // namespace

RunResult generate(const RunRequest& request)
{
    if (request.model_path.empty() || request.shader_dir.empty()) fail("requires model_path and shader_dir");
    if (request.input_token_ids.empty()) fail("requires at least one input token");
    if (request.max_new_tokens == 0) fail("requires max_new_tokens >= 1");

    const gguf::File file(request.model_path);
    Binding bound = bind_qwen2(file);
    const arc_model_dims& d = bound.dims;

    const uint64_t seq = request.input_token_ids.size();
    if (seq > kMaxPrompt) fail("prefill token count exceeds current model/runtime limit");
    if (seq + uint64_t(request.max_new_tokens) - 1 > kMaxContext) fail("request exceeds KV context limit");
    for (uint32_t t : request.input_token_ids)
        if (t >= d.vocab) fail("input token out of vocabulary");

    int ndev = 0;
    check(arc_device_count(&ndev), "device query");
    if (ndev < 1) fail("no HIP device");

    arc_model* mraw = nullptr;
    check(arc_model_create(&d, bound.ptrs.data(), &mraw), "model upload");
    std::unique_ptr<arc_model, ModelDeleter> model(mraw);
    arc_session* sraw = nullptr;
    check(arc_session_create(model.get(), uint32_t(seq) + request.max_new_tokens, &sraw), "session");
    std::unique_ptr<arc_session, SessionDeleter> session(sraw);

    RunResult result;
    result.generated_token_ids.reserve(request.max_new_tokens);
    uint32_t next = 0, nonfinite = 0;
    check(arc_session_prefill(session.get(), request.input_token_ids.data(), uint32_t(seq), 0, 0, &next, &nonfinite),
          "prefill");
    if (nonfinite) fail("non-finite prefill logits");
    result.generated_token_ids.push_back(next);
    // the prompt pass: kernel launches as issued; submits = passes of up to
    // 256 prompt rows (one decode-step graph launch per token for a 1-token prompt)
    result.stats.prefill_dispatches = arc_session_prefill_kernels(session.get());
    result.stats.prefill_submits = seq > 1 ? uint32_t((seq + 255) / 256) : 1u;
    result.stats.finite = true;

    const uint32_t steps = request.max_new_tokens - 1;
    if (steps) {
        std::vector<uint32_t> out(steps);
        check(arc_session_decode(session.get(), next, uint32_t(seq), steps, 0, out.data(), &nonfinite), "decode");
        if (nonfinite) fail("non-finite decode logits");
        result.generated_token_ids.insert(result.generated_token_ids.end(), out.begin(), out.end());
        result.stats.decode_dispatches_per_step = arc_session_kernels_per_step(session.get());
        result.stats.decode_submits_per_step = 1;
        result.stats.decode_steps = steps;
        result.stats.route_a_steps = steps;
    }
    if (result.generated_token_ids.size() != request.max_new_tokens) fail("generated-token count mismatch");
    return result;
}

}  // namespace arcllm::v1::runtime
