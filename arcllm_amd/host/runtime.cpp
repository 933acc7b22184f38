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
// Models with Q4_K ffn_down layers route them per decode step through the
// operator plugin surface, as the reference does
// (src/arcllm_v1_runtime.cpp:305-337, 459-530): before step i the policy
// (policy_v4::evaluate over the gfx950 registration) sees a future reuse of
// max_new - 1 - i tokens and the backend's residency, apply_decision carries
// its decision out against HipQ4DownBackend (acquire + validate an EXEC148
// image, evict, or resolve), and the step runs on the primitive it resolved;
// after the last step a close decision with no future reuse evicts the image.
// Consecutive steps on one route run as one arc_session_decode call.
// Every C-ABI status other than ARC_OK becomes std::runtime_error carrying
// arc_last_error(); handles are released on every path.
#include "../../include/arcllm/v1/runtime.h"
#include "../../include/arcllm_hip.h"
#include "gguf.h"
#include "q4_down_backend.h"
#include "registrations/arcllm_v1_q4k_down_reference_registration_v2.h"

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
    std::vector<uint32_t> q4_layers;
    std::vector<const uint8_t*> q4_host;
    for (uint32_t l = 0; l < d.layers; ++l)
        if (d.down_type[l] == ARC_Q4_K) {
            q4_layers.push_back(l);
            q4_host.push_back(static_cast<const uint8_t*>(
                bound.ptrs[ARC_T_GLOBAL_COUNT + size_t(l) * ARC_T_LAYER_COUNT + ARC_T_FFN_DOWN]));
        }
    if (q4_layers.empty()) {
        // no Q4_K ffn_down: every step runs the packed kernels
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
    } else {
        namespace q4reg = reference_registration_v2;
        namespace gp = policy_v4;
        namespace bind = binding_v4;
        hip_q4_down::HipQ4DownBackend backend(model.get(), q4_layers, q4_host, d.hidden, d.ffn, request.sidecar_path);
        const hip_q4_down::Mi355xRegistration registration(backend.family_bytes());
        registry_v2::PrimitiveRegistry registry;
        registry_v2::RegistryError reg_error{};
        if (registry.add_bundle(registration.bundle(), &reg_error) != registry_v2::RegistryStatus::OK)
            fail("Q4 registry bind failed");
        bind::BindingState binding{};

        auto decide = [&](uint64_t future_reuse) {
            const gp::PrimitiveRuntimeState ps[] = {
                {q4reg::kPrimitiveA, false, true, true, true, true},
                {q4reg::kPrimitiveB, backend.resident(), backend.validated(), true,
                 backend.resident() && backend.validated(), true}};
            const gp::AcquisitionRuntimeState as[] = {{q4reg::kAcquirePrimary, true, false},
                                                      {q4reg::kAcquireSecondary, backend.p3_available(), false},
                                                      {q4reg::kAcquireTertiary, true, false},
                                                      {q4reg::kAcquireDisabledWarm, false, false}};
            gp::PolicyRequest req{};
            req.capability = q4reg::kCapability;
            req.profile = request.evidence_profile == EvidenceProfile::PROFILE_0 ? q4reg::kProfile0 : q4reg::kProfile1;
            req.request_within_capability_evidence_scope = request.request_within_validated_domain;
            req.model_loaded = true;
            req.future_reuse_known = true;
            req.future_reuse_units = future_reuse;
            req.acquisition_allowed = true;
            req.primitive_states = ps;
            req.primitive_state_count = 2;
            req.acquisition_states = as;
            req.acquisition_state_count = 4;
            return gp::evaluate(registry, req);
        };
        auto apply = [&](const gp::PolicyDecision& decision, const char* what) {
            const bind::ApplyResult r = bind::apply_decision(registry, q4reg::kCapability, decision, backend, binding);
            if (!r.ready || r.backend_status != bind::BackendStatus::OK)
                fail(std::string(what) + " binding not ready" +
                     (backend.last_error().empty() ? "" : ": " + backend.last_error()));
            return r;
        };

        // steps decided but not yet run, all on route `route`
        uint32_t done = 0, pending = 0, tok = next;
        uint64_t route = 0;
        auto flush = [&]() {
            if (!pending) return;
            std::vector<uint32_t> out(pending);
            check(arc_session_decode(session.get(), tok, uint32_t(seq) + done, pending, 0, out.data(), &nonfinite),
                  "decode");
            if (nonfinite) fail("non-finite decode logits");
            const uint32_t k = arc_session_kernels_per_step(session.get());
            if (result.stats.decode_steps == 0) {
                result.stats.decode_dispatches_per_step = k;
                result.stats.decode_submits_per_step = 1;
            } else if (result.stats.decode_dispatches_per_step != k) {
                fail("decode topology changed within request");
            }
            result.generated_token_ids.insert(result.generated_token_ids.end(), out.begin(), out.end());
            result.stats.decode_steps += pending;
            done += pending;
            tok = out.back();
            pending = 0;
        };
        for (uint32_t di = 0; di < steps; ++di) {
            const gp::PolicyDecision decision = decide(uint64_t(steps - di));
            if (decision.status != gp::PolicyStatus::OK) fail("Q4 policy decision not OK");
            if (decision.lifecycle != gp::LifecycleAction::NONE) flush();
            if (decision.lifecycle == gp::LifecycleAction::ACQUIRE) ++result.stats.acquire_events;
            if (decision.lifecycle == gp::LifecycleAction::EVICT) ++result.stats.evict_events;
            const bind::ApplyResult applied = apply(decision, "Q4");
            if (applied.primitive.opaque == q4reg::kPrimitiveA.value) ++result.stats.route_a_steps;
            else if (applied.primitive.opaque == q4reg::kPrimitiveB.value) ++result.stats.route_b_steps;
            else fail("unknown Q4 primitive");
            if (applied.primitive.opaque != route) {
                flush();
                if (!backend.route(session.get(), applied.primitive)) fail("Q4 route: " + backend.last_error());
                route = applied.primitive.opaque;
            }
            ++pending;
        }
        flush();

        const gp::PolicyDecision close = decide(0);
        if (close.status != gp::PolicyStatus::OK) fail("close policy not OK");
        if (close.lifecycle == gp::LifecycleAction::EVICT) ++result.stats.evict_events;
        apply(close, "close");
        if (backend.resident()) fail("EXEC148 image still resident after request close");

        const hip_q4_down::BackendCounters& c = backend.counters();
        result.stats.b_allocations = c.b_allocations;
        result.stats.b_materializations = c.b_materializations;
        result.stats.b_validations = c.b_validations;
        result.stats.b_releases = c.b_releases;
        result.stats.p1_calls = c.p1_calls;
        result.stats.p3_calls = c.p3_calls;
        result.stats.p0_calls = c.p0_calls;
    }
    if (result.generated_token_ids.size() != request.max_new_tokens) fail("generated-token count mismatch");
    return result;
}

}  // namespace arcllm::v1::runtime
