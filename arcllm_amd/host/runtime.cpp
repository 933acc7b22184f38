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
#include "qwen2_binding.h"
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

}  // namespace

RunResult generate(const RunRequest& request)
{
    if (request.model_path.empty() || request.shader_dir.empty()) fail("requires model_path and shader_dir");
    if (request.input_token_ids.empty()) fail("requires at least one input token");
    if (request.max_new_tokens == 0) fail("requires max_new_tokens >= 1");

    const gguf::File file(request.model_path);
    const Qwen2Binding bound = bind_qwen2(file);
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
