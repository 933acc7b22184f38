/* arcllm/v1/runtime.h -- the drop-in public API of the gfx950 decode runtime.
 *
 * Same names, members and member order as the reference's public header
 * (include/arcllm/v1/runtime.h:8-57 of the reference), so callers of
 * arcllm::v1::runtime::generate compile unchanged against this one.
 *
 * Behaviour (src/arcllm_v1_runtime.cpp:149-535 of the reference):
 *  - greedy generation of max_new_tokens tokens after input_token_ids from a
 *    Qwen2-architecture GGUF (Q4_K / Q6_K / F32 tensors) at model_path;
 *  - errors (bad request, model contract mismatch, non-finite logits, device
 *    failure) throw std::runtime_error; nothing else escapes;
 *  - shader_dir must be non-empty as in the reference; the kernels are built
 *    into the library (libarcllm_hip.so), so its value is not read;
 *  - the Q4_K ffn_down layers are routed per decode step by the Q4-down
 *    policy (generic_policy_engine_v4.h) over the gfx950 registration, as in
 *    the reference (src/arcllm_v1_runtime.cpp:305-337, 459-530):
 *    evidence_profile picks the profile, request_within_validated_domain is
 *    the capability's evidence scope (outside it, route A only),
 *    sidecar_path names an EXEC148 family image for the P3 acquisition path;
 *    an image acquired for a request is evicted when it ends.
 *
 * RuntimeStats: "dispatches" are kernel launches; decode "submits" are
 * captured-graph launches (one per step) and prefill "submits" are batched
 * prompt passes of up to 256 rows; route_a_steps / route_b_steps count decode
 * steps on the packed Q4_K kernels / the EXEC148 image (a model without
 * Q4_K ffn_down counts every step as route A), acquire_events /
 * evict_events the policy's lifecycle actions, b_* and p* the backend's
 * allocations, materializations, validations, releases and acquisition
 * path calls.
 */
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace arcllm::v1::runtime {

enum class EvidenceProfile : std::uint8_t {
    PROFILE_0 = 0,
    PROFILE_1 = 1
};

struct RunRequest {
    std::string model_path;
    std::string shader_dir;
    std::string sidecar_path;
    std::vector<std::uint32_t> input_token_ids;
    std::uint32_t max_new_tokens = 1;
    EvidenceProfile evidence_profile = EvidenceProfile::PROFILE_0;
    bool request_within_validated_domain = false;
};

struct RuntimeStats {
    std::uint32_t prefill_dispatches = 0;
    std::uint32_t prefill_submits = 0;
    std::uint32_t decode_dispatches_per_step = 0;
    std::uint32_t decode_submits_per_step = 0;
    std::uint32_t decode_steps = 0;

    std::uint32_t route_a_steps = 0;
    std::uint32_t route_b_steps = 0;
    std::uint32_t acquire_events = 0;
    std::uint32_t evict_events = 0;

    std::uint64_t b_allocations = 0;
    std::uint64_t b_materializations = 0;
    std::uint64_t b_validations = 0;
    std::uint64_t b_releases = 0;
    std::uint64_t p1_calls = 0;
    std::uint64_t p3_calls = 0;
    std::uint64_t p0_calls = 0;

    bool finite = false;
};

struct RunResult {
    std::vector<std::uint32_t> generated_token_ids;
    RuntimeStats stats{};
};

RunResult generate(const RunRequest& request);

}  // namespace arcllm::v1::runtime
