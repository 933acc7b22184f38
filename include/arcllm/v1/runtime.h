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
 *    sidecar_path, evidence_profile and request_within_validated_domain are
 *    accepted and not used by generation, as in the reference.
 *
 * RuntimeStats: "dispatches" are kernel launches; decode "submits" are
 * captured-graph launches (one per step) and prefill "submits" are batched
 * prompt passes of up to 256 rows; route_a_steps counts decode steps run on the
 * direct packed kernels (route B, the EXEC148 repack, is not used), so
 * acquire/evict and the b_* / p* counters stay 0.
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
