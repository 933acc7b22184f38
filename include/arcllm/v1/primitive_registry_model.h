/* arcllm/v1/primitive_registry_model.h -- descriptor vocabulary of the
 * operator plugin registry (the types primitive_registry_v2.h builds on).
 *
 * Same names, members, member order and enumerator values as the reference's
 * include/arcllm/v1/primitive_registry_model.h:1-152, so registration bundles
 * written against the reference (positional aggregate initialisers) compile
 * unchanged.  Only the descriptors the v2 registry uses are declared; the
 * reference's v1-only bundle types are not part of this runtime.
 */
#pragma once

#include <cstddef>
#include <cstdint>

namespace arcllm::v1::registry {

/* A 64-bit identifier typed by Tag; 0 means "none". */
template <typename Tag>
struct OpaqueId {
    std::uint64_t value = 0;
    constexpr explicit operator bool() const noexcept { return value != 0; }
    friend constexpr bool operator==(OpaqueId a, OpaqueId b) noexcept { return a.value == b.value; }
    friend constexpr bool operator!=(OpaqueId a, OpaqueId b) noexcept { return a.value != b.value; }
};

struct DomainTag {};
struct CapabilityTag {};
struct PrimitiveFamilyTag {};
struct PrimitiveTag {};
struct RepresentationTag {};
struct EvidenceProfileTag {};
struct ReuseMetricTag {};
struct AcquisitionPathTag {};
struct EvidenceSetTag {};

using DomainId = OpaqueId<DomainTag>;
using CapabilityId = OpaqueId<CapabilityTag>;
using PrimitiveFamilyId = OpaqueId<PrimitiveFamilyTag>;
using PrimitiveId = OpaqueId<PrimitiveTag>;
using RepresentationId = OpaqueId<RepresentationTag>;
using EvidenceProfileId = OpaqueId<EvidenceProfileTag>;
using ReuseMetricId = OpaqueId<ReuseMetricTag>;
using AcquisitionPathId = OpaqueId<AcquisitionPathTag>;
using EvidenceSetId = OpaqueId<EvidenceSetTag>;

/* Only VALIDATED entries take part in routing decisions. */
enum class ValidationState : std::uint8_t {
    VALIDATED = 0,
    DISABLED_BY_EVIDENCE = 1,
    CAPABILITY_GATED = 2,
    HISTORICAL_REFERENCE = 3
};

enum PrimitiveFlags : std::uint32_t {
    PRIMITIVE_NONE = 0u,
    PRIMITIVE_FALLBACK = 1u << 0,
    PRIMITIVE_NO_EXTRA_REPRESENTATION = 1u << 1,      /* executes on the packed tensors as loaded */
    PRIMITIVE_REQUIRES_RESIDENCY = 1u << 2,           /* needs an acquired representation */
    PRIMITIVE_REQUIRES_IDENTITY_VALIDATION = 1u << 3  /* the representation is validated after acquisition */
};

/* Where the evidence behind a descriptor lives (informational). */
struct ProvenanceRef {
    const char* artifact_path = nullptr;
    const char* git_blob = nullptr;
};

struct DomainDescriptor {
    DomainId id{};
    ValidationState state = ValidationState::VALIDATED;
    const char* opaque_name = nullptr;
    ProvenanceRef provenance{};
};

struct ReuseMetricDescriptor {
    ReuseMetricId id{};
    ValidationState state = ValidationState::VALIDATED;
    const char* opaque_name = nullptr;
    ProvenanceRef provenance{};
};

struct EvidenceSetDescriptor {
    EvidenceSetId id{};
    ValidationState state = ValidationState::VALIDATED;
    const char* opaque_name = nullptr;
    ProvenanceRef provenance{};
};

struct PrimitiveFamilyDescriptor {
    PrimitiveFamilyId id{};
    DomainId domain{};
    ValidationState state = ValidationState::VALIDATED;
    const char* opaque_name = nullptr;
    ProvenanceRef provenance{};
};

/* An executable implementation of a capability; residency_bytes is the size
 * of its extra representation (0 for PRIMITIVE_NO_EXTRA_REPRESENTATION). */
struct PrimitiveDescriptor {
    PrimitiveId id{};
    PrimitiveFamilyId family{};
    CapabilityId capability{};
    RepresentationId representation{};
    std::uint64_t residency_bytes = 0;
    std::uint32_t flags = PRIMITIVE_NONE;
    ValidationState state = ValidationState::VALIDATED;
    const char* opaque_name = nullptr;
    ProvenanceRef provenance{};
};

/* Acquiring through `acquisition` for (capability, profile) pays off once the
 * future reuse reaches minimum_reuse_units (in the profile's reuse metric). */
struct AcquisitionThresholdDescriptor {
    CapabilityId capability{};
    EvidenceProfileId profile{};
    AcquisitionPathId acquisition{};
    ReuseMetricId reuse_metric{};
    std::uint64_t minimum_reuse_units = 0;
    ValidationState state = ValidationState::VALIDATED;
    ProvenanceRef provenance{};
};

/* When a resident representation of `primitive` is evicted or kept. */
struct LifecycleDescriptor {
    PrimitiveId primitive{};
    bool preserve_residency_outside_domain = false;
    bool evict_on_lease_revoke = false;
    bool evict_on_identity_invalid = false;
    bool evict_on_execution_unavailable = false;
    bool evict_on_model_unload = false;
    bool evict_on_zero_future_reuse = false;
    ProvenanceRef provenance{};
};

}  // namespace arcllm::v1::registry
