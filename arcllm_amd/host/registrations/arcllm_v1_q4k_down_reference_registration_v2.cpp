// Data of the reference's Q4_K FFN-down registration bundle (see the header).
#include "arcllm_v1_q4k_down_reference_registration_v2.h"

namespace arcllm::v1::reference_registration_v2 {

namespace {

using namespace registry_v2;

// where the reference keeps the evidence behind these entries
constexpr ProvenanceRef kArch{"artifacts/ARCLLM_V1/ARCLLM_V1_Q4_DOWN_PRIMITIVE_ARCHITECTURE_LOCK_v0.1.json",
                              "5c696b924038de13de8d5176b724fcd814cdcc8e"};
constexpr ProvenanceRef kPerf{"artifacts/ARCLLM_V1/ARCLLM_V1_B1_2_P1_P3_PERFORMANCE_CANONICAL_v0.1.json",
                              "339053906653e522cf711f43cc0a5fccad6e8f14"};
constexpr ProvenanceRef kPol{"artifacts/ARCLLM_V1/ARCLLM_V1_B1_SELECTION_LIFETIME_POLICY_INTEGRATION_v0.1.json",
                             "c90fb7386bbaae6fbca03aeefe6a9acd119e371d"};
constexpr auto V = ValidationState::VALIDATED;
constexpr auto AMORT = AcquisitionTrigger::REUSE_AMORTIZED;

constexpr DomainDescriptor kDomains[] = {{kDomain, V, "Q4K_DECODE_FFN_DOWN_FROZEN_DOMAIN", kArch}};
constexpr ReuseMetricDescriptor kMetrics[] = {{kReuseMetric, V, "FUTURE_REUSE_TOKENS_FROZEN_METRIC", kPol}};
constexpr EvidenceSetDescriptor kEvidence[] = {
    {kEvidenceSet, V, "B1_2_FROZEN_ACQUISITION_AND_STEADY_STATE_EVIDENCE", kPerf}};
constexpr EvidenceProfileDescriptor kProfiles[] = {
    {kProfile0, kDomain, kReuseMetric, kEvidenceSet, V, "PROFILE_0", kPerf},
    {kProfile1, kDomain, kReuseMetric, kEvidenceSet, V, "PROFILE_1", kPerf}};
constexpr PrimitiveFamilyDescriptor kFamilies[] = {{kFamily, kDomain, V, "Q4K_DOWN_REFERENCE_FAMILY", kArch}};
constexpr CapabilityDescriptor kCapabilities[] = {
    {kCapability, kDomain, kPrimitiveB, kPrimitiveA, V, "Q4K_DECODE_FFN_DOWN", kArch}};
constexpr PrimitiveDescriptor kPrimitives[] = {
    {kPrimitiveA, kFamily, kCapability, {}, 0, PRIMITIVE_FALLBACK | PRIMITIVE_NO_EXTRA_REPRESENTATION, V,
     "A_SPLIT_K32", kArch},
    {kPrimitiveB, kFamily, kCapability, kRepresentationB, 549527552ull,
     PRIMITIVE_REQUIRES_RESIDENCY | PRIMITIVE_REQUIRES_IDENTITY_VALIDATION, V, "B_EXEC148", kPerf}};
constexpr AcquisitionPathDescriptor kPaths[] = {
    {kAcquirePrimary, kPrimitiveB, 0u, AMORT, V, "P1_GPU_IN_PLACE", kPerf},
    {kAcquireSecondary, kPrimitiveB, 1u, AMORT, V, "P3_COLD_UNBUFFERED", kPerf},
    {kAcquireTertiary, kPrimitiveB, 2u, AMORT, V, "P0_CPU_DIRECT", kPerf},
    {kAcquireDisabledWarm, kPrimitiveB, 3u, AMORT, ValidationState::DISABLED_BY_EVIDENCE, "P3_WARM_PAGE_CACHE", kPerf}};
// future reuse (tokens) from which each path pays off, per evidence profile
constexpr AcquisitionThresholdDescriptor kThresholds[] = {
    {kCapability, kProfile0, kAcquirePrimary, kReuseMetric, 2ull, V, kPol},
    {kCapability, kProfile1, kAcquirePrimary, kReuseMetric, 4ull, V, kPol},
    {kCapability, kProfile0, kAcquireSecondary, kReuseMetric, 15ull, V, kPol},
    {kCapability, kProfile1, kAcquireSecondary, kReuseMetric, 33ull, V, kPol},
    {kCapability, kProfile0, kAcquireTertiary, kReuseMetric, 17ull, V, kPol},
    {kCapability, kProfile1, kAcquireTertiary, kReuseMetric, 37ull, V, kPol}};
constexpr LifecycleDescriptor kLifecycles[] = {{kPrimitiveB, true, true, true, true, true, true, kPol}};

constexpr RegistrationBundle kBundle{"Q4K_DOWN_REFERENCE_REGISTRATION_V2",
                                     kDomains, 1, kMetrics, 1, kEvidence, 1, kProfiles, 2, kFamilies, 1,
                                     kCapabilities, 1, kPrimitives, 2, kPaths, 4, kThresholds, 6, kLifecycles, 1};

}  // namespace

const registry_v2::RegistrationBundle& q4k_down_reference_bundle() noexcept { return kBundle; }

}  // namespace arcllm::v1::reference_registration_v2
