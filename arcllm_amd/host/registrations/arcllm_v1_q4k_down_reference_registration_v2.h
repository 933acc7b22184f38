// The reference's Q4_K FFN-down registration (capability, primitives A/B,
// acquisition paths P1/P3/P0 and the disabled warm path, Arc-measured reuse
// thresholds), restated as data under the reference's header name, namespace
// and ids (src/registrations/arcllm_v1_q4k_down_reference_registration_v2.h,
// .cpp:1-55 of the reference), so code written against it compiles here.
// The gfx950 runtime routes with its own MI355X-measured registration
// (arcllm_amd/host/q4_down_backend.h); this one is what the reference's
// policy decisions are reproduced on.
#pragma once

#include "../../../include/arcllm/v1/primitive_registry_v2.h"

namespace arcllm::v1::reference_registration_v2 {

inline constexpr registry_v2::DomainId kDomain{0xD0010001ull};
inline constexpr registry_v2::ReuseMetricId kReuseMetric{0xD0020001ull};
inline constexpr registry_v2::EvidenceSetId kEvidenceSet{0xE0010001ull};
inline constexpr registry_v2::EvidenceProfileId kProfile0{0x00005101ull};
inline constexpr registry_v2::EvidenceProfileId kProfile1{0x00005102ull};
inline constexpr registry_v2::PrimitiveFamilyId kFamily{0xF0010001ull};
inline constexpr registry_v2::CapabilityId kCapability{0x00010001ull};
inline constexpr registry_v2::PrimitiveId kPrimitiveA{0x0000A001ull};
inline constexpr registry_v2::PrimitiveId kPrimitiveB{0x0000B001ull};
inline constexpr registry_v2::RepresentationId kRepresentationB{0xE1480001ull};
inline constexpr registry_v2::AcquisitionPathId kAcquirePrimary{0x0000C101ull};
inline constexpr registry_v2::AcquisitionPathId kAcquireSecondary{0x0000C102ull};
inline constexpr registry_v2::AcquisitionPathId kAcquireTertiary{0x0000C103ull};
inline constexpr registry_v2::AcquisitionPathId kAcquireDisabledWarm{0x0000C104ull};

const registry_v2::RegistrationBundle& q4k_down_reference_bundle() noexcept;

}  // namespace arcllm::v1::reference_registration_v2
