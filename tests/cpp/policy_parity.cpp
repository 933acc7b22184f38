// policy_parity.cpp -- decision trace of the operator plugin surface
// (registry v2, policy v4, binding v4), for parity between two builds of
// this one program: against this repository's implementation
// (include/arcllm/v1 + arcllm_amd/host) and against the reference's own
// sources (include/arcllm/v1 + src/arcllm_v1_primitive_registry_v2.cpp,
// src/arcllm_v1_generic_policy_engine_v4.cpp,
// src/arcllm_v1_generic_backend_binding_v4.cpp and
// src/registrations/arcllm_v1_q4k_down_reference_registration_v2.cpp).
// Identical traces mean identical behaviour on every case below.
//
// Sections:
//   registry  add_bundle on the Q4-down bundle and ~70 mutations of it
//             (null arrays, zero/duplicate ids, every dangling reference,
//             residency flags, threshold/mandatory semantics, cross-bundle
//             duplicates, capacity), with status, category, id, bundle count;
//   q4        evaluate over the Q4-down bundle: 2 profiles x 2^15 runtime
//             masks x 16 reuse values (the reference's family-1 sweep of
//             tests/arcllm_v1_phase2_closed_surface_v4_zero_science.cpp:70-110
//             plus the A-ready and warm-path bits);
//   holdout   evaluate over test-defined bundles: mandatory acquisition with
//             and without a fallback, a direct (non-represented) preferred,
//             an amortized path without a reuse metric or threshold, a
//             represented preferred without lifecycle, disabled descriptors,
//             malformed runtime arrays, profile/capability domain mismatch;
//   binding   apply_decision for every lifecycle x route x acquisition x
//             validation flag x held/full binding state x backend failure
//             combination, with the backend's call log and the final state.
//
// Output: one FNV-1a-64 hash and case count per section and overall on
// stdout; with a path argument, the full trace is written there as well.
#include <arcllm/v1/generic_backend_binding_v4.h>
#include <arcllm/v1/generic_policy_engine_v4.h>
#include <arcllm/v1/primitive_registry_v2.h>

#include "arcllm_v1_q4k_down_reference_registration_v2.h"

#include <cinttypes>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

using namespace arcllm::v1;
namespace reg = registry_v2;
namespace gp = policy_v4;
namespace bind = binding_v4;
namespace q4 = reference_registration_v2;

namespace {

struct Trace {
    std::FILE* out = nullptr;
    std::uint64_t h = 1469598103934665603ull, total = 1469598103934665603ull;
    std::uint64_t n = 0, all = 0;
    void line(const char* fmt, ...) __attribute__((format(printf, 2, 3)))
    {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        const int k = std::vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        for (int i = 0; i < k; ++i) {
            h = (h ^ std::uint8_t(buf[i])) * 1099511628211ull;
            total = (total ^ std::uint8_t(buf[i])) * 1099511628211ull;
        }
        h = (h ^ '\n') * 1099511628211ull;
        total = (total ^ '\n') * 1099511628211ull;
        ++n;
        ++all;
        if (out) std::fprintf(out, "%s\n", buf);
    }
    void section(const char* name)
    {
        std::printf("%s cases=%" PRIu64 " fnv=%016" PRIx64 "\n", name, n, h);
        h = 1469598103934665603ull;
        n = 0;
    }
};

Trace T;

unsigned u(bool b) { return b ? 1u : 0u; }

void dump_decision(const char* tag, const gp::PolicyDecision& d)
{
    T.line("%s st=%u route=%" PRIx64 " lc=%u acq=%" PRIx64 " why=%u thr=%" PRIu64 " bytes=%" PRIu64 " keep=%u val=%u",
           tag, unsigned(d.status), d.route.value, unsigned(d.lifecycle), d.acquisition.value, unsigned(d.reason),
           d.threshold_units, d.requested_residency_bytes, u(d.preserve_existing_representation),
           u(d.require_post_acquisition_identity_validation));
}

// ------------------------------------------------------------ bundle copies

// A bundle with its arrays in vectors, so tests can mutate them.
struct Editable {
    std::string name;
    bool null_name = false;
    std::vector<reg::DomainDescriptor> domains;
    std::vector<reg::ReuseMetricDescriptor> metrics;
    std::vector<reg::EvidenceSetDescriptor> evidence;
    std::vector<reg::EvidenceProfileDescriptor> profiles;
    std::vector<reg::PrimitiveFamilyDescriptor> families;
    std::vector<reg::CapabilityDescriptor> capabilities;
    std::vector<reg::PrimitiveDescriptor> primitives;
    std::vector<reg::AcquisitionPathDescriptor> paths;
    std::vector<reg::AcquisitionThresholdDescriptor> thresholds;
    std::vector<reg::LifecycleDescriptor> lifecycles;
    int null_array = -1;  // 0..9: that array's pointer is null with its count kept
    int count_bump = -1;  // 0..9: that array's count is one more than its size (pointer null)
    reg::RegistrationBundle bundle{};

    explicit Editable(const reg::RegistrationBundle& b)
        : name(b.bundle_name ? b.bundle_name : ""),
          domains(b.domains, b.domains + b.domain_count),
          metrics(b.reuse_metrics, b.reuse_metrics + b.reuse_metric_count),
          evidence(b.evidence_sets, b.evidence_sets + b.evidence_set_count),
          profiles(b.profiles, b.profiles + b.profile_count),
          families(b.families, b.families + b.family_count),
          capabilities(b.capabilities, b.capabilities + b.capability_count),
          primitives(b.primitives, b.primitives + b.primitive_count),
          paths(b.acquisitions, b.acquisitions + b.acquisition_count),
          thresholds(b.thresholds, b.thresholds + b.threshold_count),
          lifecycles(b.lifecycles, b.lifecycles + b.lifecycle_count)
    {
    }
    Editable() = default;

    template <class V>
    static const typename V::value_type* ptr(const V& v, int which, int null_array)
    {
        return which == null_array ? nullptr : (v.empty() ? nullptr : v.data());
    }

    const reg::RegistrationBundle& build()
    {
        bundle = reg::RegistrationBundle{};
        bundle.bundle_name = null_name ? nullptr : name.c_str();
        bundle.domains = ptr(domains, 0, null_array);
        bundle.domain_count = domains.size();
        bundle.reuse_metrics = ptr(metrics, 1, null_array);
        bundle.reuse_metric_count = metrics.size();
        bundle.evidence_sets = ptr(evidence, 2, null_array);
        bundle.evidence_set_count = evidence.size();
        bundle.profiles = ptr(profiles, 3, null_array);
        bundle.profile_count = profiles.size();
        bundle.families = ptr(families, 4, null_array);
        bundle.family_count = families.size();
        bundle.capabilities = ptr(capabilities, 5, null_array);
        bundle.capability_count = capabilities.size();
        bundle.primitives = ptr(primitives, 6, null_array);
        bundle.primitive_count = primitives.size();
        bundle.acquisitions = ptr(paths, 7, null_array);
        bundle.acquisition_count = paths.size();
        bundle.thresholds = ptr(thresholds, 8, null_array);
        bundle.threshold_count = thresholds.size();
        bundle.lifecycles = ptr(lifecycles, 9, null_array);
        bundle.lifecycle_count = lifecycles.size();
        std::size_t* counts[] = {&bundle.domain_count,     &bundle.reuse_metric_count, &bundle.evidence_set_count,
                                 &bundle.profile_count,    &bundle.family_count,       &bundle.capability_count,
                                 &bundle.primitive_count,  &bundle.acquisition_count,  &bundle.threshold_count,
                                 &bundle.lifecycle_count};
        if (count_bump >= 0 && *counts[count_bump] == 0) *counts[count_bump] = 1;
        return bundle;
    }
};

void dump_add(const char* tag, reg::PrimitiveRegistry& r, const reg::RegistrationBundle& b)
{
    reg::RegistryError e{};
    e.category = "unset";
    e.id = 0xdeadull;
    const reg::RegistryStatus s = r.add_bundle(b, &e);
    T.line("%s st=%u estat=%u cat=%s id=%" PRIx64 " bundles=%zu", tag, unsigned(s), unsigned(e.status),
           e.category ? e.category : "(null)", e.id, r.bundle_count());
    // the null error pointer is accepted too
    reg::PrimitiveRegistry fresh;
    const reg::RegistryStatus s2 = fresh.add_bundle(b, nullptr);
    T.line("%s nullerr st=%u bundles=%zu", tag, unsigned(s2), fresh.bundle_count());
}

// ------------------------------------------------------------ registry

const reg::DomainId kD2{0xD0990001ull};
const reg::EvidenceSetId kE2{0xE0990001ull};
const reg::EvidenceProfileId kP2{0x59900001ull};
const reg::PrimitiveFamilyId kF2{0xF0990001ull};
const reg::CapabilityId kC2{0x19900001ull};
const reg::PrimitiveId kX2{0xA9900001ull};
const reg::ReuseMetricId kM2{0xD0990002ull};

void registry_section()
{
    const reg::RegistrationBundle& base = q4::q4k_down_reference_bundle();
    using Mut = void (*)(Editable&);
    struct Case {
        const char* name;
        Mut m;
    };
    static const Case cases[] = {
        {"as_is", [](Editable&) {}},
        {"null_name", [](Editable& e) { e.null_name = true; }},
        {"null_domains", [](Editable& e) { e.null_array = 0; }},
        {"null_metrics", [](Editable& e) { e.null_array = 1; }},
        {"null_evidence", [](Editable& e) { e.null_array = 2; }},
        {"null_profiles", [](Editable& e) { e.null_array = 3; }},
        {"null_families", [](Editable& e) { e.null_array = 4; }},
        {"null_caps", [](Editable& e) { e.null_array = 5; }},
        {"null_prims", [](Editable& e) { e.null_array = 6; }},
        {"null_paths", [](Editable& e) { e.null_array = 7; }},
        {"null_thresholds", [](Editable& e) { e.null_array = 8; }},
        {"null_lifecycles", [](Editable& e) { e.null_array = 9; }},
        {"zero_domain", [](Editable& e) { e.domains[0].id = {}; }},
        {"zero_metric", [](Editable& e) { e.metrics[0].id = {}; }},
        {"zero_evidence", [](Editable& e) { e.evidence[0].id = {}; }},
        {"zero_profile", [](Editable& e) { e.profiles[1].id = {}; }},
        {"zero_family", [](Editable& e) { e.families[0].id = {}; }},
        {"zero_cap", [](Editable& e) { e.capabilities[0].id = {}; }},
        {"zero_prim", [](Editable& e) { e.primitives[1].id = {}; }},
        {"zero_path", [](Editable& e) { e.paths[3].id = {}; }},
        {"dup_domain", [](Editable& e) { e.domains.push_back(e.domains[0]); }},
        {"dup_metric", [](Editable& e) { e.metrics.push_back(e.metrics[0]); }},
        {"dup_evidence", [](Editable& e) { e.evidence.push_back(e.evidence[0]); }},
        {"dup_profile", [](Editable& e) { e.profiles[1].id = e.profiles[0].id; }},
        {"dup_family", [](Editable& e) { e.families.push_back(e.families[0]); }},
        {"dup_cap", [](Editable& e) { e.capabilities.push_back(e.capabilities[0]); }},
        {"dup_prim", [](Editable& e) { e.primitives[1].id = e.primitives[0].id; }},
        {"dup_path", [](Editable& e) { e.paths[2].id = e.paths[1].id; }},
        {"dup_threshold", [](Editable& e) { e.thresholds.push_back(e.thresholds[3]); }},
        {"dup_lifecycle", [](Editable& e) { e.lifecycles.push_back(e.lifecycles[0]); }},
        {"zero_and_dup", [](Editable& e) {  // zero id checked before a later duplicate
             e.domains.push_back(e.domains[0]);
             e.metrics[0].id = {};
         }},
        {"profile_domain", [](Editable& e) { e.profiles[0].domain = kD2; }},
        {"profile_evidence", [](Editable& e) { e.profiles[1].evidence_set = kE2; }},
        {"profile_metric", [](Editable& e) { e.profiles[0].reuse_metric = kM2; }},
        {"family_domain", [](Editable& e) { e.families[0].domain = kD2; }},
        {"prim_family", [](Editable& e) { e.primitives[0].family = kF2; }},
        {"prim_cap", [](Editable& e) { e.primitives[1].capability = kC2; }},
        {"prim_domain_mismatch", [](Editable& e) {
             e.domains.push_back({kD2, reg::ValidationState::VALIDATED, "D2", {}});
             e.families[0].domain = kD2;
         }},
        {"residency_no_rep", [](Editable& e) { e.primitives[1].representation = {}; }},
        {"residency_zero_bytes", [](Editable& e) { e.primitives[1].residency_bytes = 0; }},
        {"no_extra_with_rep", [](Editable& e) { e.primitives[0].representation = reg::RepresentationId{7}; }},
        {"no_extra_with_bytes", [](Editable& e) { e.primitives[0].residency_bytes = 1; }},
        {"both_flags", [](Editable& e) { e.primitives[1].flags |= reg::PRIMITIVE_NO_EXTRA_REPRESENTATION; }},
        {"cap_domain", [](Editable& e) { e.capabilities[0].domain = kD2; }},
        {"cap_preferred_missing", [](Editable& e) { e.capabilities[0].preferred_primitive = kX2; }},
        {"cap_fallback_missing", [](Editable& e) { e.capabilities[0].fallback_primitive = kX2; }},
        {"cap_no_fallback", [](Editable& e) { e.capabilities[0].fallback_primitive = {}; }},
        {"cap_preferred_other_cap", [](Editable& e) {
             e.capabilities.push_back({kC2, e.capabilities[0].domain, e.primitives[1].id, {},
                                       reg::ValidationState::VALIDATED, "C2", {}});
         }},
        {"path_target", [](Editable& e) { e.paths[2].target_primitive = kX2; }},
        {"mandatory_with_threshold", [](Editable& e) {
             e.paths[0].trigger = reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY;
         }},
        {"mandatory_no_threshold", [](Editable& e) {
             e.paths[3].trigger = reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY;
         }},
        {"threshold_cap", [](Editable& e) { e.thresholds[2].capability = kC2; }},
        {"threshold_profile", [](Editable& e) { e.thresholds[2].profile = kP2; }},
        {"threshold_path", [](Editable& e) { e.thresholds[4].acquisition = reg::AcquisitionPathId{0xC1FF}; }},
        {"threshold_metric", [](Editable& e) { e.thresholds[5].reuse_metric = kM2; }},
        {"threshold_profile_without_metric", [](Editable& e) {
             e.profiles[1].reuse_metric = {};
         }},
        {"threshold_on_disabled_path_ok", [](Editable& e) {
             e.thresholds.push_back({e.capabilities[0].id, e.profiles[0].id, e.paths[3].id, e.metrics[0].id, 9,
                                     reg::ValidationState::VALIDATED, {}});
         }},
        {"threshold_target_other_cap", [](Editable& e) {
             e.primitives.push_back({kX2, e.families[0].id, kC2, {}, 0, reg::PRIMITIVE_NO_EXTRA_REPRESENTATION,
                                     reg::ValidationState::VALIDATED, "X2", {}});
             e.capabilities.push_back({kC2, e.capabilities[0].domain, kX2, {}, reg::ValidationState::VALIDATED,
                                       "C2", {}});
             e.paths.push_back({reg::AcquisitionPathId{0xC1F0}, kX2, 5, reg::AcquisitionTrigger::REUSE_AMORTIZED,
                                reg::ValidationState::VALIDATED, "PX", {}});
             e.thresholds.push_back({e.capabilities[0].id, e.profiles[0].id, reg::AcquisitionPathId{0xC1F0},
                                     e.metrics[0].id, 3, reg::ValidationState::VALIDATED, {}});
         }},
        {"lifecycle_prim", [](Editable& e) { e.lifecycles[0].primitive = kX2; }},
        {"no_lifecycle", [](Editable& e) { e.lifecycles.clear(); }},
        {"disabled_descriptors_ok", [](Editable& e) {
             e.capabilities[0].state = reg::ValidationState::DISABLED_BY_EVIDENCE;
             e.profiles[1].state = reg::ValidationState::DISABLED_BY_EVIDENCE;
         }},
        {"empty_bundle", [](Editable& e) {
             Editable x;
             x.name = "EMPTY";
             e = x;
         }},
    };
    for (const Case& c : cases) {
        Editable e(base);
        c.m(e);
        reg::PrimitiveRegistry r;
        dump_add(c.name, r, e.build());
        if (r.bundle_count()) {
            // lookups after a successful add, and after a failed second add of the same bundle
            T.line("%s find cap=%u prof0=%u prim=%u path=%u thr=%u life=%u", c.name,
                   u(r.find_capability(q4::kCapability) != nullptr), u(r.find_profile(q4::kProfile0) != nullptr),
                   u(r.find_primitive(q4::kPrimitiveB) != nullptr), u(r.find_acquisition(q4::kAcquireTertiary) != nullptr),
                   u(r.find_threshold(q4::kCapability, q4::kProfile1, q4::kAcquireSecondary) != nullptr),
                   u(r.find_lifecycle(q4::kPrimitiveB) != nullptr));
            Editable again(base);
            dump_add("readd", r, again.build());
        } else {
            T.line("%s rolled_back cap=%u dom=%u", c.name, u(r.find_capability(q4::kCapability) != nullptr),
                   u(r.find_domain(q4::kDomain) != nullptr));
        }
    }
    // count > 0 with a null pointer, per array
    for (int k = 0; k < 10; ++k) {
        Editable e(base);
        e.count_bump = k;
        e.null_array = k;
        if (k == 0) e.domains.clear();
        reg::PrimitiveRegistry r;
        char tag[32];
        std::snprintf(tag, sizeof tag, "bump%d", k);
        dump_add(tag, r, e.build());
    }
    // cross-bundle: a second bundle repeating only a threshold key or a lifecycle key
    {
        reg::PrimitiveRegistry r;
        dump_add("xb_base", r, base);
        Editable t;
        t.name = "T";
        t.thresholds.push_back(base.thresholds[1]);
        dump_add("xb_threshold", r, t.build());
        Editable l;
        l.name = "L";
        l.lifecycles.push_back(base.lifecycles[0]);
        dump_add("xb_lifecycle", r, l.build());
        Editable m;  // a bundle referring to the first one's descriptors
        m.name = "M";
        m.profiles.push_back({kP2, q4::kDomain, q4::kReuseMetric, q4::kEvidenceSet, reg::ValidationState::VALIDATED,
                              "P2", {}});
        m.thresholds.push_back({q4::kCapability, kP2, q4::kAcquirePrimary, q4::kReuseMetric, 77,
                                reg::ValidationState::VALIDATED, {}});
        dump_add("xb_refers", r, m.build());
        const reg::AcquisitionThresholdDescriptor* xt = r.find_threshold(q4::kCapability, kP2, q4::kAcquirePrimary);
        T.line("xb thr=%" PRIu64, xt ? std::uint64_t(xt->minimum_reuse_units) : std::uint64_t(0));
        for (const reg::DomainId d : {q4::kDomain, kD2}) {
            Editable x;
            x.name = "X";
            x.domains.push_back({d, reg::ValidationState::VALIDATED, "X", {}});
            dump_add("xb_domain", r, x.build());
        }
    }
    // capacity: 64 bundles fit, the 65th does not
    {
        reg::PrimitiveRegistry r;
        static std::vector<Editable> many(66);
        for (std::size_t i = 0; i < many.size(); ++i) {
            many[i] = Editable();
            many[i].name = "CAP" + std::to_string(i);
            many[i].domains.push_back({reg::DomainId{0xDD000000ull + i}, reg::ValidationState::VALIDATED, "C", {}});
            char tag[32];
            std::snprintf(tag, sizeof tag, "cap%zu", i);
            reg::RegistryError e{};
            const reg::RegistryStatus s = r.add_bundle(many[i].build(), &e);
            T.line("%s st=%u cat=%s bundles=%zu at=%u", tag, unsigned(s), e.category ? e.category : "(null)",
                   r.bundle_count(), u(r.bundle_at(i) != nullptr));
        }
        T.line("cap past_end=%u", u(r.bundle_at(r.bundle_count()) != nullptr));
    }
    T.section("registry");
}

// ------------------------------------------------------------ Q4 sweep

void q4_section()
{
    reg::PrimitiveRegistry r;
    if (r.add_bundle(q4::q4k_down_reference_bundle(), nullptr) != reg::RegistryStatus::OK) {
        std::printf("q4 bundle rejected\n");
        std::exit(2);
    }
    static const std::uint64_t H[] = {0, 1, 2, 3, 4, 5, 14, 15, 16, 17, 32, 33, 36, 37, 64, 1000000};
    char tag[64];
    for (int prof = 0; prof < 2; ++prof)
        for (std::uint64_t h : H)
            for (std::uint32_t m = 0; m < (1u << 15); ++m) {
                auto bit = [&](int k) { return (m >> k) & 1u; };
                const gp::PrimitiveRuntimeState ps[] = {
                    {q4::kPrimitiveA, false, true, true, bit(9) != 0, true},
                    {q4::kPrimitiveB, bit(4) != 0, bit(5) != 0, bit(6) != 0, bit(7) != 0, bit(8) != 0}};
                const gp::AcquisitionRuntimeState as[] = {{q4::kAcquirePrimary, bit(10) != 0, bit(11) != 0},
                                                          {q4::kAcquireSecondary, bit(12) != 0, false},
                                                          {q4::kAcquireTertiary, bit(13) != 0, false},
                                                          {q4::kAcquireDisabledWarm, bit(14) != 0, false}};
                gp::PolicyRequest q{};
                q.capability = q4::kCapability;
                q.profile = prof ? q4::kProfile1 : q4::kProfile0;
                q.request_within_capability_evidence_scope = bit(0);
                q.model_loaded = bit(1);
                q.future_reuse_known = bit(2);
                q.future_reuse_units = h;
                q.acquisition_allowed = bit(3);
                q.primitive_states = ps;
                q.primitive_state_count = 2;
                q.acquisition_states = as;
                q.acquisition_state_count = 4;
                std::snprintf(tag, sizeof tag, "q4 p%d h%" PRIu64 " m%04x", prof, h, m);
                dump_decision(tag, gp::evaluate(r, q));
            }
    T.section("q4");
}

// ------------------------------------------------------------ holdouts

namespace ho {
const reg::DomainId D{0xD7000001ull};
const reg::EvidenceSetId E{0xE7000001ull};
const reg::ReuseMetricId M{0xD7000002ull};
const reg::EvidenceProfileId P{0x57000001ull}, PM{0x57000002ull};
const reg::PrimitiveFamilyId F{0xF7000001ull};
const reg::CapabilityId C{0x17000001ull};
const reg::PrimitiveId S{0xA7000001ull}, FB{0xA7000002ull};
const reg::RepresentationId R{0xE7000009ull};
const reg::AcquisitionPathId M1{0xC7000001ull}, M2{0xC7000002ull}, M3{0xC7000003ull}, A1{0xC7000004ull},
    A2{0xC7000005ull};
const auto V = reg::ValidationState::VALIDATED;
const auto OFF = reg::ValidationState::DISABLED_BY_EVIDENCE;

// S represented (mandatory paths M1..M3, amortized A1/A2), FB direct fallback.
Editable base(int variant)
{
    Editable e;
    e.name = "HOLDOUT" + std::to_string(variant);
    e.domains.push_back({D, V, "D", {}});
    e.evidence.push_back({E, V, "E", {}});
    e.metrics.push_back({M, V, "M", {}});
    e.profiles.push_back({P, D, {}, E, V, "P", {}});   // no reuse metric
    e.profiles.push_back({PM, D, M, E, V, "PM", {}});  // with reuse metric
    e.families.push_back({F, D, V, "F", {}});
    e.capabilities.push_back({C, D, S, FB, V, "C", {}});
    e.primitives.push_back({S, F, C, R, 4096, reg::PRIMITIVE_REQUIRES_RESIDENCY | reg::PRIMITIVE_REQUIRES_IDENTITY_VALIDATION,
                            V, "S", {}});
    e.primitives.push_back({FB, F, C, {}, 0, reg::PRIMITIVE_FALLBACK | reg::PRIMITIVE_NO_EXTRA_REPRESENTATION, V, "FB", {}});
    e.lifecycles.push_back({S, false, false, true, false, true, true, {}});
    return e;
}
}  // namespace ho

void holdout_sweep(const char* name, Editable& e, reg::EvidenceProfileId profile, bool with_fallback_state)
{
    reg::PrimitiveRegistry r;
    reg::RegistryError err{};
    const reg::RegistryStatus s = r.add_bundle(e.build(), &err);
    T.line("%s add st=%u cat=%s", name, unsigned(s), err.category ? err.category : "(null)");
    if (s != reg::RegistryStatus::OK) return;
    static const std::uint64_t H[] = {0, 3, 8, 1000};
    char tag[96];
    for (int hk = 0; hk < 5; ++hk)
        for (std::uint32_t m = 0; m < (1u << 12); ++m) {
            auto bit = [&](int k) { return ((m >> k) & 1u) != 0; };
            const gp::PrimitiveRuntimeState ps[] = {{ho::S, bit(3), bit(4), bit(5), bit(6), bit(7)},
                                                    {ho::FB, false, false, bit(8), bit(8), false}};
            const gp::AcquisitionRuntimeState as[] = {{ho::M1, bit(9), false},
                                                      {ho::M2, bit(10), bit(11)},
                                                      {ho::M3, true, false},
                                                      {ho::A1, bit(9), false},
                                                      {ho::A2, true, bit(10)}};
            gp::PolicyRequest q{};
            q.capability = ho::C;
            q.profile = profile;
            q.request_within_capability_evidence_scope = bit(0);
            q.model_loaded = bit(1);
            q.acquisition_allowed = bit(2);
            q.future_reuse_known = hk < 4;
            q.future_reuse_units = hk < 4 ? H[hk] : 5;
            q.primitive_states = ps;
            q.primitive_state_count = with_fallback_state ? 2 : 1;
            q.acquisition_states = as;
            q.acquisition_state_count = 5;
            std::snprintf(tag, sizeof tag, "%s h%d m%03x", name, hk, m);
            dump_decision(tag, gp::evaluate(r, q));
        }
}

void holdout_section()
{
    using namespace ho;
    {
        Editable e = base(0);  // three mandatory paths; M2 and M3 tie on priority
        e.paths.push_back({M1, S, 1, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M1", {}});
        e.paths.push_back({M3, S, 0, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M3", {}});
        e.paths.push_back({M2, S, 0, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M2", {}});
        holdout_sweep("mand_fb", e, P, true);
        holdout_sweep("mand_nofbstate", e, P, false);
        e.capabilities[0].fallback_primitive = {};
        holdout_sweep("mand_nofb", e, P, true);
    }
    {
        Editable e = base(1);  // amortized paths with thresholds, one path without a threshold row
        e.paths.push_back({A1, S, 0, reg::AcquisitionTrigger::REUSE_AMORTIZED, V, "A1", {}});
        e.paths.push_back({A2, S, 1, reg::AcquisitionTrigger::REUSE_AMORTIZED, V, "A2", {}});
        e.paths.push_back({M1, S, 2, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M1", {}});
        e.thresholds.push_back({C, PM, A1, M, 8, V, {}});
        holdout_sweep("amort_missing_thr", e, PM, true);
        e.thresholds.push_back({C, PM, A2, M, 3, V, {}});
        holdout_sweep("amort_mixed", e, PM, true);
        holdout_sweep("amort_no_metric", e, P, true);
        e.thresholds[1].state = OFF;
        holdout_sweep("amort_thr_disabled", e, PM, true);
        e.capabilities[0].fallback_primitive = {};
        holdout_sweep("amort_nofb", e, PM, true);
    }
    {
        Editable e = base(2);  // direct preferred: S without residency
        e.primitives[0].flags = reg::PRIMITIVE_NO_EXTRA_REPRESENTATION;
        e.primitives[0].representation = {};
        e.primitives[0].residency_bytes = 0;
        e.lifecycles.clear();
        holdout_sweep("direct", e, P, true);
        e.capabilities[0].fallback_primitive = {};
        holdout_sweep("direct_nofb", e, P, true);
    }
    {
        Editable e = base(3);  // represented preferred without a lifecycle row
        e.lifecycles.clear();
        e.paths.push_back({M1, S, 0, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M1", {}});
        holdout_sweep("no_lifecycle", e, P, true);
    }
    {
        Editable e = base(4);  // every lifecycle flag off but preserve
        e.lifecycles[0] = {S, true, false, false, false, false, false, {}};
        e.paths.push_back({M1, S, 0, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M1", {}});
        e.paths.push_back({M2, S, 1, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, OFF, "M2", {}});
        holdout_sweep("life_off", e, P, true);
    }
    // disabled descriptors, one at a time
    for (int k = 0; k < 7; ++k) {
        Editable e = base(10 + k);
        e.paths.push_back({M1, S, 0, reg::AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY, V, "M1", {}});
        const char* what = "";
        switch (k) {
            case 0: e.capabilities[0].state = OFF, what = "off_cap"; break;
            case 1: e.profiles[0].state = OFF, what = "off_profile"; break;
            case 2: e.domains[0].state = OFF, what = "off_domain"; break;
            case 3: e.evidence[0].state = OFF, what = "off_evidence"; break;
            case 4: e.primitives[0].state = OFF, what = "off_preferred"; break;
            case 5: e.primitives[1].state = OFF, what = "off_fallback"; break;
            case 6: e.metrics[0].state = OFF, what = "off_metric"; break;
        }
        holdout_sweep(what, e, k == 6 ? PM : P, true);
    }
    // malformed requests and a profile of another domain
    {
        reg::PrimitiveRegistry r;
        Editable e = base(20);
        e.domains.push_back({kD2, V, "D2", {}});
        e.profiles.push_back({kP2, kD2, {}, E, V, "P2", {}});
        const reg::RegistryStatus s = r.add_bundle(e.build(), nullptr);
        T.line("malformed add st=%u", unsigned(s));
        gp::PrimitiveRuntimeState ok[] = {{S, false, true, true, true, true}, {FB, false, true, true, true, true}};
        gp::PrimitiveRuntimeState dup[] = {{S, false, true, true, true, true}, {S, false, true, true, true, true}};
        gp::PrimitiveRuntimeState zero[] = {{{}, false, true, true, true, true}};
        gp::AcquisitionRuntimeState adup[] = {{M1, true, false}, {M1, true, false}};
        gp::AcquisitionRuntimeState azero[] = {{{}, true, false}};
        struct Q {
            const char* name;
            reg::CapabilityId cap;
            reg::EvidenceProfileId prof;
            const gp::PrimitiveRuntimeState* ps;
            std::size_t pn;
            const gp::AcquisitionRuntimeState* as;
            std::size_t an;
        } qs[] = {
            {"req_ok", C, P, ok, 2, nullptr, 0},
            {"req_null_prims", C, P, nullptr, 2, nullptr, 0},
            {"req_null_acqs", C, P, ok, 2, nullptr, 1},
            {"req_dup_prims", C, P, dup, 2, nullptr, 0},
            {"req_zero_prim", C, P, zero, 1, nullptr, 0},
            {"req_dup_acqs", C, P, ok, 2, adup, 2},
            {"req_zero_acq", C, P, ok, 2, azero, 1},
            {"req_unknown_cap", reg::CapabilityId{0x123}, P, ok, 2, nullptr, 0},
            {"req_zero_cap", {}, P, ok, 2, nullptr, 0},
            {"req_unknown_prof", C, reg::EvidenceProfileId{0x456}, ok, 2, nullptr, 0},
            {"req_other_domain", C, kP2, ok, 2, nullptr, 0},
            {"req_empty", C, P, nullptr, 0, nullptr, 0},
        };
        for (const Q& x : qs)
            for (int flags = 0; flags < 4; ++flags) {
                gp::PolicyRequest q{};
                q.capability = x.cap;
                q.profile = x.prof;
                q.request_within_capability_evidence_scope = flags & 1;
                q.model_loaded = (flags & 2) != 0;
                q.primitive_states = x.ps;
                q.primitive_state_count = x.pn;
                q.acquisition_states = x.as;
                q.acquisition_state_count = x.an;
                char tag[64];
                std::snprintf(tag, sizeof tag, "%s f%d", x.name, flags);
                dump_decision(tag, gp::evaluate(r, q));
            }
        // the default-constructed request, and an empty registry
        dump_decision("req_default", gp::evaluate(r, gp::PolicyRequest{}));
        reg::PrimitiveRegistry empty;
        gp::PolicyRequest q{};
        q.capability = C;
        q.profile = P;
        dump_decision("req_empty_registry", gp::evaluate(empty, q));
    }
    T.section("holdout");
}

// ------------------------------------------------------------ binding

class RecordingBackend final : public bind::BackendAdapter {
public:
    unsigned fail = 0;  // bit 0 resolve, 1 acquire, 2 acquire returns a null handle, 3 validate, 4 release,
                        // 5 resolve returns a null handle
    std::uint64_t next_rep = 100;
    std::string log;

    bind::BackendStatus acquire(reg::AcquisitionPathId path, reg::PrimitiveId target, std::uint64_t bytes,
                                bind::RepresentationHandle& out) noexcept override
    {
        note("acq", path.value, target.value, bytes);
        if (fail & 2u) return bind::BackendStatus::RESOURCE_DENIED;
        out = (fail & 4u) ? bind::RepresentationHandle{} : bind::RepresentationHandle{next_rep++};
        return bind::BackendStatus::OK;
    }
    bind::BackendStatus validate(bind::RepresentationHandle rep, reg::CapabilityId cap,
                                 reg::PrimitiveId target) noexcept override
    {
        note("val", rep.opaque, cap.value, target.value);
        return (fail & 8u) ? bind::BackendStatus::VALIDATION_FAILED : bind::BackendStatus::OK;
    }
    bind::BackendStatus release(reg::PrimitiveId target, bind::RepresentationHandle rep) noexcept override
    {
        note("rel", target.value, rep.opaque, 0);
        return (fail & 16u) ? bind::BackendStatus::RELEASE_FAILED : bind::BackendStatus::OK;
    }
    bind::BackendStatus resolve_primitive(reg::PrimitiveId p, bind::PrimitiveHandle& out) noexcept override
    {
        note("res", p.value, 0, 0);
        if (fail & 1u) return bind::BackendStatus::PRIMITIVE_UNAVAILABLE;
        out = (fail & 32u) ? bind::PrimitiveHandle{} : bind::PrimitiveHandle{p.value ^ 0x5000000ull};
        return bind::BackendStatus::OK;
    }

private:
    void note(const char* what, std::uint64_t a, std::uint64_t b, std::uint64_t c)
    {
        char buf[96];
        std::snprintf(buf, sizeof buf, "%s(%" PRIx64 ",%" PRIx64 ",%" PRIu64 ");", what, a, b, c);
        log += buf;
    }
};

void binding_section()
{
    reg::PrimitiveRegistry r;
    (void)r.add_bundle(q4::q4k_down_reference_bundle(), nullptr);
    const reg::PrimitiveId routes[] = {{}, q4::kPrimitiveA, q4::kPrimitiveB, reg::PrimitiveId{0x77}};
    const reg::AcquisitionPathId acqs[] = {{}, q4::kAcquirePrimary};
    const reg::CapabilityId caps[] = {q4::kCapability, reg::CapabilityId{0x999}};
    char tag[128];
    for (int ci = 0; ci < 2; ++ci)
        for (int lc = 0; lc < 4; ++lc)
            for (int ri = 0; ri < 4; ++ri)
                for (int ai = 0; ai < 2; ++ai)
                    for (int val = 0; val < 2; ++val)
                        for (int held = 0; held < 3; ++held)  // 0 none, 1 B held, 2 all slots taken by others
                            for (unsigned fail = 0; fail < 64; ++fail) {
                                gp::PolicyDecision d{};
                                d.route = routes[ri];
                                d.lifecycle = gp::LifecycleAction(lc);  // 3: not a valid action
                                d.acquisition = acqs[ai];
                                d.requested_residency_bytes = 549527552ull;
                                d.require_post_acquisition_identity_validation = val;
                                d.threshold_units = 7;
                                bind::BindingState st{};
                                if (held == 1) (void)st.set(q4::kPrimitiveB, bind::RepresentationHandle{42});
                                if (held == 2)
                                    for (std::size_t k = 0; k < bind::BindingState::kMaxRepresentations; ++k)
                                        (void)st.set(reg::PrimitiveId{0x100 + k}, bind::RepresentationHandle{k + 1});
                                RecordingBackend be;
                                be.fail = fail;
                                const bind::ApplyResult a = bind::apply_decision(r, caps[ci], d, be, st);
                                std::snprintf(tag, sizeof tag, "bind c%d l%d r%d a%d v%d h%d f%02u", ci, lc, ri, ai,
                                              val, held, fail);
                                T.line("%s bs=%u cs=%u unrel=%" PRIu64 " prim=%" PRIx64 " ready=%u held=%" PRIu64
                                       " first=%" PRIx64 " dec=%" PRIx64 "/%u log=%s",
                                       tag, unsigned(a.backend_status), unsigned(a.cleanup_status),
                                       a.unreleased_representation.opaque, a.primitive.opaque, u(a.ready),
                                       st.find(q4::kPrimitiveB).opaque, st.slots[0].primitive.value,
                                       a.decision.route.value, unsigned(a.decision.lifecycle), be.log.c_str());
                            }
    // BindingState on its own
    bind::BindingState st{};
    T.line("state empty find=%" PRIu64, st.find(q4::kPrimitiveA).opaque);
    T.line("state set=%u", u(st.set(q4::kPrimitiveA, bind::RepresentationHandle{5})));
    T.line("state set2=%u", u(st.set(q4::kPrimitiveB, bind::RepresentationHandle{6})));
    T.line("state overwrite=%u", u(st.set(q4::kPrimitiveA, bind::RepresentationHandle{7})));
    T.line("state find=%" PRIu64 "/%" PRIu64, st.find(q4::kPrimitiveA).opaque, st.find(q4::kPrimitiveB).opaque);
    st.clear(q4::kPrimitiveA);
    T.line("state cleared=%" PRIu64 " slot0=%" PRIx64 " slot1=%" PRIx64, st.find(q4::kPrimitiveA).opaque,
           st.slots[0].primitive.value, st.slots[1].primitive.value);
    T.line("state refill=%u slot0=%" PRIx64, u(st.set(q4::kPrimitiveA, bind::RepresentationHandle{8})),
           st.slots[0].primitive.value);
    st.clear(reg::PrimitiveId{0x31337});
    T.line("state zero_id_find=%" PRIu64, st.find(reg::PrimitiveId{}).opaque);
    T.section("binding");
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc > 1) {
        T.out = std::fopen(argv[1], "w");
        if (!T.out) {
            std::perror(argv[1]);
            return 2;
        }
    }
    registry_section();
    q4_section();
    holdout_section();
    binding_section();
    std::printf("total cases=%" PRIu64 " fnv=%016" PRIx64 "\n", T.all, T.total);
    if (T.out) std::fclose(T.out);
    return 0;
}
