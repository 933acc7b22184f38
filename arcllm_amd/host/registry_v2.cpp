// registry_v2.cpp -- PrimitiveRegistry (include/arcllm/v1/primitive_registry_v2.h).
//
// Observable behaviour is that of src/arcllm_v1_primitive_registry_v2.cpp of
// the reference: a lookup returns the first entry with the key over the
// bundles in registration order, and add_bundle reports the FIRST failing
// check with the same status, category and id.  The implementation is table
// driven: the eight id-bearing tables of a bundle are described once
// (kIdTables) and the per-table id checks and the clash checks run over that
// description; the cross-reference rules are an ordered list of rule
// functions (kReferenceRules) run with the bundle tentatively registered.
#include "../../include/arcllm/v1/primitive_registry_v2.h"

#include <utility>

namespace arcllm::v1::registry_v2 {

namespace {

// ------------------------------------------------------------ table access
// Each descriptor type maps to its bundle table (rows, count).
template <typename T>
struct Rows;
#define ARC_ROWS(T, ROWS, COUNT)                                                           \
    template <>                                                                            \
    struct Rows<T> {                                                                       \
        static const T* data(const RegistrationBundle& b) noexcept { return b.ROWS; }     \
        static std::size_t size(const RegistrationBundle& b) noexcept { return b.COUNT; }  \
    };
ARC_ROWS(DomainDescriptor, domains, domain_count)
ARC_ROWS(ReuseMetricDescriptor, reuse_metrics, reuse_metric_count)
ARC_ROWS(EvidenceSetDescriptor, evidence_sets, evidence_set_count)
ARC_ROWS(EvidenceProfileDescriptor, profiles, profile_count)
ARC_ROWS(PrimitiveFamilyDescriptor, families, family_count)
ARC_ROWS(CapabilityDescriptor, capabilities, capability_count)
ARC_ROWS(PrimitiveDescriptor, primitives, primitive_count)
ARC_ROWS(AcquisitionPathDescriptor, acquisitions, acquisition_count)
ARC_ROWS(AcquisitionThresholdDescriptor, thresholds, threshold_count)
ARC_ROWS(LifecycleDescriptor, lifecycles, lifecycle_count)
#undef ARC_ROWS

// The first row of type T, over the registry's bundles in registration
// order, that `match` accepts.
template <typename T, typename Match>
const T* first_row(const PrimitiveRegistry& r, Match match) noexcept
{
    for (std::size_t b = 0; b < r.bundle_count(); ++b) {
        const RegistrationBundle& bundle = *r.bundle_at(b);
        const T* rows = Rows<T>::data(bundle);
        for (std::size_t i = 0, m = Rows<T>::size(bundle); i < m; ++i)
            if (match(rows[i])) return &rows[i];
    }
    return nullptr;
}

// ------------------------------------------------------------------ verdicts
struct Verdict {
    RegistryStatus status = RegistryStatus::OK;
    const char* category = nullptr;
    std::uint64_t id = 0;
    explicit operator bool() const noexcept { return status != RegistryStatus::OK; }  // true: a failure
};
constexpr Verdict kPass{};
Verdict failure(RegistryStatus s, const char* category, std::uint64_t id = 0) noexcept { return Verdict{s, category, id}; }

// ---------------------------------------------------------------- id tables
// An id-bearing table of a bundle: its error category, its rows' ids, and
// whether an id is already registered.
struct IdTable {
    const char* category;
    std::size_t (*size)(const RegistrationBundle&);
    std::uint64_t (*id_at)(const RegistrationBundle&, std::size_t);
    bool (*taken)(const PrimitiveRegistry&, std::uint64_t);
};

template <typename T, typename Id, const T* (PrimitiveRegistry::*Find)(Id) const noexcept>
constexpr IdTable id_table(const char* category) noexcept
{
    return IdTable{category, [](const RegistrationBundle& b) { return Rows<T>::size(b); },
                   [](const RegistrationBundle& b, std::size_t i) { return std::uint64_t(Rows<T>::data(b)[i].id.value); },
                   [](const PrimitiveRegistry& r, std::uint64_t v) {
                       Id id{};
                       id.value = static_cast<decltype(id.value)>(v);
                       return (r.*Find)(id) != nullptr;
                   }};
}

// In the order the checks report them.
const IdTable kIdTables[] = {
    id_table<DomainDescriptor, DomainId, &PrimitiveRegistry::find_domain>("domain"),
    id_table<ReuseMetricDescriptor, ReuseMetricId, &PrimitiveRegistry::find_reuse_metric>("reuse_metric"),
    id_table<EvidenceSetDescriptor, EvidenceSetId, &PrimitiveRegistry::find_evidence_set>("evidence_set"),
    id_table<EvidenceProfileDescriptor, EvidenceProfileId, &PrimitiveRegistry::find_profile>("profile"),
    id_table<PrimitiveFamilyDescriptor, PrimitiveFamilyId, &PrimitiveRegistry::find_family>("family"),
    id_table<CapabilityDescriptor, CapabilityId, &PrimitiveRegistry::find_capability>("capability"),
    id_table<PrimitiveDescriptor, PrimitiveId, &PrimitiveRegistry::find_primitive>("primitive"),
    id_table<AcquisitionPathDescriptor, AcquisitionPathId, &PrimitiveRegistry::find_acquisition>("acquisition"),
};

// Row by row: a zero id is an invalid bundle; an id repeated further down the
// table is a duplicate (reported with the row it first appears at).
Verdict ids_well_formed(const IdTable& t, const RegistrationBundle& b) noexcept
{
    const std::size_t n = t.size(b);
    for (std::size_t i = 0; i < n; ++i) {
        const std::uint64_t v = t.id_at(b, i);
        if (v == 0) return failure(RegistryStatus::INVALID_BUNDLE, t.category);
        for (std::size_t j = i + 1; j < n; ++j)
            if (t.id_at(b, j) == v) return failure(RegistryStatus::DUPLICATE_ID, t.category, v);
    }
    return kPass;
}

Verdict ids_unregistered(const IdTable& t, const RegistrationBundle& b, const PrimitiveRegistry& r) noexcept
{
    for (std::size_t i = 0, n = t.size(b); i < n; ++i)
        if (t.taken(r, t.id_at(b, i))) return failure(RegistryStatus::DUPLICATE_ID, t.category, t.id_at(b, i));
    return kPass;
}

// ------------------------------------------------------------- policy keys
bool same_threshold_key(const AcquisitionThresholdDescriptor& a, const AcquisitionThresholdDescriptor& b) noexcept
{
    return a.capability == b.capability && a.profile == b.profile && a.acquisition == b.acquisition;
}

// Threshold keys, then lifecycle primitives, of `x` against the rows of `y`
// (y == x: against the rows after each one).
Verdict keys_disjoint(const RegistrationBundle& x, const RegistrationBundle& y) noexcept
{
    const bool self = &x == &y;
    for (std::size_t i = 0; i < x.threshold_count; ++i)
        for (std::size_t j = self ? i + 1 : 0; j < y.threshold_count; ++j)
            if (same_threshold_key(x.thresholds[i], y.thresholds[j]))
                return failure(RegistryStatus::DUPLICATE_POLICY_KEY, "threshold");
    for (std::size_t i = 0; i < x.lifecycle_count; ++i)
        for (std::size_t j = self ? i + 1 : 0; j < y.lifecycle_count; ++j)
            if (x.lifecycles[i].primitive == y.lifecycles[j].primitive)
                return failure(RegistryStatus::DUPLICATE_POLICY_KEY, "lifecycle", x.lifecycles[i].primitive.value);
    return kPass;
}

// -------------------------------------------------------- reference rules
// Each rule walks one table of the new bundle x, resolving references
// through the registry r (x already included), and reports its first row
// that breaks the rule.
using Rule = Verdict (*)(const PrimitiveRegistry& r, const RegistrationBundle& x);

Verdict profile_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.profile_count; ++i) {
        const EvidenceProfileDescriptor& p = x.profiles[i];
        const bool resolved = r.find_domain(p.domain) && r.find_evidence_set(p.evidence_set);
        if (!resolved) return failure(RegistryStatus::INVALID_REFERENCE, "profile_reference", p.id.value);
        if (p.reuse_metric && !r.find_reuse_metric(p.reuse_metric))
            return failure(RegistryStatus::INVALID_REFERENCE, "profile_reuse_metric", p.id.value);
    }
    return kPass;
}

Verdict family_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.family_count; ++i)
        if (!r.find_domain(x.families[i].domain))
            return failure(RegistryStatus::INVALID_REFERENCE, "family_domain", x.families[i].id.value);
    return kPass;
}

Verdict primitive_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.primitive_count; ++i) {
        const PrimitiveDescriptor& p = x.primitives[i];
        const PrimitiveFamilyDescriptor* family = r.find_family(p.family);
        const CapabilityDescriptor* owner = r.find_capability(p.capability);
        if (!family || !owner || family->domain != owner->domain)
            return failure(RegistryStatus::INVALID_REFERENCE, "primitive_reference", p.id.value);
        const bool holds = p.representation && p.residency_bytes != 0;
        const bool none = !p.representation && p.residency_bytes == 0;
        if ((p.flags & PRIMITIVE_REQUIRES_RESIDENCY) && !holds)
            return failure(RegistryStatus::INVALID_REFERENCE, "primitive_residency", p.id.value);
        if ((p.flags & PRIMITIVE_NO_EXTRA_REPRESENTATION) && !none)
            return failure(RegistryStatus::INVALID_REFERENCE, "primitive_no_extra_representation", p.id.value);
    }
    return kPass;
}

// A primitive that exists and belongs to capability c.
bool owned_by(const PrimitiveRegistry& r, PrimitiveId p, CapabilityId c) noexcept
{
    const PrimitiveDescriptor* d = r.find_primitive(p);
    return d && d->capability == c;
}

Verdict capability_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.capability_count; ++i) {
        const CapabilityDescriptor& c = x.capabilities[i];
        if (!r.find_domain(c.domain)) return failure(RegistryStatus::INVALID_REFERENCE, "capability_domain", c.id.value);
        if (!owned_by(r, c.preferred_primitive, c.id))
            return failure(RegistryStatus::INVALID_REFERENCE, "capability_preferred", c.id.value);
        if (c.fallback_primitive && !owned_by(r, c.fallback_primitive, c.id))
            return failure(RegistryStatus::INVALID_REFERENCE, "capability_fallback", c.id.value);
    }
    return kPass;
}

Verdict acquisition_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.acquisition_count; ++i) {
        const AcquisitionPathDescriptor& a = x.acquisitions[i];
        if (!r.find_primitive(a.target_primitive))
            return failure(RegistryStatus::INVALID_REFERENCE, "acquisition_target", a.id.value);
        // a mandatory path carries no threshold anywhere in the registry
        const auto on_path = [&](const AcquisitionThresholdDescriptor& t) { return t.acquisition == a.id; };
        if (a.trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY &&
            first_row<AcquisitionThresholdDescriptor>(r, on_path))
            return failure(RegistryStatus::INVALID_ACQUISITION_SEMANTICS, "mandatory_path_has_threshold", a.id.value);
    }
    return kPass;
}

Verdict threshold_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.threshold_count; ++i) {
        const AcquisitionThresholdDescriptor& t = x.thresholds[i];
        const CapabilityDescriptor* c = r.find_capability(t.capability);
        const EvidenceProfileDescriptor* p = r.find_profile(t.profile);
        const AcquisitionPathDescriptor* a = r.find_acquisition(t.acquisition);
        const bool metric = r.find_reuse_metric(t.reuse_metric) != nullptr;
        const bool coherent = c && p && a && metric && p->domain == c->domain && p->reuse_metric &&
                              p->reuse_metric == t.reuse_metric;
        if (!coherent) return failure(RegistryStatus::INVALID_REFERENCE, "threshold_reference");
        if (a->trigger != AcquisitionTrigger::REUSE_AMORTIZED)
            return failure(RegistryStatus::INVALID_ACQUISITION_SEMANTICS, "threshold_on_non_amortized_path", a->id.value);
        if (!owned_by(r, a->target_primitive, c->id)) return failure(RegistryStatus::INVALID_REFERENCE, "threshold_target");
    }
    return kPass;
}

Verdict lifecycle_refs(const PrimitiveRegistry& r, const RegistrationBundle& x)
{
    for (std::size_t i = 0; i < x.lifecycle_count; ++i)
        if (!r.find_primitive(x.lifecycles[i].primitive))
            return failure(RegistryStatus::INVALID_REFERENCE, "lifecycle_primitive", x.lifecycles[i].primitive.value);
    return kPass;
}

const Rule kReferenceRules[] = {profile_refs,    family_refs,      primitive_refs, capability_refs,
                                acquisition_refs, threshold_refs, lifecycle_refs};

// Every table pointer present where its count is nonzero, and a name.
bool well_shaped(const RegistrationBundle& b) noexcept
{
    const std::pair<const void*, std::size_t> tables[] = {
        {b.domains, b.domain_count},         {b.reuse_metrics, b.reuse_metric_count},
        {b.evidence_sets, b.evidence_set_count}, {b.profiles, b.profile_count},
        {b.families, b.family_count},        {b.capabilities, b.capability_count},
        {b.primitives, b.primitive_count},   {b.acquisitions, b.acquisition_count},
        {b.thresholds, b.threshold_count},   {b.lifecycles, b.lifecycle_count}};
    if (!b.bundle_name) return false;
    for (const auto& t : tables)
        if (t.second != 0 && t.first == nullptr) return false;
    return true;
}

}  // namespace

const RegistrationBundle* PrimitiveRegistry::bundle_at(std::size_t index) const noexcept
{
    return index < bundle_count_ ? bundles_[index] : nullptr;
}

#define ARC_FIND_BY_ID(T, Id, Name)                                                                  \
    const T* PrimitiveRegistry::Name(Id id) const noexcept                                           \
    {                                                                                                \
        if (!id) return nullptr;                                                                     \
        return first_row<T>(*this, [&](const T& row) { return row.id == id; });                      \
    }
ARC_FIND_BY_ID(DomainDescriptor, DomainId, find_domain)
ARC_FIND_BY_ID(ReuseMetricDescriptor, ReuseMetricId, find_reuse_metric)
ARC_FIND_BY_ID(EvidenceSetDescriptor, EvidenceSetId, find_evidence_set)
ARC_FIND_BY_ID(EvidenceProfileDescriptor, EvidenceProfileId, find_profile)
ARC_FIND_BY_ID(PrimitiveFamilyDescriptor, PrimitiveFamilyId, find_family)
ARC_FIND_BY_ID(CapabilityDescriptor, CapabilityId, find_capability)
ARC_FIND_BY_ID(PrimitiveDescriptor, PrimitiveId, find_primitive)
ARC_FIND_BY_ID(AcquisitionPathDescriptor, AcquisitionPathId, find_acquisition)
#undef ARC_FIND_BY_ID

const AcquisitionThresholdDescriptor* PrimitiveRegistry::find_threshold(CapabilityId capability,
                                                                       EvidenceProfileId profile,
                                                                       AcquisitionPathId acquisition) const noexcept
{
    const AcquisitionThresholdDescriptor key{capability, profile, acquisition};
    return first_row<AcquisitionThresholdDescriptor>(
        *this, [&](const AcquisitionThresholdDescriptor& row) { return same_threshold_key(row, key); });
}

const LifecycleDescriptor* PrimitiveRegistry::find_lifecycle(PrimitiveId primitive) const noexcept
{
    return first_row<LifecycleDescriptor>(*this,
                                          [&](const LifecycleDescriptor& row) { return row.primitive == primitive; });
}

RegistryStatus PrimitiveRegistry::add_bundle(const RegistrationBundle& x, RegistryError* error) noexcept
{
    auto report = [error](const Verdict& v) noexcept {
        if (error) *error = RegistryError{v.status, v.category, v.id};
        return v.status;
    };
    report(kPass);
    if (bundle_count_ >= kMaxBundles) return report(failure(RegistryStatus::CAPACITY_EXCEEDED, "bundle"));
    if (!well_shaped(x)) return report(failure(RegistryStatus::INVALID_BUNDLE, "bundle"));

    // the bundle on its own, then against what is registered
    for (const IdTable& t : kIdTables)
        if (const Verdict v = ids_well_formed(t, x)) return report(v);
    if (const Verdict v = keys_disjoint(x, x)) return report(v);
    for (const IdTable& t : kIdTables)
        if (const Verdict v = ids_unregistered(t, x, *this)) return report(v);
    for (std::size_t b = 0; b < bundle_count_; ++b)
        if (const Verdict v = keys_disjoint(x, *bundles_[b])) return report(v);

    // references resolve with the bundle in place; withdrawn on failure
    bundles_[bundle_count_++] = &x;
    for (Rule rule : kReferenceRules)
        if (const Verdict v = rule(*this, x)) {
            bundles_[--bundle_count_] = nullptr;
            return report(v);
        }
    return report(kPass);
}

}  // namespace arcllm::v1::registry_v2
