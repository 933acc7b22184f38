// registry_v2.cpp -- PrimitiveRegistry (include/arcllm/v1/primitive_registry_v2.h).
//
// Behaviour of src/arcllm_v1_primitive_registry_v2.cpp of the reference:
// lookups scan the registered bundles in registration order and return the
// first entry with the id; add_bundle runs its checks in a fixed order (shape,
// per-table ids, policy keys, clashes with registered bundles, then
// references with the bundle tentatively registered) and reports the first
// failure with the same status, category and id.
#include "../../include/arcllm/v1/primitive_registry_v2.h"

namespace arcllm::v1::registry_v2 {

namespace {

RegistryStatus fail(RegistryError* e, RegistryStatus s, const char* category, std::uint64_t id = 0) noexcept
{
    if (e) {
        e->status = s;
        e->category = category;
        e->id = id;
    }
    return s;
}

template <typename T>
bool table_ok(const T* p, std::size_t n) noexcept
{
    return n == 0 || p != nullptr;
}

// Every id of a table is nonzero and unique within the table.
template <typename T>
RegistryStatus check_table_ids(const T* t, std::size_t n, const char* category, RegistryError* e) noexcept
{
    for (std::size_t i = 0; i < n; ++i) {
        if (!t[i].id) return fail(e, RegistryStatus::INVALID_BUNDLE, category);
        for (std::size_t j = i + 1; j < n; ++j)
            if (t[j].id == t[i].id) return fail(e, RegistryStatus::DUPLICATE_ID, category, t[i].id.value);
    }
    return RegistryStatus::OK;
}

bool same_key(const AcquisitionThresholdDescriptor& a, const AcquisitionThresholdDescriptor& b) noexcept
{
    return a.capability == b.capability && a.profile == b.profile && a.acquisition == b.acquisition;
}

// First entry with `id` over the bundles, in registration order.
template <typename T, typename Id>
const T* lookup(const RegistrationBundle* const* bundles, std::size_t nb, Id id,
                const T* RegistrationBundle::*table, std::size_t RegistrationBundle::*count) noexcept
{
    if (!id) return nullptr;
    for (std::size_t b = 0; b < nb; ++b) {
        const T* t = bundles[b]->*table;
        const std::size_t n = bundles[b]->*count;
        for (std::size_t i = 0; i < n; ++i)
            if (t[i].id == id) return &t[i];
    }
    return nullptr;
}

}  // namespace

const RegistrationBundle* PrimitiveRegistry::bundle_at(std::size_t index) const noexcept
{
    return index < bundle_count_ ? bundles_[index] : nullptr;
}

const DomainDescriptor* PrimitiveRegistry::find_domain(DomainId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::domains, &RegistrationBundle::domain_count);
}
const ReuseMetricDescriptor* PrimitiveRegistry::find_reuse_metric(ReuseMetricId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::reuse_metrics,
                  &RegistrationBundle::reuse_metric_count);
}
const EvidenceSetDescriptor* PrimitiveRegistry::find_evidence_set(EvidenceSetId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::evidence_sets,
                  &RegistrationBundle::evidence_set_count);
}
const EvidenceProfileDescriptor* PrimitiveRegistry::find_profile(EvidenceProfileId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::profiles, &RegistrationBundle::profile_count);
}
const PrimitiveFamilyDescriptor* PrimitiveRegistry::find_family(PrimitiveFamilyId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::families, &RegistrationBundle::family_count);
}
const CapabilityDescriptor* PrimitiveRegistry::find_capability(CapabilityId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::capabilities,
                  &RegistrationBundle::capability_count);
}
const PrimitiveDescriptor* PrimitiveRegistry::find_primitive(PrimitiveId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::primitives, &RegistrationBundle::primitive_count);
}
const AcquisitionPathDescriptor* PrimitiveRegistry::find_acquisition(AcquisitionPathId id) const noexcept
{
    return lookup(bundles_, bundle_count_, id, &RegistrationBundle::acquisitions,
                  &RegistrationBundle::acquisition_count);
}

const AcquisitionThresholdDescriptor* PrimitiveRegistry::find_threshold(CapabilityId capability,
                                                                       EvidenceProfileId profile,
                                                                       AcquisitionPathId acquisition) const noexcept
{
    for (std::size_t b = 0; b < bundle_count_; ++b)
        for (std::size_t i = 0; i < bundles_[b]->threshold_count; ++i) {
            const AcquisitionThresholdDescriptor& t = bundles_[b]->thresholds[i];
            if (t.capability == capability && t.profile == profile && t.acquisition == acquisition) return &t;
        }
    return nullptr;
}

const LifecycleDescriptor* PrimitiveRegistry::find_lifecycle(PrimitiveId primitive) const noexcept
{
    for (std::size_t b = 0; b < bundle_count_; ++b)
        for (std::size_t i = 0; i < bundles_[b]->lifecycle_count; ++i)
            if (bundles_[b]->lifecycles[i].primitive == primitive) return &bundles_[b]->lifecycles[i];
    return nullptr;
}

RegistryStatus PrimitiveRegistry::add_bundle(const RegistrationBundle& x, RegistryError* e) noexcept
{
    fail(e, RegistryStatus::OK, nullptr);
    if (bundle_count_ >= kMaxBundles) return fail(e, RegistryStatus::CAPACITY_EXCEEDED, "bundle");
    const bool shape_ok = x.bundle_name && table_ok(x.domains, x.domain_count) &&
                          table_ok(x.reuse_metrics, x.reuse_metric_count) &&
                          table_ok(x.evidence_sets, x.evidence_set_count) && table_ok(x.profiles, x.profile_count) &&
                          table_ok(x.families, x.family_count) && table_ok(x.capabilities, x.capability_count) &&
                          table_ok(x.primitives, x.primitive_count) && table_ok(x.acquisitions, x.acquisition_count) &&
                          table_ok(x.thresholds, x.threshold_count) && table_ok(x.lifecycles, x.lifecycle_count);
    if (!shape_ok) return fail(e, RegistryStatus::INVALID_BUNDLE, "bundle");

    // ids: nonzero and unique inside each table
    RegistryStatus s;
    if ((s = check_table_ids(x.domains, x.domain_count, "domain", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.reuse_metrics, x.reuse_metric_count, "reuse_metric", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.evidence_sets, x.evidence_set_count, "evidence_set", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.profiles, x.profile_count, "profile", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.families, x.family_count, "family", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.capabilities, x.capability_count, "capability", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.primitives, x.primitive_count, "primitive", e)) != RegistryStatus::OK) return s;
    if ((s = check_table_ids(x.acquisitions, x.acquisition_count, "acquisition", e)) != RegistryStatus::OK) return s;

    // policy keys: one threshold per (capability, profile, path), one lifecycle per primitive
    for (std::size_t i = 0; i < x.threshold_count; ++i)
        for (std::size_t j = i + 1; j < x.threshold_count; ++j)
            if (same_key(x.thresholds[i], x.thresholds[j]))
                return fail(e, RegistryStatus::DUPLICATE_POLICY_KEY, "threshold");
    for (std::size_t i = 0; i < x.lifecycle_count; ++i)
        for (std::size_t j = i + 1; j < x.lifecycle_count; ++j)
            if (x.lifecycles[i].primitive == x.lifecycles[j].primitive)
                return fail(e, RegistryStatus::DUPLICATE_POLICY_KEY, "lifecycle", x.lifecycles[i].primitive.value);

    // clashes with what is registered
    for (std::size_t i = 0; i < x.domain_count; ++i)
        if (find_domain(x.domains[i].id)) return fail(e, RegistryStatus::DUPLICATE_ID, "domain", x.domains[i].id.value);
    for (std::size_t i = 0; i < x.reuse_metric_count; ++i)
        if (find_reuse_metric(x.reuse_metrics[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "reuse_metric", x.reuse_metrics[i].id.value);
    for (std::size_t i = 0; i < x.evidence_set_count; ++i)
        if (find_evidence_set(x.evidence_sets[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "evidence_set", x.evidence_sets[i].id.value);
    for (std::size_t i = 0; i < x.profile_count; ++i)
        if (find_profile(x.profiles[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "profile", x.profiles[i].id.value);
    for (std::size_t i = 0; i < x.family_count; ++i)
        if (find_family(x.families[i].id)) return fail(e, RegistryStatus::DUPLICATE_ID, "family", x.families[i].id.value);
    for (std::size_t i = 0; i < x.capability_count; ++i)
        if (find_capability(x.capabilities[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "capability", x.capabilities[i].id.value);
    for (std::size_t i = 0; i < x.primitive_count; ++i)
        if (find_primitive(x.primitives[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "primitive", x.primitives[i].id.value);
    for (std::size_t i = 0; i < x.acquisition_count; ++i)
        if (find_acquisition(x.acquisitions[i].id))
            return fail(e, RegistryStatus::DUPLICATE_ID, "acquisition", x.acquisitions[i].id.value);
    for (std::size_t b = 0; b < bundle_count_; ++b) {
        const RegistrationBundle& old = *bundles_[b];
        for (std::size_t i = 0; i < x.threshold_count; ++i)
            for (std::size_t j = 0; j < old.threshold_count; ++j)
                if (same_key(x.thresholds[i], old.thresholds[j]))
                    return fail(e, RegistryStatus::DUPLICATE_POLICY_KEY, "threshold");
        for (std::size_t i = 0; i < x.lifecycle_count; ++i)
            for (std::size_t j = 0; j < old.lifecycle_count; ++j)
                if (x.lifecycles[i].primitive == old.lifecycles[j].primitive)
                    return fail(e, RegistryStatus::DUPLICATE_POLICY_KEY, "lifecycle", x.lifecycles[i].primitive.value);
    }

    // references, resolved with the bundle in place; undone on failure
    bundles_[bundle_count_++] = &x;
    auto reject = [&](RegistryStatus st, const char* category, std::uint64_t id = 0) noexcept {
        bundles_[--bundle_count_] = nullptr;
        return fail(e, st, category, id);
    };

    for (std::size_t i = 0; i < x.profile_count; ++i) {
        const EvidenceProfileDescriptor& p = x.profiles[i];
        if (!find_domain(p.domain) || !find_evidence_set(p.evidence_set))
            return reject(RegistryStatus::INVALID_REFERENCE, "profile_reference", p.id.value);
        if (p.reuse_metric && !find_reuse_metric(p.reuse_metric))
            return reject(RegistryStatus::INVALID_REFERENCE, "profile_reuse_metric", p.id.value);
    }
    for (std::size_t i = 0; i < x.family_count; ++i)
        if (!find_domain(x.families[i].domain))
            return reject(RegistryStatus::INVALID_REFERENCE, "family_domain", x.families[i].id.value);
    for (std::size_t i = 0; i < x.primitive_count; ++i) {
        const PrimitiveDescriptor& p = x.primitives[i];
        const PrimitiveFamilyDescriptor* fam = find_family(p.family);
        const CapabilityDescriptor* cap = find_capability(p.capability);
        if (!fam || !cap || fam->domain != cap->domain)
            return reject(RegistryStatus::INVALID_REFERENCE, "primitive_reference", p.id.value);
        if ((p.flags & PRIMITIVE_REQUIRES_RESIDENCY) && (!p.representation || p.residency_bytes == 0))
            return reject(RegistryStatus::INVALID_REFERENCE, "primitive_residency", p.id.value);
        if ((p.flags & PRIMITIVE_NO_EXTRA_REPRESENTATION) && (p.representation || p.residency_bytes != 0))
            return reject(RegistryStatus::INVALID_REFERENCE, "primitive_no_extra_representation", p.id.value);
    }
    for (std::size_t i = 0; i < x.capability_count; ++i) {
        const CapabilityDescriptor& c = x.capabilities[i];
        if (!find_domain(c.domain)) return reject(RegistryStatus::INVALID_REFERENCE, "capability_domain", c.id.value);
        const PrimitiveDescriptor* pref = find_primitive(c.preferred_primitive);
        if (!pref || pref->capability != c.id)
            return reject(RegistryStatus::INVALID_REFERENCE, "capability_preferred", c.id.value);
        if (c.fallback_primitive) {
            const PrimitiveDescriptor* fb = find_primitive(c.fallback_primitive);
            if (!fb || fb->capability != c.id)
                return reject(RegistryStatus::INVALID_REFERENCE, "capability_fallback", c.id.value);
        }
    }
    for (std::size_t i = 0; i < x.acquisition_count; ++i) {
        const AcquisitionPathDescriptor& a = x.acquisitions[i];
        if (!find_primitive(a.target_primitive))
            return reject(RegistryStatus::INVALID_REFERENCE, "acquisition_target", a.id.value);
        if (a.trigger != AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY) continue;
        // a mandatory path carries no threshold, here or in an earlier bundle
        for (std::size_t b = 0; b < bundle_count_; ++b) {
            const RegistrationBundle& y = *bundles_[b];
            for (std::size_t j = 0; j < y.threshold_count; ++j)
                if (y.thresholds[j].acquisition == a.id)
                    return reject(RegistryStatus::INVALID_ACQUISITION_SEMANTICS, "mandatory_path_has_threshold",
                                  a.id.value);
        }
    }
    for (std::size_t i = 0; i < x.threshold_count; ++i) {
        const AcquisitionThresholdDescriptor& t = x.thresholds[i];
        const CapabilityDescriptor* c = find_capability(t.capability);
        const EvidenceProfileDescriptor* p = find_profile(t.profile);
        const AcquisitionPathDescriptor* a = find_acquisition(t.acquisition);
        const ReuseMetricDescriptor* m = find_reuse_metric(t.reuse_metric);
        if (!c || !p || !a || !m || p->domain != c->domain || !p->reuse_metric || p->reuse_metric != t.reuse_metric)
            return reject(RegistryStatus::INVALID_REFERENCE, "threshold_reference");
        if (a->trigger != AcquisitionTrigger::REUSE_AMORTIZED)
            return reject(RegistryStatus::INVALID_ACQUISITION_SEMANTICS, "threshold_on_non_amortized_path",
                          a->id.value);
        const PrimitiveDescriptor* target = find_primitive(a->target_primitive);
        if (!target || target->capability != c->id)
            return reject(RegistryStatus::INVALID_REFERENCE, "threshold_target");
    }
    for (std::size_t i = 0; i < x.lifecycle_count; ++i)
        if (!find_primitive(x.lifecycles[i].primitive))
            return reject(RegistryStatus::INVALID_REFERENCE, "lifecycle_primitive", x.lifecycles[i].primitive.value);
    return RegistryStatus::OK;
}

}  // namespace arcllm::v1::registry_v2
