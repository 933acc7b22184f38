// policy_v4.cpp -- policy_v4::evaluate (include/arcllm/v1/generic_policy_engine_v4.h).
//
// The decision procedure of src/arcllm_v1_generic_policy_engine_v4.cpp of the
// reference, in this order:
//  1. request/registry consistency (runtime arrays, capability, profile and
//     its domain, evidence, reuse metric, preferred and fallback primitives,
//     lifecycle of a represented preferred primitive);
//  2. a resident representation of the preferred primitive: evict it when its
//     lifecycle says so (model unloaded, identity invalid, execution
//     unavailable, lease revoked, zero future reuse), route to the fallback
//     outside the evidence scope, else reuse it if routable;
//  3. no residency: model unloaded or outside the scope -> fallback; a
//     preferred primitive without a representation is routed directly;
//  4. acquisition: among the available, unvetoed, leased paths to the
//     preferred primitive, mandatory paths always qualify and reuse-amortized
//     paths when the known future reuse meets their threshold; the best path
//     (lowest priority value, then lowest id) is acquired; otherwise the
//     fallback with the reason that explains why nothing was acquired.
// "Routable" = execution available and ready, and for a represented
// primitive also resident, identity-valid and leased.
#include "../../include/arcllm/v1/generic_policy_engine_v4.h"

namespace arcllm::v1::policy_v4 {

namespace {

using registry_v2::AcquisitionPathDescriptor;
using registry_v2::AcquisitionThresholdDescriptor;
using registry_v2::AcquisitionTrigger;
using registry_v2::LifecycleDescriptor;
using registry_v2::PrimitiveDescriptor;
using registry_v2::ValidationState;

bool is_validated(ValidationState s) noexcept { return s == ValidationState::VALIDATED; }

bool has_representation(const PrimitiveDescriptor& p) noexcept
{
    return (p.flags & registry_v2::PRIMITIVE_REQUIRES_RESIDENCY) != 0;
}

// Nonzero, pairwise distinct ids in both runtime arrays.
bool runtime_arrays_ok(const PolicyRequest& r) noexcept
{
    if ((r.primitive_state_count && !r.primitive_states) || (r.acquisition_state_count && !r.acquisition_states))
        return false;
    for (std::size_t i = 0; i < r.primitive_state_count; ++i) {
        if (!r.primitive_states[i].primitive) return false;
        for (std::size_t j = 0; j < i; ++j)
            if (r.primitive_states[j].primitive == r.primitive_states[i].primitive) return false;
    }
    for (std::size_t i = 0; i < r.acquisition_state_count; ++i) {
        if (!r.acquisition_states[i].acquisition) return false;
        for (std::size_t j = 0; j < i; ++j)
            if (r.acquisition_states[j].acquisition == r.acquisition_states[i].acquisition) return false;
    }
    return true;
}

const PrimitiveRuntimeState* state_of(const PolicyRequest& r, PrimitiveId id) noexcept
{
    for (std::size_t i = 0; i < r.primitive_state_count; ++i)
        if (r.primitive_states[i].primitive == id) return &r.primitive_states[i];
    return nullptr;
}

const AcquisitionRuntimeState* state_of(const PolicyRequest& r, AcquisitionPathId id) noexcept
{
    for (std::size_t i = 0; i < r.acquisition_state_count; ++i)
        if (r.acquisition_states[i].acquisition == id) return &r.acquisition_states[i];
    return nullptr;
}

bool routable(const PrimitiveDescriptor& p, const PrimitiveRuntimeState* s) noexcept
{
    if (!s || !s->execution_available || !s->execution_ready) return false;
    return !has_representation(p) || (s->resident && s->identity_valid && s->residency_lease_granted);
}

PolicyDecision make(PolicyStatus status, PrimitiveId route, PolicyReason reason, bool preserve = false) noexcept
{
    PolicyDecision d{};
    d.status = status;
    d.route = route;
    d.reason = reason;
    d.preserve_existing_representation = preserve;
    return d;
}

PolicyDecision unsupported(PolicyStatus status) noexcept
{
    return make(status, {}, PolicyReason::UNSUPPORTED_REQUEST);
}

// The fallback primitive if it can run now; otherwise no route, with
// FALLBACK_NOT_READY when a fallback exists and `none_reason` when not.
PolicyDecision to_fallback(const PrimitiveDescriptor* fb, const PrimitiveRuntimeState* fs, PolicyReason reason,
                           PolicyStatus none_status, PolicyReason none_reason, bool preserve = false) noexcept
{
    if (fb && routable(*fb, fs)) return make(PolicyStatus::OK, fb->id, reason, preserve);
    return make(none_status, {}, fb ? PolicyReason::FALLBACK_NOT_READY : none_reason, preserve);
}

PolicyDecision evict(const PrimitiveDescriptor* fb, const PrimitiveRuntimeState* fs, PolicyReason reason) noexcept
{
    PolicyDecision d = to_fallback(fb, fs, reason, PolicyStatus::NOT_READY, reason);
    d.lifecycle = LifecycleAction::EVICT;
    return d;
}

struct PathChoice {
    const AcquisitionPathDescriptor* path = nullptr;
    const AcquisitionThresholdDescriptor* threshold = nullptr;
    const PrimitiveDescriptor* target = nullptr;
};

// `c` replaces the current choice when there is none or c's path ranks first.
void keep_best(PathChoice& cur, const PathChoice& c) noexcept
{
    if (!cur.path || c.path->priority < cur.path->priority ||
        (c.path->priority == cur.path->priority && c.path->id.value < cur.path->id.value))
        cur = c;
}

}  // namespace

PolicyDecision evaluate(const PrimitiveRegistry& registry, const PolicyRequest& r) noexcept
{
    // 1. consistency
    if (!runtime_arrays_ok(r)) return unsupported(PolicyStatus::INVALID_RUNTIME_STATE);
    const registry_v2::CapabilityDescriptor* cap = registry.find_capability(r.capability);
    if (!cap || !is_validated(cap->state)) return unsupported(PolicyStatus::UNSUPPORTED_CAPABILITY);
    const registry_v2::EvidenceProfileDescriptor* prof = registry.find_profile(r.profile);
    if (!prof || !is_validated(prof->state)) return unsupported(PolicyStatus::UNSUPPORTED_PROFILE);
    if (prof->domain != cap->domain) return unsupported(PolicyStatus::PROFILE_DOMAIN_MISMATCH);
    const auto* dom = registry.find_domain(cap->domain);
    const auto* evid = registry.find_evidence_set(prof->evidence_set);
    if (!dom || !evid || !is_validated(dom->state) || !is_validated(evid->state))
        return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    if (prof->reuse_metric) {
        const auto* metric = registry.find_reuse_metric(prof->reuse_metric);
        if (!metric || !is_validated(metric->state)) return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    }
    const PrimitiveDescriptor* pref = registry.find_primitive(cap->preferred_primitive);
    if (!pref || !is_validated(pref->state) || pref->capability != cap->id)
        return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    const PrimitiveDescriptor* fb = nullptr;
    if (cap->fallback_primitive) {
        fb = registry.find_primitive(cap->fallback_primitive);
        if (!fb || !is_validated(fb->state) || fb->capability != cap->id)
            return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    }
    const PrimitiveRuntimeState* ps = state_of(r, pref->id);
    const PrimitiveRuntimeState* fs = fb ? state_of(r, fb->id) : nullptr;
    const LifecycleDescriptor* life = registry.find_lifecycle(pref->id);
    if (has_representation(*pref) && !life) return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);

    // 2. a resident representation of the preferred primitive
    if (ps && ps->resident && has_representation(*pref)) {
        if (!r.model_loaded && life->evict_on_model_unload) return evict(fb, fs, PolicyReason::MODEL_UNAVAILABLE);
        if (!ps->identity_valid && life->evict_on_identity_invalid)
            return evict(fb, fs, PolicyReason::RESIDENT_PRIMITIVE_INVALID);
        if (!ps->execution_available && life->evict_on_execution_unavailable)
            return evict(fb, fs, PolicyReason::RESIDENT_EXECUTION_UNAVAILABLE);
        if (!ps->residency_lease_granted && life->evict_on_lease_revoke)
            return evict(fb, fs, PolicyReason::RESIDENCY_LEASE_REVOKED);
        if (r.future_reuse_known && r.future_reuse_units == 0 && life->evict_on_zero_future_reuse)
            return evict(fb, fs, PolicyReason::NO_FUTURE_REUSE);
        if (!r.request_within_capability_evidence_scope)
            return to_fallback(fb, fs, PolicyReason::OUTSIDE_VALIDATED_DOMAIN,
                               PolicyStatus::OUTSIDE_VALIDATED_CAPABILITY,
                               PolicyReason::OUTSIDE_EVIDENCE_SCOPE_NO_FALLBACK,
                               life->preserve_residency_outside_domain);
        if (routable(*pref, ps))
            return make(PolicyStatus::OK, pref->id, PolicyReason::RESIDENT_PRIMITIVE_REUSED, true);
        return to_fallback(fb, fs, PolicyReason::PREFERRED_NOT_READY, PolicyStatus::NOT_READY,
                           PolicyReason::PREFERRED_NOT_READY, true);
    }

    // 3. nothing resident
    if (!r.model_loaded)
        return to_fallback(fb, fs, PolicyReason::MODEL_UNAVAILABLE, PolicyStatus::NOT_READY,
                           PolicyReason::MODEL_UNAVAILABLE);
    if (!r.request_within_capability_evidence_scope)
        return to_fallback(fb, fs, PolicyReason::OUTSIDE_VALIDATED_DOMAIN, PolicyStatus::OUTSIDE_VALIDATED_CAPABILITY,
                           PolicyReason::OUTSIDE_EVIDENCE_SCOPE_NO_FALLBACK);
    if (!has_representation(*pref)) {
        if (routable(*pref, ps)) return make(PolicyStatus::OK, pref->id, PolicyReason::DIRECT_PRIMITIVE_READY);
        return to_fallback(fb, fs, PolicyReason::PREFERRED_NOT_READY, PolicyStatus::NOT_READY,
                           PolicyReason::PREFERRED_NOT_READY);
    }
    if (!r.acquisition_allowed)
        return to_fallback(fb, fs, PolicyReason::ACQUISITION_GLOBALLY_VETOED, PolicyStatus::NOT_READY,
                           PolicyReason::MANDATORY_ACQUISITION_UNAVAILABLE);

    // 4. acquisition
    PathChoice best, below;
    bool any_active = false, any_available = false, mandatory = false, mandatory_blocked = false;
    bool amortized = false, reuse_blocked = false, incomplete = false;
    for (std::size_t b = 0; b < registry.bundle_count(); ++b) {
        const registry_v2::RegistrationBundle* bundle = registry.bundle_at(b);
        if (!bundle) continue;
        for (std::size_t i = 0; i < bundle->acquisition_count; ++i) {
            const AcquisitionPathDescriptor& path = bundle->acquisitions[i];
            if (!is_validated(path.state) || path.target_primitive != pref->id) continue;
            any_active = true;
            const bool is_mandatory = path.trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY;
            (is_mandatory ? mandatory : amortized) = true;
            const AcquisitionRuntimeState* as = state_of(r, path.id);
            if (!as || !as->available || as->vetoed) {
                mandatory_blocked |= is_mandatory;
                continue;
            }
            any_available = true;
            const PrimitiveRuntimeState* ts = state_of(r, path.target_primitive);
            if (!ts || !ts->residency_lease_granted) {
                mandatory_blocked |= is_mandatory;
                continue;
            }
            const PrimitiveDescriptor* target = registry.find_primitive(path.target_primitive);
            if (!target || !is_validated(target->state) || target->capability != cap->id) {
                incomplete = true;
                continue;
            }
            if (is_mandatory) {
                keep_best(best, PathChoice{&path, nullptr, target});
                continue;
            }
            if (!prof->reuse_metric) {
                incomplete = true;
                continue;
            }
            if (!r.future_reuse_known || r.future_reuse_units == 0) {
                reuse_blocked = true;
                continue;
            }
            const AcquisitionThresholdDescriptor* th = registry.find_threshold(cap->id, prof->id, path.id);
            if (!th || !is_validated(th->state) || th->reuse_metric != prof->reuse_metric) {
                incomplete = true;
                continue;
            }
            const PathChoice c{&path, th, target};
            keep_best(r.future_reuse_units < th->minimum_reuse_units ? below : best, c);
        }
    }

    if (best.path) {
        PolicyDecision d{};
        d.route = best.target->id;
        d.lifecycle = LifecycleAction::ACQUIRE;
        d.acquisition = best.path->id;
        d.reason = best.path->trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY
                       ? PolicyReason::MANDATORY_ACQUISITION_REQUIRED
                       : PolicyReason::ACQUISITION_THRESHOLD_MET;
        d.threshold_units = best.threshold ? best.threshold->minimum_reuse_units : 0;
        d.requested_residency_bytes = best.target->residency_bytes;
        d.require_post_acquisition_identity_validation =
            (best.target->flags & registry_v2::PRIMITIVE_REQUIRES_IDENTITY_VALIDATION) != 0;
        return d;
    }
    if (incomplete) return unsupported(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    if (fb && routable(*fb, fs)) {
        if (below.path) {
            PolicyDecision d = make(PolicyStatus::OK, fb->id, PolicyReason::BELOW_ALL_ACTIVE_THRESHOLDS);
            d.threshold_units = below.threshold->minimum_reuse_units;
            return d;
        }
        if (reuse_blocked && !r.future_reuse_known)
            return make(PolicyStatus::OK, fb->id, PolicyReason::FUTURE_REUSE_UNKNOWN);
        if (reuse_blocked && r.future_reuse_units == 0)
            return make(PolicyStatus::OK, fb->id, PolicyReason::NO_FUTURE_REUSE);
        return make(PolicyStatus::OK, fb->id, PolicyReason::NO_AVAILABLE_ACQUISITION_PATH);
    }
    (void)any_active;
    (void)any_available;
    if (mandatory || mandatory_blocked)
        return make(PolicyStatus::NOT_READY, {}, PolicyReason::MANDATORY_ACQUISITION_UNAVAILABLE);
    return make(PolicyStatus::NOT_READY, {},
                fb ? PolicyReason::FALLBACK_NOT_READY : PolicyReason::NO_AVAILABLE_ACQUISITION_PATH);
}

}  // namespace arcllm::v1::policy_v4
