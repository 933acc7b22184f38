// policy_v4.cpp -- policy_v4::evaluate (include/arcllm/v1/generic_policy_engine_v4.h).
//
// Decides the same cases, with the same status, route, reason and lifecycle
// action, as src/arcllm_v1_generic_policy_engine_v4.cpp of the reference.
// The procedure is four ordered tables run over a Scene (the request with
// everything it names looked up):
//  kGates         admission: each gate looks up one thing the request names
//                 and refuses with its own status when it is missing,
//                 unvalidated or inconsistent;
//  kEvictions     a resident representation of the preferred primitive: the
//                 first armed lifecycle rule whose condition holds evicts it;
//  kLadder        no residency: the first rung whose condition holds sends
//                 the request to the preferred primitive or the fallback;
//  acquisition    every validated path to the preferred primitive is graded
//                 (grade_path) and the grades are folded into a Survey, from
//                 which the decision and, failing that, the reason are read.
// A primitive "can run" when its execution is available and ready and, if it
// needs an acquired representation, that representation is resident,
// identity-valid and leased.
#include "../../include/arcllm/v1/generic_policy_engine_v4.h"

namespace arcllm::v1::policy_v4 {

namespace {

using registry_v2::AcquisitionPathDescriptor;
using registry_v2::AcquisitionThresholdDescriptor;
using registry_v2::AcquisitionTrigger;
using registry_v2::CapabilityDescriptor;
using registry_v2::EvidenceProfileDescriptor;
using registry_v2::LifecycleDescriptor;
using registry_v2::PrimitiveDescriptor;
using registry_v2::ValidationState;

bool validated(ValidationState s) noexcept { return s == ValidationState::VALIDATED; }

bool needs_representation(const PrimitiveDescriptor& p) noexcept
{
    return (p.flags & registry_v2::PRIMITIVE_REQUIRES_RESIDENCY) != 0;
}

bool can_run(const PrimitiveDescriptor& p, const PrimitiveRuntimeState* rt) noexcept
{
    if (!rt || !rt->execution_available || !rt->execution_ready) return false;
    return !needs_representation(p) || (rt->resident && rt->identity_valid && rt->residency_lease_granted);
}

// Runtime rows are keyed by the id member `Key`.
template <typename Row, typename Id, Id Row::*Key>
bool keys_distinct(const Row* rows, std::size_t n) noexcept
{
    if (n != 0 && rows == nullptr) return false;
    for (std::size_t i = 0; i < n; ++i) {
        if (!(rows[i].*Key)) return false;
        for (std::size_t j = i + 1; j < n; ++j)
            if (rows[j].*Key == rows[i].*Key) return false;
    }
    return true;
}

template <typename Row, typename Id, Id Row::*Key>
const Row* row_with(const Row* rows, std::size_t n, Id id) noexcept
{
    for (std::size_t i = 0; i < n; ++i)
        if (rows[i].*Key == id) return &rows[i];
    return nullptr;
}

// ------------------------------------------------------------------ scene
struct Scene {
    const PrimitiveRegistry& reg;
    const PolicyRequest& req;
    const CapabilityDescriptor* cap = nullptr;
    const EvidenceProfileDescriptor* profile = nullptr;
    const PrimitiveDescriptor* preferred = nullptr;
    const PrimitiveDescriptor* fallback = nullptr;  // null: the capability has none
    const LifecycleDescriptor* lifecycle = nullptr;
    const PrimitiveRuntimeState* preferred_rt = nullptr;
    const PrimitiveRuntimeState* fallback_rt = nullptr;

    const PrimitiveRuntimeState* runtime(PrimitiveId id) const noexcept
    {
        return row_with<PrimitiveRuntimeState, PrimitiveId, &PrimitiveRuntimeState::primitive>(
            req.primitive_states, req.primitive_state_count, id);
    }
    const AcquisitionRuntimeState* runtime(AcquisitionPathId id) const noexcept
    {
        return row_with<AcquisitionRuntimeState, AcquisitionPathId, &AcquisitionRuntimeState::acquisition>(
            req.acquisition_states, req.acquisition_state_count, id);
    }
    bool fallback_can_run() const noexcept { return fallback && can_run(*fallback, fallback_rt); }
};

// A primitive of the capability that is validated.
bool usable_member(const Scene& s, const PrimitiveDescriptor* p) noexcept
{
    return p && validated(p->state) && p->capability == s.cap->id;
}

// ------------------------------------------------------------- decisions
PolicyDecision refusal(PolicyStatus status) noexcept
{
    PolicyDecision d{};
    d.status = status;
    d.reason = PolicyReason::UNSUPPORTED_REQUEST;
    return d;
}

PolicyDecision route_to(PrimitiveId route, PolicyReason reason, bool preserve = false) noexcept
{
    PolicyDecision d{};
    d.route = route;
    d.reason = reason;
    d.preserve_existing_representation = preserve;
    return d;
}

PolicyDecision no_route(PolicyStatus status, PolicyReason reason, bool preserve = false) noexcept
{
    PolicyDecision d{};
    d.status = status;
    d.reason = reason;
    d.preserve_existing_representation = preserve;
    return d;
}

// The request goes to the fallback, for `why`; when the fallback cannot run
// there is no route: FALLBACK_NOT_READY, or `orphan` when there is no fallback.
struct Detour {
    PolicyReason why;
    PolicyStatus stuck;
    PolicyReason orphan;
};

PolicyDecision take(const Scene& s, const Detour& d, bool preserve = false) noexcept
{
    if (s.fallback_can_run()) return route_to(s.fallback->id, d.why, preserve);
    return no_route(d.stuck, s.fallback ? PolicyReason::FALLBACK_NOT_READY : d.orphan, preserve);
}

constexpr Detour kOutOfScope{PolicyReason::OUTSIDE_VALIDATED_DOMAIN, PolicyStatus::OUTSIDE_VALIDATED_CAPABILITY,
                             PolicyReason::OUTSIDE_EVIDENCE_SCOPE_NO_FALLBACK};
constexpr Detour kPreferredIdle{PolicyReason::PREFERRED_NOT_READY, PolicyStatus::NOT_READY,
                                PolicyReason::PREFERRED_NOT_READY};

// ------------------------------------------------------------------- gates
struct Gate {
    bool (*admit)(Scene&);
    PolicyStatus refused_as;
};

const Gate kGates[] = {
    {[](Scene& s) {
         return keys_distinct<PrimitiveRuntimeState, PrimitiveId, &PrimitiveRuntimeState::primitive>(
                    s.req.primitive_states, s.req.primitive_state_count) &&
                keys_distinct<AcquisitionRuntimeState, AcquisitionPathId, &AcquisitionRuntimeState::acquisition>(
                    s.req.acquisition_states, s.req.acquisition_state_count);
     },
     PolicyStatus::INVALID_RUNTIME_STATE},
    {[](Scene& s) {
         s.cap = s.reg.find_capability(s.req.capability);
         return s.cap && validated(s.cap->state);
     },
     PolicyStatus::UNSUPPORTED_CAPABILITY},
    {[](Scene& s) {
         s.profile = s.reg.find_profile(s.req.profile);
         return s.profile && validated(s.profile->state);
     },
     PolicyStatus::UNSUPPORTED_PROFILE},
    {[](Scene& s) { return s.profile->domain == s.cap->domain; }, PolicyStatus::PROFILE_DOMAIN_MISMATCH},
    {[](Scene& s) {
         const auto* domain = s.reg.find_domain(s.cap->domain);
         const auto* evidence = s.reg.find_evidence_set(s.profile->evidence_set);
         return domain && evidence && validated(domain->state) && validated(evidence->state);
     },
     PolicyStatus::REGISTRY_POLICY_INCOMPLETE},
    {[](Scene& s) {
         if (!s.profile->reuse_metric) return true;
         const auto* metric = s.reg.find_reuse_metric(s.profile->reuse_metric);
         return metric && validated(metric->state);
     },
     PolicyStatus::REGISTRY_POLICY_INCOMPLETE},
    {[](Scene& s) {
         s.preferred = s.reg.find_primitive(s.cap->preferred_primitive);
         s.preferred_rt = s.preferred ? s.runtime(s.preferred->id) : nullptr;
         return usable_member(s, s.preferred);
     },
     PolicyStatus::REGISTRY_POLICY_INCOMPLETE},
    {[](Scene& s) {
         if (!s.cap->fallback_primitive) return true;
         s.fallback = s.reg.find_primitive(s.cap->fallback_primitive);
         s.fallback_rt = s.fallback ? s.runtime(s.fallback->id) : nullptr;
         return usable_member(s, s.fallback);
     },
     PolicyStatus::REGISTRY_POLICY_INCOMPLETE},
    {[](Scene& s) {
         s.lifecycle = s.reg.find_lifecycle(s.preferred->id);
         return s.lifecycle || !needs_representation(*s.preferred);
     },
     PolicyStatus::REGISTRY_POLICY_INCOMPLETE},
};

// --------------------------------------------------------------- residency
struct EvictionRule {
    bool LifecycleDescriptor::*armed;
    bool (*holds)(const Scene&);
    PolicyReason reason;
};

const EvictionRule kEvictions[] = {
    {&LifecycleDescriptor::evict_on_model_unload, [](const Scene& s) { return !s.req.model_loaded; },
     PolicyReason::MODEL_UNAVAILABLE},
    {&LifecycleDescriptor::evict_on_identity_invalid, [](const Scene& s) { return !s.preferred_rt->identity_valid; },
     PolicyReason::RESIDENT_PRIMITIVE_INVALID},
    {&LifecycleDescriptor::evict_on_execution_unavailable,
     [](const Scene& s) { return !s.preferred_rt->execution_available; }, PolicyReason::RESIDENT_EXECUTION_UNAVAILABLE},
    {&LifecycleDescriptor::evict_on_lease_revoke,
     [](const Scene& s) { return !s.preferred_rt->residency_lease_granted; }, PolicyReason::RESIDENCY_LEASE_REVOKED},
    {&LifecycleDescriptor::evict_on_zero_future_reuse,
     [](const Scene& s) { return s.req.future_reuse_known && s.req.future_reuse_units == 0; },
     PolicyReason::NO_FUTURE_REUSE},
};

PolicyDecision with_resident(const Scene& s) noexcept
{
    for (const EvictionRule& rule : kEvictions)
        if (s.lifecycle->*rule.armed && rule.holds(s)) {
            PolicyDecision d = take(s, Detour{rule.reason, PolicyStatus::NOT_READY, rule.reason});
            d.lifecycle = LifecycleAction::EVICT;
            return d;
        }
    if (!s.req.request_within_capability_evidence_scope)
        return take(s, kOutOfScope, s.lifecycle->preserve_residency_outside_domain);
    if (can_run(*s.preferred, s.preferred_rt))
        return route_to(s.preferred->id, PolicyReason::RESIDENT_PRIMITIVE_REUSED, true);
    return take(s, kPreferredIdle, true);
}

// ------------------------------------------------------------------ ladder
// A rung applies when `applies` holds; it routes to the preferred primitive
// (for `direct`) when `direct_ok` and the preferred primitive can run, and
// otherwise takes its detour.
struct Rung {
    bool (*applies)(const Scene&);
    bool direct_ok;
    PolicyReason direct;
    Detour detour;
};

const Rung kLadder[] = {
    {[](const Scene& s) { return !s.req.model_loaded; }, false, {},
     Detour{PolicyReason::MODEL_UNAVAILABLE, PolicyStatus::NOT_READY, PolicyReason::MODEL_UNAVAILABLE}},
    {[](const Scene& s) { return !s.req.request_within_capability_evidence_scope; }, false, {}, kOutOfScope},
    {[](const Scene& s) { return !needs_representation(*s.preferred); }, true, PolicyReason::DIRECT_PRIMITIVE_READY,
     kPreferredIdle},
    {[](const Scene& s) { return !s.req.acquisition_allowed; }, false, {},
     Detour{PolicyReason::ACQUISITION_GLOBALLY_VETOED, PolicyStatus::NOT_READY,
            PolicyReason::MANDATORY_ACQUISITION_UNAVAILABLE}},
};

// ------------------------------------------------------------- acquisition
enum class Grade {
    NOT_A_CANDIDATE,  // unvalidated, or acquires some other primitive
    BLOCKED,          // unavailable, vetoed, or the target holds no lease
    MISCONFIGURED,    // the registry lacks what an amortized path needs
    REUSE_UNSURE,     // future reuse unknown or zero
    SHORT,            // amortized, reuse below its threshold
    QUALIFIES
};

Grade grade_path(const Scene& s, const AcquisitionPathDescriptor& p, const AcquisitionThresholdDescriptor*& bar) noexcept
{
    bar = nullptr;
    if (!validated(p.state) || p.target_primitive != s.preferred->id) return Grade::NOT_A_CANDIDATE;
    const AcquisitionRuntimeState* rt = s.runtime(p.id);
    if (!rt || !rt->available || rt->vetoed) return Grade::BLOCKED;
    // the path's target is the preferred primitive, admitted by the gates
    if (!s.preferred_rt || !s.preferred_rt->residency_lease_granted) return Grade::BLOCKED;
    if (p.trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY) return Grade::QUALIFIES;
    if (!s.profile->reuse_metric) return Grade::MISCONFIGURED;
    if (!s.req.future_reuse_known || s.req.future_reuse_units == 0) return Grade::REUSE_UNSURE;
    bar = s.reg.find_threshold(s.cap->id, s.profile->id, p.id);
    if (!bar || !validated(bar->state) || bar->reuse_metric != s.profile->reuse_metric) return Grade::MISCONFIGURED;
    return s.req.future_reuse_units < bar->minimum_reuse_units ? Grade::SHORT : Grade::QUALIFIES;
}

struct Pick {
    const AcquisitionPathDescriptor* path = nullptr;
    const AcquisitionThresholdDescriptor* bar = nullptr;

    // lower priority first, then lower id
    void offer(const AcquisitionPathDescriptor& p, const AcquisitionThresholdDescriptor* b) noexcept
    {
        const bool first = !path || p.priority < path->priority ||
                           (p.priority == path->priority && p.id.value < path->id.value);
        if (first) {
            path = &p;
            bar = b;
        }
    }
};

struct Survey {
    Pick winner, nearest_short;
    bool mandatory_targets = false;  // a validated mandatory path acquires the preferred primitive
    bool misconfigured = false;
    bool reuse_unsure = false;
};

Survey survey_paths(const Scene& s) noexcept
{
    Survey v;
    for (std::size_t b = 0; b < s.reg.bundle_count(); ++b) {
        const registry_v2::RegistrationBundle* bundle = s.reg.bundle_at(b);
        for (std::size_t i = 0; bundle && i < bundle->acquisition_count; ++i) {
            const AcquisitionPathDescriptor& p = bundle->acquisitions[i];
            const AcquisitionThresholdDescriptor* bar = nullptr;
            const Grade g = grade_path(s, p, bar);
            if (g == Grade::NOT_A_CANDIDATE) continue;
            v.mandatory_targets |= p.trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY;
            switch (g) {
            case Grade::QUALIFIES: v.winner.offer(p, bar); break;
            case Grade::SHORT: v.nearest_short.offer(p, bar); break;
            case Grade::MISCONFIGURED: v.misconfigured = true; break;
            case Grade::REUSE_UNSURE: v.reuse_unsure = true; break;
            default: break;
            }
        }
    }
    return v;
}

PolicyDecision acquire_or_explain(const Scene& s) noexcept
{
    const Survey v = survey_paths(s);
    if (const AcquisitionPathDescriptor* p = v.winner.path) {
        const PrimitiveDescriptor& target = *s.preferred;
        PolicyDecision d = route_to(target.id, p->trigger == AcquisitionTrigger::MANDATORY_FOR_FEASIBILITY
                                                   ? PolicyReason::MANDATORY_ACQUISITION_REQUIRED
                                                   : PolicyReason::ACQUISITION_THRESHOLD_MET);
        d.lifecycle = LifecycleAction::ACQUIRE;
        d.acquisition = p->id;
        d.threshold_units = v.winner.bar ? v.winner.bar->minimum_reuse_units : 0;
        d.requested_residency_bytes = target.residency_bytes;
        d.require_post_acquisition_identity_validation =
            (target.flags & registry_v2::PRIMITIVE_REQUIRES_IDENTITY_VALIDATION) != 0;
        return d;
    }
    if (v.misconfigured) return refusal(PolicyStatus::REGISTRY_POLICY_INCOMPLETE);
    if (s.fallback_can_run()) {
        PolicyDecision d = route_to(s.fallback->id, PolicyReason::NO_AVAILABLE_ACQUISITION_PATH);
        if (v.nearest_short.path) {
            d.reason = PolicyReason::BELOW_ALL_ACTIVE_THRESHOLDS;
            d.threshold_units = v.nearest_short.bar->minimum_reuse_units;
        } else if (v.reuse_unsure) {
            d.reason = s.req.future_reuse_known ? PolicyReason::NO_FUTURE_REUSE : PolicyReason::FUTURE_REUSE_UNKNOWN;
        }
        return d;
    }
    if (v.mandatory_targets) return no_route(PolicyStatus::NOT_READY, PolicyReason::MANDATORY_ACQUISITION_UNAVAILABLE);
    return no_route(PolicyStatus::NOT_READY,
                    s.fallback ? PolicyReason::FALLBACK_NOT_READY : PolicyReason::NO_AVAILABLE_ACQUISITION_PATH);
}

}  // namespace

PolicyDecision evaluate(const PrimitiveRegistry& registry, const PolicyRequest& request) noexcept
{
    Scene s{registry, request};
    for (const Gate& g : kGates)
        if (!g.admit(s)) return refusal(g.refused_as);

    if (s.preferred_rt && s.preferred_rt->resident && needs_representation(*s.preferred)) return with_resident(s);

    for (const Rung& rung : kLadder) {
        if (!rung.applies(s)) continue;
        if (rung.direct_ok && can_run(*s.preferred, s.preferred_rt)) return route_to(s.preferred->id, rung.direct);
        return take(s, rung.detour);
    }
    return acquire_or_explain(s);
}

}  // namespace arcllm::v1::policy_v4
