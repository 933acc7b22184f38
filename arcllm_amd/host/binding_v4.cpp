// binding_v4.cpp -- BindingState and apply_decision
// (include/arcllm/v1/generic_backend_binding_v4.h).
//
// Observable behaviour of src/arcllm_v1_generic_backend_binding_v4.cpp of the
// reference: a decision is carried out against the backend and never falls
// back by itself; a failing step leaves ready == false with that step's
// status, and a representation acquired in the same call is released again
// (a release that fails is reported as the unreleased representation).
//
// An acquisition runs as a transaction: the ordered steps in kAcquireSteps
// (check, acquire, validate, record, open the route) over one Txn, which
// knows what it holds at every point; the first step that fails ends the
// run, and give_back() returns what the transaction holds.
#include "../../include/arcllm/v1/generic_backend_binding_v4.h"

#include <algorithm>
#include <iterator>

namespace arcllm::v1::binding_v4 {

// -------------------------------------------------------------- the slots
// A slot belongs to the primitive it records; a zero primitive marks it free.
RepresentationHandle BindingState::find(PrimitiveId primitive) const noexcept
{
    const auto hit = std::find_if(std::begin(slots), std::end(slots),
                                  [primitive](const RepresentationSlot& s) { return s.primitive == primitive; });
    return hit == std::end(slots) ? RepresentationHandle{} : hit->representation;
}

// Takes the first slot, in slot order, that records `primitive` or is free:
// a primitive recorded behind a free slot is not updated in place.
bool BindingState::set(PrimitiveId primitive, RepresentationHandle representation) noexcept
{
    const auto hit = std::find_if(std::begin(slots), std::end(slots), [primitive](const RepresentationSlot& s) {
        return s.primitive == primitive || !s.primitive;
    });
    if (hit == std::end(slots)) return false;
    *hit = RepresentationSlot{primitive, representation};
    return true;
}

void BindingState::clear(PrimitiveId primitive) noexcept
{
    const auto hit = std::find_if(std::begin(slots), std::end(slots),
                                  [primitive](const RepresentationSlot& s) { return s.primitive == primitive; });
    if (hit != std::end(slots)) *hit = RepresentationSlot{};
}

namespace {

using policy_v4::LifecycleAction;

// The executable handle of `route` into res (ready on success).  A zero route
// asks for nothing and leaves res untouched.
BackendStatus open_route(PrimitiveId route, BackendAdapter& backend, ApplyResult& res) noexcept
{
    if (!route) return BackendStatus::OK;
    PrimitiveHandle handle{};
    BackendStatus s = backend.resolve_primitive(route, handle);
    if (s == BackendStatus::OK && !handle) s = BackendStatus::PRIMITIVE_UNAVAILABLE;
    res.backend_status = s;
    res.ready = s == BackendStatus::OK;
    if (res.ready) res.primitive = handle;
    return s;
}

// ------------------------------------------------------------ acquisition
struct Txn {
    const PolicyDecision& decision;
    CapabilityId capability;
    PrimitiveId target;  // the capability's preferred primitive
    BackendAdapter& backend;
    BindingState& state;
    ApplyResult& res;
    RepresentationHandle held{};  // acquired in this call
    bool recorded = false;        // held is in the binding state
};

using Step = BackendStatus (*)(Txn&);

const Step kAcquireSteps[] = {
    // the decision acquires for the primitive it routes to
    [](Txn& t) {
        const bool coherent = t.decision.acquisition && t.decision.route == t.target;
        return coherent ? BackendStatus::OK : BackendStatus::INVALID_BINDING_STATE;
    },
    [](Txn& t) {
        RepresentationHandle rep{};
        const BackendStatus s =
            t.backend.acquire(t.decision.acquisition, t.target, t.decision.requested_residency_bytes, rep);
        if (s != BackendStatus::OK) return s;
        t.held = rep;
        return rep ? BackendStatus::OK : BackendStatus::ACQUISITION_FAILED;
    },
    [](Txn& t) {
        if (!t.decision.require_post_acquisition_identity_validation) return BackendStatus::OK;
        return t.backend.validate(t.held, t.capability, t.target);
    },
    [](Txn& t) {
        t.recorded = t.state.set(t.target, t.held);
        return t.recorded ? BackendStatus::OK : BackendStatus::INVALID_BINDING_STATE;
    },
    [](Txn& t) { return open_route(t.decision.route, t.backend, t.res); },
};

// Releases what the transaction holds; a recorded representation leaves the
// binding state once the backend has let it go.
void give_back(Txn& t) noexcept
{
    if (!t.held) return;
    t.res.cleanup_status = t.backend.release(t.target, t.held);
    if (t.res.cleanup_status != BackendStatus::OK)
        t.res.unreleased_representation = t.held;
    else if (t.recorded)
        t.state.clear(t.target);
}

void run_acquisition(Txn& t) noexcept
{
    for (Step step : kAcquireSteps) {
        const BackendStatus s = step(t);
        t.res.backend_status = s;
        if (s != BackendStatus::OK) {
            give_back(t);
            return;
        }
    }
}

// --------------------------------------------------------------- eviction
// The held representation of `target` goes back to the backend before the
// route opens; a failed release keeps it recorded and opens nothing.
void run_eviction(PrimitiveId target, PrimitiveId route, BackendAdapter& backend, BindingState& state,
                  ApplyResult& res) noexcept
{
    if (const RepresentationHandle held = state.find(target)) {
        res.cleanup_status = backend.release(target, held);
        if (res.cleanup_status != BackendStatus::OK) {
            res.backend_status = res.cleanup_status;
            res.unreleased_representation = held;
            return;
        }
        state.clear(target);
    }
    open_route(route, backend, res);
}

}  // namespace

ApplyResult apply_decision(const PrimitiveRegistry& registry, CapabilityId capability, const PolicyDecision& decision,
                           BackendAdapter& backend, BindingState& state) noexcept
{
    ApplyResult res{};
    res.decision = decision;
    const registry_v2::CapabilityDescriptor* cap = registry.find_capability(capability);
    const registry_v2::PrimitiveDescriptor* preferred = cap ? registry.find_primitive(cap->preferred_primitive) : nullptr;
    if (!preferred) {
        res.backend_status = BackendStatus::INVALID_BINDING_STATE;
        return res;
    }
    switch (decision.lifecycle) {
    case LifecycleAction::ACQUIRE: {
        Txn t{decision, capability, preferred->id, backend, state, res};
        run_acquisition(t);
        break;
    }
    case LifecycleAction::EVICT: run_eviction(preferred->id, decision.route, backend, state, res); break;
    default: open_route(decision.route, backend, res); break;
    }
    return res;
}

}  // namespace arcllm::v1::binding_v4
