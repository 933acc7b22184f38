// binding_v4.cpp -- BindingState and apply_decision
// (include/arcllm/v1/generic_backend_binding_v4.h).
//
// Behaviour of src/arcllm_v1_generic_backend_binding_v4.cpp of the reference:
// a decision is carried out against the backend without ever falling back on
// its own -- any failing step leaves ready == false with the failing status,
// and whatever was acquired in this call is released again (a release that
// fails is reported as the unreleased representation).
#include "../../include/arcllm/v1/generic_backend_binding_v4.h"

namespace arcllm::v1::binding_v4 {

RepresentationHandle BindingState::find(PrimitiveId primitive) const noexcept
{
    for (const RepresentationSlot& s : slots)
        if (s.primitive == primitive) return s.representation;
    return {};
}

// Writes the first slot that holds `primitive` or is free.
bool BindingState::set(PrimitiveId primitive, RepresentationHandle representation) noexcept
{
    for (RepresentationSlot& s : slots)
        if (s.primitive == primitive || !s.primitive) {
            s.primitive = primitive;
            s.representation = representation;
            return true;
        }
    return false;
}

void BindingState::clear(PrimitiveId primitive) noexcept
{
    for (RepresentationSlot& s : slots)
        if (s.primitive == primitive) {
            s = RepresentationSlot{};
            return;
        }
}

namespace {

// Resolves `route` (nothing to do for a zero route) into res.primitive.
BackendStatus resolve(PrimitiveId route, BackendAdapter& backend, ApplyResult& res) noexcept
{
    if (!route) return BackendStatus::OK;
    PrimitiveHandle h{};
    BackendStatus s = backend.resolve_primitive(route, h);
    if (s == BackendStatus::OK && !h) s = BackendStatus::PRIMITIVE_UNAVAILABLE;
    res.backend_status = s;
    if (s == BackendStatus::OK) {
        res.primitive = h;
        res.ready = true;
    }
    return s;
}

// Releases `rep` of `target` after a failed step of an acquisition.
void undo(BackendAdapter& backend, PrimitiveId target, RepresentationHandle rep, ApplyResult& res) noexcept
{
    res.cleanup_status = backend.release(target, rep);
    if (res.cleanup_status != BackendStatus::OK) res.unreleased_representation = rep;
}

}  // namespace

ApplyResult apply_decision(const PrimitiveRegistry& registry, CapabilityId capability, const PolicyDecision& decision,
                           BackendAdapter& backend, BindingState& state) noexcept
{
    ApplyResult res{};
    res.decision = decision;
    const registry_v2::CapabilityDescriptor* cap = registry.find_capability(capability);
    const registry_v2::PrimitiveDescriptor* pref = cap ? registry.find_primitive(cap->preferred_primitive) : nullptr;
    if (!pref) {
        res.backend_status = BackendStatus::INVALID_BINDING_STATE;
        return res;
    }

    if (decision.lifecycle == policy_v4::LifecycleAction::EVICT) {
        const RepresentationHandle held = state.find(pref->id);
        if (held) {
            res.cleanup_status = backend.release(pref->id, held);
            if (res.cleanup_status != BackendStatus::OK) {
                res.backend_status = res.cleanup_status;
                res.unreleased_representation = held;
                return res;
            }
            state.clear(pref->id);
        }
        resolve(decision.route, backend, res);
        return res;
    }

    if (decision.lifecycle == policy_v4::LifecycleAction::ACQUIRE) {
        if (!decision.acquisition || decision.route != pref->id) {
            res.backend_status = BackendStatus::INVALID_BINDING_STATE;
            return res;
        }
        RepresentationHandle rep{};
        BackendStatus s = backend.acquire(decision.acquisition, pref->id, decision.requested_residency_bytes, rep);
        if (s == BackendStatus::OK && !rep) s = BackendStatus::ACQUISITION_FAILED;
        res.backend_status = s;
        if (s != BackendStatus::OK) return res;
        if (decision.require_post_acquisition_identity_validation) {
            res.backend_status = backend.validate(rep, capability, pref->id);
            if (res.backend_status != BackendStatus::OK) {
                undo(backend, pref->id, rep, res);
                return res;
            }
        }
        if (!state.set(pref->id, rep)) {
            res.backend_status = BackendStatus::INVALID_BINDING_STATE;
            undo(backend, pref->id, rep, res);
            return res;
        }
        if (resolve(decision.route, backend, res) != BackendStatus::OK) {
            const RepresentationHandle held = state.find(pref->id);
            if (held) {
                undo(backend, pref->id, held, res);
                if (res.cleanup_status == BackendStatus::OK) state.clear(pref->id);
            }
        }
        return res;
    }

    resolve(decision.route, backend, res);
    return res;
}

}  // namespace arcllm::v1::binding_v4
