// q4_down_backend.h -- the gfx950 backend of the Q4_K FFN-down capability
// behind the operator plugin interface (binding_v4::BackendAdapter), and its
// MI355X registration.
//
// Primitive A is the direct packed Q4_K split-K GEMV (route A, nothing
// extra resident).  Primitive B multiplies by an EXEC148 image of every Q4_K
// ffn_down tensor of the model (route B): the image is one device allocation
// ("the family"), acquired through one of three paths --
//   P1 (kAcquirePrimary):   repacked on the GPU from the resident Q4_K tensors
//                           (arc_exec148_materialize, one launch per layer);
//   P3 (kAcquireSecondary): read from a sidecar file holding the family image
//                           (layer images back to back in layer order) and
//                           uploaded;
//   P0 (kAcquireTertiary):  repacked on the host from the GGUF payload and
//                           uploaded;
// validated block by block against the Q4_K source on the GPU
// (arc_exec148_validate), and released on eviction.  The image lives in the
// model's EXEC148 reserve (arc_model_exec148_reserve), planned with the
// model's arena: acquiring fills it and releasing gives it up, and neither
// allocates or frees device memory.  The shape of this class
// follows the reference's Q4VulkanBackendV4
// (src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:196-420): same statuses for
// the same conditions, same counters, one representation with handle 1,
// primitives resolved to handles carrying the primitive id.
#pragma once

#include "../../include/arcllm/v1/generic_backend_binding_v4.h"
#include "../../include/arcllm_hip.h"

#include <array>
#include <cstdint>
#include <string>
#include <vector>

namespace arcllm::v1::hip_q4_down {

namespace reg = registry_v2;
namespace bind = binding_v4;

struct BackendCounters {
    std::uint64_t b_allocations = 0;
    std::uint64_t b_materializations = 0;
    std::uint64_t b_validations = 0;
    std::uint64_t b_releases = 0;
    std::uint64_t p1_calls = 0;
    std::uint64_t p3_calls = 0;
    std::uint64_t p0_calls = 0;
    std::uint64_t resolve_a = 0;
    std::uint64_t resolve_b = 0;
};

/* Bytes of the EXEC148 image of one rows x K Q4_K tensor. */
std::uint64_t exec148_bytes(std::uint32_t rows, std::uint32_t K);

/* Host repack of a rows x K Q4_K tensor into EXEC148 (the P0 path), over up to
 * `threads` threads. */
void exec148_repack_host(const std::uint8_t* q4, std::uint32_t rows, std::uint32_t K, std::uint8_t* exec,
                         unsigned threads);

/* The Q4_K FFN-down registration of the gfx950 backend: the reference's ids
 * (capability, primitives, paths, profiles), primitive B's residency set to
 * this model's family bytes, and the reuse thresholds measured on MI355X
 * (future decode tokens from which each acquisition path pays for itself).
 * Holds the descriptor arrays the bundle points into; keep it alive while a
 * registry uses the bundle. */
class Mi355xRegistration {
public:
    explicit Mi355xRegistration(std::uint64_t family_bytes);
    Mi355xRegistration(const Mi355xRegistration&) = delete;
    Mi355xRegistration& operator=(const Mi355xRegistration&) = delete;
    const reg::RegistrationBundle& bundle() const noexcept { return bundle_; }

    /* measured reuse thresholds: {P1, P3, P0} for profile 0, then profile 1 */
    static const std::array<std::uint64_t, 6>& thresholds() noexcept;

private:
    reg::PrimitiveDescriptor primitives_[2];
    reg::RegistrationBundle bundle_{};
};

class HipQ4DownBackend final : public bind::BackendAdapter {
public:
    /* `layers`: the model's layers whose ffn_down is Q4_K (rows x K each);
     * `host_src[i]`: that layer's packed tensor in host memory (the P0
     * source); the device copies come from `model`. */
    HipQ4DownBackend(arc_model* model, std::vector<std::uint32_t> layers, std::vector<const std::uint8_t*> host_src,
                     std::uint32_t rows, std::uint32_t K, std::string sidecar);
    ~HipQ4DownBackend() override;
    HipQ4DownBackend(const HipQ4DownBackend&) = delete;
    HipQ4DownBackend& operator=(const HipQ4DownBackend&) = delete;

    bind::BackendStatus acquire(reg::AcquisitionPathId path, reg::PrimitiveId target, std::uint64_t residency_bytes,
                                bind::RepresentationHandle& out) noexcept override;
    bind::BackendStatus validate(bind::RepresentationHandle representation, reg::CapabilityId capability,
                                 reg::PrimitiveId target) noexcept override;
    bind::BackendStatus release(reg::PrimitiveId target, bind::RepresentationHandle representation) noexcept override;
    bind::BackendStatus resolve_primitive(reg::PrimitiveId primitive, bind::PrimitiveHandle& out) noexcept override;

    /* Routes every Q4_K ffn_down of `session` to `primitive` (A: the packed
     * tensors; B: this backend's image, which must be resident and
     * validated) from its next decode call on; the session must stay
     * attached until it is destroyed or routed back to A.  Returns false with
     * last_error() set when the route cannot be taken. */
    bool route(arc_session* session, bind::PrimitiveHandle primitive) noexcept;

    bool resident() const noexcept { return resident_; }
    bool validated() const noexcept { return validated_; }
    bool p3_available() const noexcept;
    std::uint64_t family_bytes() const noexcept { return family_bytes_; }
    /* the device image while resident: layer i's EXEC148 bytes (layer_bytes())
     * at device_image() + i * slot_stride() */
    const std::uint8_t* device_image() const noexcept { return exec_; }
    std::uint64_t layer_bytes() const noexcept { return layer_bytes_; }
    std::uint64_t slot_stride() const noexcept { return slot_stride_; }
    const std::vector<std::uint32_t>& layers() const noexcept { return layers_; }
    const BackendCounters& counters() const noexcept { return counters_; }
    std::uint64_t last_mismatched_blocks() const noexcept { return last_mismatched_; }
    const std::string& last_error() const noexcept { return last_error_; }

private:
    bool acquire_p1();
    bool acquire_p3();
    bool acquire_p0();
    bool unroute() noexcept;
    void drop() noexcept;

    arc_model* model_;
    std::vector<std::uint32_t> layers_;
    std::vector<const std::uint8_t*> host_src_;
    std::uint32_t rows_, K_;
    std::string sidecar_;
    std::uint64_t layer_bytes_ = 0;   // one layer's image
    std::uint64_t slot_stride_ = 0;   // its offset step in the model's EXEC148 reserve
    std::uint64_t family_bytes_ = 0;  // layers x layer_bytes (the residency and sidecar size)
    std::uint8_t* reserve_ = nullptr; // the model's EXEC148 reserve (null: none)
    std::uint32_t reserve_slots_ = 0;
    std::uint8_t* exec_ = nullptr;    // device image while resident (= reserve_)
    arc_session* routed_ = nullptr;   // session currently routed to the image
    bool resident_ = false;
    bool validated_ = false;
    BackendCounters counters_{};
    std::uint64_t last_mismatched_ = 0;
    std::string last_error_;
};

}  // namespace arcllm::v1::hip_q4_down
