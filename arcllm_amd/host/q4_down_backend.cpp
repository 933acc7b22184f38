// q4_down_backend.cpp -- HipQ4DownBackend, its MI355X registration and the
// host EXEC148 repack (the P0 path).
#include "q4_down_backend.h"

#include "registrations/arcllm_v1_q4k_down_reference_registration_v2.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <memory>
#include <thread>

namespace arcllm::v1::hip_q4_down {

namespace q4reg = reference_registration_v2;

namespace {

constexpr std::uint32_t kQK = 256;          // elements per block
constexpr std::uint32_t kQ4Block = 144;     // Q4_K block bytes
constexpr std::uint32_t kE148Block = 148;   // EXEC148 block bytes

// One Q4_K block -> one EXEC148 block: d and dmin bytes as they are, the
// eight 6-bit (scale, min) pairs unpacked to a byte each, then the 256 codes
// two per byte in element order (element 2p in the low nibble of byte p).
// Q4_K stores group g (64 elements) as 32 bytes whose low nibbles are
// elements 0..31 and high nibbles 32..63 of the group.
void repack_block(const std::uint8_t* q, std::uint8_t* e)
{
    std::memcpy(e, q, 4);
    const std::uint8_t* s = q + 4;
    for (std::uint32_t j = 0; j < 8; ++j) {
        std::uint8_t sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = std::uint8_t((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
            mn = std::uint8_t((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
        e[4 + 2 * j] = sc;
        e[5 + 2 * j] = mn;
    }
    const std::uint8_t* qs = q + 16;
    std::uint8_t* c = e + 20;
    for (std::uint32_t g = 0; g < 4; ++g) {
        const std::uint8_t* b = qs + 32 * g;
        for (std::uint32_t i = 0; i < 16; ++i) {  // elements 2i, 2i+1 of the low half
            c[32 * g + i] = std::uint8_t((b[2 * i] & 15) | ((b[2 * i + 1] & 15) << 4));
            c[32 * g + 16 + i] = std::uint8_t((b[2 * i] >> 4) | (b[2 * i + 1] & 0xf0));
        }
    }
}

}  // namespace

std::uint64_t exec148_bytes(std::uint32_t rows, std::uint32_t K)
{
    return std::uint64_t(rows) * (K / kQK) * kE148Block;
}

void exec148_repack_host(const std::uint8_t* q4, std::uint32_t rows, std::uint32_t K, std::uint8_t* exec,
                         unsigned threads)
{
    const std::uint64_t nb = std::uint64_t(rows) * (K / kQK);
    threads = std::max(1u, std::min<unsigned>(threads, unsigned((nb + 4095) / 4096)));
    auto run = [&](std::uint64_t b0, std::uint64_t b1) {
        for (std::uint64_t b = b0; b < b1; ++b) repack_block(q4 + b * kQ4Block, exec + b * kE148Block);
    };
    if (threads == 1) return run(0, nb);
    std::vector<std::thread> pool;
    pool.reserve(threads);
    for (unsigned t = 0; t < threads; ++t) pool.emplace_back(run, nb * t / threads, nb * (t + 1) / threads);
    for (std::thread& th : pool) th.join();
}

// ------------------------------------------------------------ registration

namespace {

// Future decode tokens from which each path pays for itself on MI355X,
// measured with arcllm_q4_paths on the Qwen2.5-7B shape with the 14 Q4_K
// ffn_down layers of its Q4_K_M file (family image 549,527,552 bytes):
//   saving per decode token, route B over route A: 12.1 us (28-layer step,
//     1.603 -> 1.591 ms at context 512);
//   P1: allocation + GPU repack 0.89 ms, GPU validation 0.39 ms -> 106;
//   P3: sidecar read (page cache dropped) + upload ~100 ms + validation -> 8355;
//   P0: host repack (16 threads) + upload ~65 ms + validation -> 5392;
// threshold = ceil(cost / saving).  Profile 1 doubles profile 0, as the
// reference's conservative profile roughly does (src/registrations/
// arcllm_v1_q4k_down_reference_registration_v2.cpp:39-46: 2/4, 15/33, 17/37).
constexpr std::array<std::uint64_t, 6> kThresholds = {106, 8355, 5392, 212, 16710, 10784};

constexpr reg::ProvenanceRef kMeasured{"profiles/q4_down_routes_mi355x.md", nullptr};
constexpr auto V = reg::ValidationState::VALIDATED;
constexpr auto AMORT = reg::AcquisitionTrigger::REUSE_AMORTIZED;

constexpr reg::DomainDescriptor kDomains[] = {{q4reg::kDomain, V, "Q4K_DECODE_FFN_DOWN_GFX950", kMeasured}};
constexpr reg::ReuseMetricDescriptor kMetrics[] = {{q4reg::kReuseMetric, V, "FUTURE_REUSE_TOKENS", kMeasured}};
constexpr reg::EvidenceSetDescriptor kEvidence[] = {{q4reg::kEvidenceSet, V, "MI355X_ROUTE_AND_ACQUISITION_TIMING", kMeasured}};
constexpr reg::EvidenceProfileDescriptor kProfiles[] = {
    {q4reg::kProfile0, q4reg::kDomain, q4reg::kReuseMetric, q4reg::kEvidenceSet, V, "PROFILE_0", kMeasured},
    {q4reg::kProfile1, q4reg::kDomain, q4reg::kReuseMetric, q4reg::kEvidenceSet, V, "PROFILE_1", kMeasured}};
constexpr reg::PrimitiveFamilyDescriptor kFamilies[] = {{q4reg::kFamily, q4reg::kDomain, V, "Q4K_DOWN_GFX950", kMeasured}};
constexpr reg::CapabilityDescriptor kCapabilities[] = {
    {q4reg::kCapability, q4reg::kDomain, q4reg::kPrimitiveB, q4reg::kPrimitiveA, V, "Q4K_DECODE_FFN_DOWN", kMeasured}};
constexpr reg::AcquisitionPathDescriptor kPaths[] = {
    {q4reg::kAcquirePrimary, q4reg::kPrimitiveB, 0u, AMORT, V, "P1_GPU_REPACK", kMeasured},
    {q4reg::kAcquireSecondary, q4reg::kPrimitiveB, 1u, AMORT, V, "P3_SIDECAR_UPLOAD", kMeasured},
    {q4reg::kAcquireTertiary, q4reg::kPrimitiveB, 2u, AMORT, V, "P0_HOST_REPACK_UPLOAD", kMeasured},
    {q4reg::kAcquireDisabledWarm, q4reg::kPrimitiveB, 3u, AMORT, reg::ValidationState::DISABLED_BY_EVIDENCE,
     "P3_WARM_PAGE_CACHE", kMeasured}};
constexpr reg::AcquisitionThresholdDescriptor kThresholdRows[] = {
    {q4reg::kCapability, q4reg::kProfile0, q4reg::kAcquirePrimary, q4reg::kReuseMetric, kThresholds[0], V, kMeasured},
    {q4reg::kCapability, q4reg::kProfile0, q4reg::kAcquireSecondary, q4reg::kReuseMetric, kThresholds[1], V, kMeasured},
    {q4reg::kCapability, q4reg::kProfile0, q4reg::kAcquireTertiary, q4reg::kReuseMetric, kThresholds[2], V, kMeasured},
    {q4reg::kCapability, q4reg::kProfile1, q4reg::kAcquirePrimary, q4reg::kReuseMetric, kThresholds[3], V, kMeasured},
    {q4reg::kCapability, q4reg::kProfile1, q4reg::kAcquireSecondary, q4reg::kReuseMetric, kThresholds[4], V, kMeasured},
    {q4reg::kCapability, q4reg::kProfile1, q4reg::kAcquireTertiary, q4reg::kReuseMetric, kThresholds[5], V, kMeasured}};
constexpr reg::LifecycleDescriptor kLifecycles[] = {{q4reg::kPrimitiveB, true, true, true, true, true, true, kMeasured}};

}  // namespace

const std::array<std::uint64_t, 6>& Mi355xRegistration::thresholds() noexcept { return kThresholds; }

Mi355xRegistration::Mi355xRegistration(std::uint64_t family_bytes)
    : primitives_{{q4reg::kPrimitiveA, q4reg::kFamily, q4reg::kCapability, {}, 0,
                   reg::PRIMITIVE_FALLBACK | reg::PRIMITIVE_NO_EXTRA_REPRESENTATION, V, "A_Q4K_SPLITK", kMeasured},
                  {q4reg::kPrimitiveB, q4reg::kFamily, q4reg::kCapability, q4reg::kRepresentationB, family_bytes,
                   reg::PRIMITIVE_REQUIRES_RESIDENCY | reg::PRIMITIVE_REQUIRES_IDENTITY_VALIDATION, V,
                   "B_EXEC148_SPLITK", kMeasured}}
{
    bundle_ = reg::RegistrationBundle{"Q4K_DOWN_GFX950_REGISTRATION_V2",
                                      kDomains, 1, kMetrics, 1, kEvidence, 1, kProfiles, 2, kFamilies, 1,
                                      kCapabilities, 1, primitives_, 2, kPaths, 4, kThresholdRows, 6, kLifecycles, 1};
}

// ------------------------------------------------------------ backend

HipQ4DownBackend::HipQ4DownBackend(arc_model* model, std::vector<std::uint32_t> layers,
                                   std::vector<const std::uint8_t*> host_src, std::uint32_t rows, std::uint32_t K,
                                   std::string sidecar)
    : model_(model), layers_(std::move(layers)), host_src_(std::move(host_src)), rows_(rows), K_(K),
      sidecar_(std::move(sidecar))
{
    layer_bytes_ = exec148_bytes(rows_, K_);
    family_bytes_ = layer_bytes_ * layers_.size();
    void* base = nullptr;
    if (arc_model_exec148_reserve(model_, &base, &slot_stride_, &reserve_slots_) == ARC_OK)
        reserve_ = static_cast<std::uint8_t*>(base);
}

HipQ4DownBackend::~HipQ4DownBackend() { (void)unroute(); }

bool HipQ4DownBackend::p3_available() const noexcept
{
    try {
        return !sidecar_.empty() && std::filesystem::exists(sidecar_) &&
               std::filesystem::file_size(sidecar_) == family_bytes_;
    } catch (...) {
        return false;
    }
}

// Gives the reserve up and resets the state after a failed acquisition.
void HipQ4DownBackend::drop() noexcept
{
    exec_ = nullptr;
    resident_ = false;
    validated_ = false;
}

bool HipQ4DownBackend::acquire_p1()
{
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        const void* src = nullptr;
        if (arc_model_tensor_device(model_, int(layers_[i]), ARC_T_FFN_DOWN, &src) != ARC_OK ||
            arc_exec148_materialize(src, rows_, K_, exec_ + i * slot_stride_, nullptr) != ARC_OK) {
            last_error_ = arc_last_error();
            return false;
        }
    }
    if (arc_synchronize() != ARC_OK) {
        last_error_ = arc_last_error();
        return false;
    }
    return true;
}

bool HipQ4DownBackend::acquire_p3()
{
    std::unique_ptr<std::FILE, int (*)(std::FILE*)> f(std::fopen(sidecar_.c_str(), "rb"), &std::fclose);
    if (!f) {
        last_error_ = "cannot open sidecar " + sidecar_;
        return false;
    }
    std::vector<std::uint8_t> staging(layer_bytes_);
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        if (std::fread(staging.data(), 1, layer_bytes_, f.get()) != layer_bytes_) {
            last_error_ = "short read from sidecar " + sidecar_;
            return false;
        }
        if (arc_memcpy_htod(exec_ + i * slot_stride_, staging.data(), layer_bytes_, nullptr) != ARC_OK ||
            arc_synchronize() != ARC_OK) {
            last_error_ = arc_last_error();
            return false;
        }
    }
    return true;
}

bool HipQ4DownBackend::acquire_p0()
{
    if (host_src_.size() != layers_.size()) {
        last_error_ = "host sources do not cover the Q4_K layers";
        return false;
    }
    const unsigned threads = std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
    std::vector<std::uint8_t> staging(layer_bytes_);
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        exec148_repack_host(host_src_[i], rows_, K_, staging.data(), threads);
        if (arc_memcpy_htod(exec_ + i * slot_stride_, staging.data(), layer_bytes_, nullptr) != ARC_OK ||
            arc_synchronize() != ARC_OK) {
            last_error_ = arc_last_error();
            return false;
        }
    }
    return true;
}

bind::BackendStatus HipQ4DownBackend::acquire(reg::AcquisitionPathId path, reg::PrimitiveId target,
                                              std::uint64_t residency_bytes, bind::RepresentationHandle& out) noexcept
{
    out = {};
    if (target != q4reg::kPrimitiveB || residency_bytes != family_bytes_ || layers_.empty())
        return bind::BackendStatus::INVALID_BINDING_STATE;
    if (resident_) return bind::BackendStatus::INVALID_BINDING_STATE;
    if (path == q4reg::kAcquireSecondary && !p3_available()) return bind::BackendStatus::UNAVAILABLE;
    if (path != q4reg::kAcquirePrimary && path != q4reg::kAcquireSecondary && path != q4reg::kAcquireTertiary)
        return bind::BackendStatus::UNAVAILABLE;
    try {
        // the model's reserve holds one slot per Q4_K ffn_down, in layer order
        if (!reserve_ || reserve_slots_ < layers_.size() || slot_stride_ < layer_bytes_) {
            last_error_ = "the model has no EXEC148 reserve for these layers";
            return bind::BackendStatus::ACQUISITION_FAILED;
        }
        exec_ = reserve_;
        ++counters_.b_allocations;
        bool ok;
        if (path == q4reg::kAcquirePrimary) {
            ++counters_.p1_calls;
            ok = acquire_p1();
        } else if (path == q4reg::kAcquireSecondary) {
            ++counters_.p3_calls;
            ok = acquire_p3();
        } else {
            ++counters_.p0_calls;
            ok = acquire_p0();
        }
        if (!ok) {
            drop();
            return bind::BackendStatus::ACQUISITION_FAILED;
        }
        ++counters_.b_materializations;
        resident_ = true;
        validated_ = false;
        out = {1ull};
        return bind::BackendStatus::OK;
    } catch (const std::exception& e) {
        last_error_ = e.what();
    } catch (...) {
        last_error_ = "unknown acquisition failure";
    }
    drop();
    return bind::BackendStatus::ACQUISITION_FAILED;
}

bind::BackendStatus HipQ4DownBackend::validate(bind::RepresentationHandle representation,
                                               reg::CapabilityId capability, reg::PrimitiveId target) noexcept
{
    if (representation.opaque != 1ull || capability != q4reg::kCapability || target != q4reg::kPrimitiveB ||
        !resident_)
        return bind::BackendStatus::INVALID_BINDING_STATE;
    ++counters_.b_validations;
    validated_ = false;
    std::vector<const void*> src(layers_.size()), img(layers_.size());
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        if (arc_model_tensor_device(model_, int(layers_[i]), ARC_T_FFN_DOWN, &src[i]) != ARC_OK) {
            last_error_ = arc_last_error();
            return bind::BackendStatus::VALIDATION_FAILED;
        }
        img[i] = exec_ + i * slot_stride_;
    }
    std::uint64_t total = 0;
    if (arc_exec148_validate_many(src.data(), img.data(), std::uint32_t(layers_.size()), rows_, K_, &total, nullptr) !=
        ARC_OK) {
        last_error_ = arc_last_error();
        return bind::BackendStatus::VALIDATION_FAILED;
    }
    last_mismatched_ = total;
    if (total) {
        last_error_ = std::to_string(total) + " EXEC148 blocks differ from their Q4_K source";
        return bind::BackendStatus::VALIDATION_FAILED;
    }
    validated_ = true;
    return bind::BackendStatus::OK;
}

bool HipQ4DownBackend::unroute() noexcept
{
    if (!routed_) return true;
    bool ok = true;
    for (std::uint32_t l : layers_)
        if (arc_session_route_down(routed_, l, nullptr) != ARC_OK) ok = false;
    if (ok) routed_ = nullptr;
    else last_error_ = arc_last_error();
    return ok;
}

bind::BackendStatus HipQ4DownBackend::release(reg::PrimitiveId target, bind::RepresentationHandle representation) noexcept
{
    if (target != q4reg::kPrimitiveB || representation.opaque != 1ull || !resident_)
        return bind::BackendStatus::INVALID_BINDING_STATE;
    // a session must not keep a route into freed memory
    if (!unroute()) return bind::BackendStatus::RELEASE_FAILED;
    exec_ = nullptr;
    resident_ = false;
    validated_ = false;
    ++counters_.b_releases;
    return bind::BackendStatus::OK;
}

bind::BackendStatus HipQ4DownBackend::resolve_primitive(reg::PrimitiveId primitive, bind::PrimitiveHandle& out) noexcept
{
    out = {};
    if (primitive == q4reg::kPrimitiveA) {
        ++counters_.resolve_a;
        out = {primitive.value};
        return bind::BackendStatus::OK;
    }
    if (primitive == q4reg::kPrimitiveB) {
        ++counters_.resolve_b;
        if (!resident_ || !validated_) return bind::BackendStatus::PRIMITIVE_UNAVAILABLE;
        out = {primitive.value};
        return bind::BackendStatus::OK;
    }
    return bind::BackendStatus::PRIMITIVE_UNAVAILABLE;
}

bool HipQ4DownBackend::route(arc_session* session, bind::PrimitiveHandle primitive) noexcept
{
    if (!session) {
        last_error_ = "null session";
        return false;
    }
    if (primitive.opaque == q4reg::kPrimitiveA.value) {
        if (routed_ && routed_ != session && !unroute()) return false;
        for (std::uint32_t l : layers_)
            if (arc_session_route_down(session, l, nullptr) != ARC_OK) {
                last_error_ = arc_last_error();
                return false;
            }
        if (routed_ == session) routed_ = nullptr;
        return true;
    }
    if (primitive.opaque == q4reg::kPrimitiveB.value && resident_ && validated_) {
        if (routed_ && routed_ != session) {
            last_error_ = "the EXEC148 image is routed into another session";
            return false;
        }
        for (std::size_t i = 0; i < layers_.size(); ++i)
            if (arc_session_route_down(session, layers_[i], exec_ + i * slot_stride_) != ARC_OK) {
                last_error_ = arc_last_error();
                return false;
            }
        routed_ = session;
        return true;
    }
    last_error_ = "primitive handle not routable";
    return false;
}

}  // namespace arcllm::v1::hip_q4_down
