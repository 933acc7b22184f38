// q4_backend_host_check.cpp -- host-side checks of the gfx950 Q4-down backend
// that need no GPU:
//   repack <in.q4> <rows> <K> <out.e148> <threads>
//       the P0 host repack (exec148_repack_host) of a Q4_K tensor file;
//   registration <family_bytes>
//       registers the MI355X bundle and prints, per profile, the first future
//       reuse at which each acquisition path is chosen when it is the only
//       available one ("p<k> <profile> <path> <first>"), the threshold table
//       ("thr ...") and the add_bundle status.
#include "../../arcllm_amd/host/q4_down_backend.h"
#include "../../arcllm_amd/host/registrations/arcllm_v1_q4k_down_reference_registration_v2.h"

#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace arcllm::v1;
namespace q4 = reference_registration_v2;
namespace gp = policy_v4;

static int repack(int argc, char** argv)
{
    if (argc != 7) return 2;
    const std::uint32_t rows = std::uint32_t(std::strtoul(argv[3], nullptr, 10));
    const std::uint32_t K = std::uint32_t(std::strtoul(argv[4], nullptr, 10));
    const unsigned threads = unsigned(std::strtoul(argv[6], nullptr, 10));
    const std::size_t in_bytes = std::size_t(rows) * (K / 256) * 144;
    std::vector<std::uint8_t> in(in_bytes), out(hip_q4_down::exec148_bytes(rows, K));
    std::FILE* f = std::fopen(argv[2], "rb");
    if (!f || std::fread(in.data(), 1, in_bytes, f) != in_bytes) return 3;
    std::fclose(f);
    hip_q4_down::exec148_repack_host(in.data(), rows, K, out.data(), threads);
    f = std::fopen(argv[5], "wb");
    if (!f || std::fwrite(out.data(), 1, out.size(), f) != out.size()) return 4;
    std::fclose(f);
    return 0;
}

static int registration(int argc, char** argv)
{
    if (argc != 3) return 2;
    const std::uint64_t family = std::strtoull(argv[2], nullptr, 10);
    const hip_q4_down::Mi355xRegistration regn(family);
    registry_v2::PrimitiveRegistry r;
    registry_v2::RegistryError e{};
    const auto s = r.add_bundle(regn.bundle(), &e);
    std::printf("add %u %s\n", unsigned(s), e.category ? e.category : "-");
    const auto& t = hip_q4_down::Mi355xRegistration::thresholds();
    std::printf("thr %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 "\n", t[0], t[1], t[2], t[3],
                t[4], t[5]);
    const registry_v2::AcquisitionPathId paths[] = {q4::kAcquirePrimary, q4::kAcquireSecondary, q4::kAcquireTertiary};
    for (int prof = 0; prof < 2; ++prof)
        for (int k = 0; k < 3; ++k) {
            std::uint64_t first = 0;
            std::uint64_t bytes = 0;
            for (std::uint64_t h = 1; h <= 100000 && !first; ++h) {
                const gp::PrimitiveRuntimeState ps[] = {{q4::kPrimitiveA, false, true, true, true, true},
                                                        {q4::kPrimitiveB, false, false, true, false, true}};
                const gp::AcquisitionRuntimeState as[] = {{q4::kAcquirePrimary, k == 0, false},
                                                          {q4::kAcquireSecondary, k == 1, false},
                                                          {q4::kAcquireTertiary, k == 2, false},
                                                          {q4::kAcquireDisabledWarm, true, false}};
                gp::PolicyRequest q{};
                q.capability = q4::kCapability;
                q.profile = prof ? q4::kProfile1 : q4::kProfile0;
                q.future_reuse_known = true;
                q.future_reuse_units = h;
                q.primitive_states = ps;
                q.primitive_state_count = 2;
                q.acquisition_states = as;
                q.acquisition_state_count = 4;
                const gp::PolicyDecision d = gp::evaluate(r, q);
                if (d.status != gp::PolicyStatus::OK) return 5;
                if (d.lifecycle == gp::LifecycleAction::ACQUIRE) {
                    if (d.acquisition != paths[k]) return 6;
                    first = h;
                    bytes = d.requested_residency_bytes;
                }
            }
            std::printf("p%d %d %" PRIu64 " %" PRIu64 "\n", prof, k, first, bytes);
        }
    return 0;
}

int main(int argc, char** argv)
{
    if (argc >= 2 && !std::strcmp(argv[1], "repack")) return repack(argc, argv);
    if (argc >= 2 && !std::strcmp(argv[1], "registration")) return registration(argc, argv);
    std::fprintf(stderr, "usage: repack IN ROWS K OUT THREADS | registration FAMILY_BYTES\n");
    return 2;
}
