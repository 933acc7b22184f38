// q4_paths.cpp -- arcllm_q4_paths: the Q4_K ffn_down routes and EXEC148
// acquisition paths of the gfx950 backend, exercised and timed end to end.
//
//   arcllm_q4_paths (--model M.gguf | --synthetic-7b [--seed S] [--q4-layers 3,4,...])
//                   [--ctx C] [--steps N] [--paths p1,p3,p0] [--sidecar FILE]
//   arcllm_q4_paths --thresholds
//       prints the registration's reuse thresholds (no GPU use):
//       {"profile0": {"p1": .., "p3": .., "p0": ..}, "profile1": {...}}
//
// On one session (KV prefilled to C positions with N(0,1)):
//   1. route A: N greedy decode steps from a fixed token at position C, timed
//      (after a warm-up call that captures the step graph);
//   2. per path in --paths order: acquire (allocation + repack or upload;
//      P3 reads --sidecar, which is first written from the P1 image and
//      dropped from the page cache when it does not exist yet), validate on the
//      GPU against the Q4_K sources, hash the downloaded image, and after the
//      first path: route B for the same N steps, timed; then release;
//   3. the reuse threshold of each path on this model: ceil((acquire +
//      validate) / (route A - route B per token)).
// Prints one JSON object.  The synthetic model is the Qwen2.5-7B shape with
// the Q4_K ffn_down layers of its Q4_K_M file (3, 4, 6, 7, 8, 11, 12, 14, 15,
// 17, 18, 19, 21, 22: src/arcllm_v1_q4_vulkan_backend_v4_runtime.h:35-37 of
// the reference) and random-init weights.
#include "../../include/arcllm_hip.h"
#include "gguf.h"
#include "q4_down_backend.h"
#include "qwen2_binding.h"
#include "registrations/arcllm_v1_q4k_down_reference_registration_v2.h"

#include <fcntl.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

using namespace arcllm::v1;
namespace q4reg = reference_registration_v2;
namespace bind = binding_v4;
using Clock = std::chrono::steady_clock;

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }
void check(int rc, const char* what)
{
    if (rc != ARC_OK) fail(std::string(what) + ": " + arc_last_error());
}
double ms_since(Clock::time_point t0) { return std::chrono::duration<double, std::milli>(Clock::now() - t0).count(); }
void progress(const std::string& what) { std::cerr << "arcllm_q4_paths: " << what << std::endl; }

std::vector<std::uint32_t> parse_list(const std::string& csv)
{
    std::vector<std::uint32_t> v;
    std::stringstream ss(csv);
    std::string item;
    while (std::getline(ss, item, ',')) v.push_back(std::uint32_t(std::stoul(item)));
    return v;
}

std::uint64_t fnv(const std::uint8_t* p, std::size_t n, std::uint64_t h)
{
    for (std::size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

struct Decoded {
    double ms_per_token = 0;
    std::vector<std::uint32_t> tokens;
};

Decoded decode(arc_session* s, std::uint32_t ctx, std::uint32_t steps)
{
    Decoded d;
    d.tokens.resize(steps);
    std::uint32_t nf = 0;
    check(arc_session_decode(s, 1234, ctx, 2, 0, nullptr, &nf), "warm-up decode");
    const auto t0 = Clock::now();
    check(arc_session_decode(s, 1234, ctx, steps, 0, d.tokens.data(), &nf), "decode");
    d.ms_per_token = ms_since(t0) / steps;
    if (nf) fail("non-finite logits");
    return d;
}

std::string tokens_json(const std::vector<std::uint32_t>& t)
{
    std::string s = "[";
    for (std::size_t i = 0; i < t.size(); ++i) s += (i ? "," : "") + std::to_string(t[i]);
    return s + "]";
}

// Writes the resident image to `path` (layer images back to back) and drops
// the file from the page cache, so a following P3 read comes from storage.
void write_sidecar(const hip_q4_down::HipQ4DownBackend& be, const std::string& path)
{
    std::vector<std::uint8_t> buf(be.layer_bytes());
    std::unique_ptr<std::FILE, int (*)(std::FILE*)> f(std::fopen(path.c_str(), "wb"), &std::fclose);
    if (!f) fail("cannot create " + path);
    for (std::size_t i = 0; i < be.layers().size(); ++i) {
        check(arc_memcpy_dtoh(buf.data(), be.device_image() + i * be.slot_stride(), buf.size(), nullptr), "download");
        check(arc_synchronize(), "download");
        if (std::fwrite(buf.data(), 1, buf.size(), f.get()) != buf.size()) fail("short write to " + path);
    }
    std::fflush(f.get());
    const int fd = fileno(f.get());
    (void)fsync(fd);
    (void)posix_fadvise(fd, 0, 0, POSIX_FADV_DONTNEED);
}

std::uint64_t image_hash(const hip_q4_down::HipQ4DownBackend& be)
{
    std::vector<std::uint8_t> buf(be.layer_bytes());
    std::uint64_t h = 1469598103934665603ull;
    for (std::size_t i = 0; i < be.layers().size(); ++i) {
        check(arc_memcpy_dtoh(buf.data(), be.device_image() + i * be.slot_stride(), buf.size(), nullptr), "download");
        check(arc_synchronize(), "download");
        h = fnv(buf.data(), buf.size(), h);
    }
    return h;
}

int run(int argc, char** argv)
{
    if (argc == 2 && std::string(argv[1]) == "--thresholds") {
        const auto& t = hip_q4_down::Mi355xRegistration::thresholds();
        std::cout << "{\"profile0\":{\"p1\":" << t[0] << ",\"p3\":" << t[1] << ",\"p0\":" << t[2]
                  << "},\"profile1\":{\"p1\":" << t[3] << ",\"p3\":" << t[4] << ",\"p0\":" << t[5] << "}}"
                  << std::endl;
        return 0;
    }
    std::string model_path, sidecar, paths_csv = "p1,p3,p0", layers_csv = "3,4,6,7,8,11,12,14,15,17,18,19,21,22";
    bool synthetic = false;
    std::uint64_t seed = 0x5EED;
    std::uint32_t ctx = 512, steps = 64;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&]() -> std::string {
            if (i + 1 >= argc) fail("missing value for " + a);
            return argv[++i];
        };
        if (a == "--model") model_path = value();
        else if (a == "--synthetic-7b") synthetic = true;
        else if (a == "--seed") seed = std::stoull(value());
        else if (a == "--q4-layers") layers_csv = value();
        else if (a == "--ctx") ctx = std::uint32_t(std::stoul(value()));
        else if (a == "--steps") steps = std::uint32_t(std::stoul(value()));
        else if (a == "--paths") paths_csv = value();
        else if (a == "--sidecar") sidecar = value();
        else fail("unknown argument " + a);
    }
    if (synthetic == !model_path.empty()) fail("give exactly one of --model and --synthetic-7b");
    if (steps == 0) fail("--steps must be >= 1");

    std::unique_ptr<arcllm::gguf::File> file;
    runtime::Qwen2Binding bound;
    std::vector<std::vector<std::uint8_t>> synth_src;
    synth_src.reserve(ARC_MAX_LAYERS);
    arc_model_dims d{};
    arc_model* mraw = nullptr;
    if (synthetic) {
        check(arc_model_dims_qwen25_7b(&d), "dims");
        for (std::uint32_t l : parse_list(layers_csv)) {
            if (l >= d.layers) fail("--q4-layers entry out of range");
            d.down_type[l] = ARC_Q4_K;
        }
        check(arc_model_create_synthetic(&d, seed, &mraw), "synthetic model");
    } else {
        file = std::make_unique<arcllm::gguf::File>(model_path);
        bound = runtime::bind_qwen2(*file);
        d = bound.dims;
        check(arc_model_create(&d, bound.ptrs.data(), &mraw), "model upload");
    }
    std::unique_ptr<arc_model, int (*)(arc_model*)> model(mraw, &arc_model_destroy);
    progress("model resident");

    std::vector<std::uint32_t> layers;
    std::vector<const std::uint8_t*> host;
    for (std::uint32_t l = 0; l < d.layers; ++l) {
        if (d.down_type[l] != ARC_Q4_K) continue;
        layers.push_back(l);
        if (synthetic) {
            int qt;
            std::uint32_t rows, K;
            std::uint64_t bytes;
            check(arc_model_tensor_info(&d, int(l), ARC_T_FFN_DOWN, &qt, &rows, &K, &bytes), "tensor info");
            synth_src.emplace_back(bytes);
            check(arc_model_synth_tensor(&d, seed, int(l), ARC_T_FFN_DOWN, synth_src.back().data()), "host tensor");
            host.push_back(synth_src.back().data());
        } else {
            host.push_back(static_cast<const std::uint8_t*>(
                bound.ptrs[ARC_T_GLOBAL_COUNT + std::size_t(l) * ARC_T_LAYER_COUNT + ARC_T_FFN_DOWN]));
        }
    }
    if (layers.empty()) fail("the model has no Q4_K ffn_down layer");

    arc_session* sraw = nullptr;
    check(arc_session_create(model.get(), ctx + steps + 2, &sraw), "session");
    std::unique_ptr<arc_session, int (*)(arc_session*)> session(sraw, &arc_session_destroy);
    check(arc_session_fill_kv(session.get(), ctx, seed + 1), "KV fill");

    hip_q4_down::HipQ4DownBackend be(model.get(), layers, host, d.hidden, d.ffn, sidecar);
    const Decoded a = decode(session.get(), ctx, steps);
    progress("route A decoded");

    struct PathResult {
        std::string name;
        double acquire_ms = 0, validate_ms = 0;
        std::uint64_t mismatched = 0, hash = 0;
    };
    std::vector<PathResult> results;
    Decoded b;
    bool have_b = false;
    for (const std::string& p : [&] {
             std::vector<std::string> v;
             std::stringstream ss(paths_csv);
             std::string x;
             while (std::getline(ss, x, ',')) v.push_back(x);
             return v;
         }()) {
        const registry_v2::AcquisitionPathId id = p == "p1"   ? q4reg::kAcquirePrimary
                                                  : p == "p3" ? q4reg::kAcquireSecondary
                                                  : p == "p0" ? q4reg::kAcquireTertiary
                                                              : registry_v2::AcquisitionPathId{};
        if (!id) fail("unknown path " + p);
        if (p == "p3" && !be.p3_available()) fail("P3 needs a sidecar of the family size (run p1 first with --sidecar)");
        PathResult r;
        r.name = p;
        bind::RepresentationHandle rep{};
        auto t0 = Clock::now();
        if (be.acquire(id, q4reg::kPrimitiveB, be.family_bytes(), rep) != bind::BackendStatus::OK)
            fail(p + " acquisition failed: " + be.last_error());
        r.acquire_ms = ms_since(t0);
        t0 = Clock::now();
        const bind::BackendStatus vs = be.validate(rep, q4reg::kCapability, q4reg::kPrimitiveB);
        r.validate_ms = ms_since(t0);
        r.mismatched = be.last_mismatched_blocks();
        if (vs != bind::BackendStatus::OK) fail(p + " validation failed: " + be.last_error());
        r.hash = image_hash(be);
        if (!have_b) {
            if (!be.route(session.get(), bind::PrimitiveHandle{q4reg::kPrimitiveB.value})) fail(be.last_error());
            b = decode(session.get(), ctx, steps);
            have_b = true;
        }
        if (p == "p1" && !sidecar.empty() && !std::filesystem::exists(sidecar)) write_sidecar(be, sidecar);
        if (be.release(q4reg::kPrimitiveB, rep) != bind::BackendStatus::OK) fail("release failed: " + be.last_error());
        results.push_back(r);
        progress(p + " acquired, validated and released");
    }

    const double save_us = have_b ? (a.ms_per_token - b.ms_per_token) * 1e3 : 0.0;
    std::ostringstream o;
    o.setf(std::ios::fixed);
    o.precision(4);
    o << "{\"model\":\"" << (synthetic ? "synthetic Qwen2.5-7B shape" : model_path) << "\",\"q4_layers\":"
      << tokens_json(layers) << ",\"rows\":" << d.hidden << ",\"K\":" << d.ffn
      << ",\"family_bytes\":" << be.family_bytes() << ",\"ctx\":" << ctx << ",\"steps\":" << steps
      << ",\"route_a\":{\"ms_per_token\":" << a.ms_per_token << ",\"tokens\":" << tokens_json(a.tokens) << "}";
    if (have_b)
        o << ",\"route_b\":{\"ms_per_token\":" << b.ms_per_token << ",\"tokens\":" << tokens_json(b.tokens)
          << "},\"saving_us_per_token\":" << save_us;
    o << ",\"paths\":{";
    bool same = true;
    for (std::size_t i = 0; i < results.size(); ++i) {
        const PathResult& r = results[i];
        same = same && r.hash == results[0].hash;
        char h[20];
        std::snprintf(h, sizeof h, "%016llx", static_cast<unsigned long long>(r.hash));
        o << (i ? "," : "") << "\"" << r.name << "\":{\"acquire_ms\":" << r.acquire_ms
          << ",\"validate_ms\":" << r.validate_ms << ",\"mismatched_blocks\":" << r.mismatched << ",\"image_fnv\":\""
          << h << "\",\"threshold_tokens\":";
        if (save_us > 0) o << std::uint64_t(std::ceil((r.acquire_ms + r.validate_ms) * 1e3 / save_us));
        else o << "null";
        o << "}";
    }
    o << "},\"images_equal\":" << (same ? "true" : "false") << "}";
    std::cout << o.str() << std::endl;
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "arcllm_q4_paths: " << e.what() << std::endl;
        return 2;
    }
}
