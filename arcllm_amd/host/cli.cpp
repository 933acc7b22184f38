// cli.cpp -- command-line front end of generate(), with the reference CLI's
// flags and result schema (src/arcllm_v1_runtime_cli.cpp:9-103):
//   arcllm_runtime --model M.gguf --shader-dir D --tokens 1,2,3 --max-new N
//                  --profile 0|1 --within-validated-domain 0|1
//                  [--sidecar S] [--out result.json]
// Prints {"schema":"arcllm.v1.runtime.result.v0.1", "generated_token_ids":
// [...], "stats":{...}} to stdout or --out; errors go to stderr with exit
// status 2.
#include "../../include/arcllm/v1/runtime.h"

#include <cstdint>
#include <fstream>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

namespace rt = arcllm::v1::runtime;

std::vector<std::uint32_t> parse_token_list(const std::string& csv)
{
    std::vector<std::uint32_t> ids;
    std::size_t start = 0;
    while (start <= csv.size()) {
        const std::size_t comma = csv.find(',', start);
        const std::string item = csv.substr(start, comma == std::string::npos ? std::string::npos : comma - start);
        if (item.empty() || item.find_first_not_of("0123456789") != std::string::npos)
            throw std::runtime_error("bad token in --tokens: '" + item + "'");
        const unsigned long long v = std::stoull(item);
        if (v > 0xffffffffull) throw std::runtime_error("token exceeds uint32");
        ids.push_back(static_cast<std::uint32_t>(v));
        if (comma == std::string::npos) break;
        start = comma + 1;
    }
    return ids;
}

void emit(std::ostream& o, const rt::RunResult& r)
{
    const rt::RuntimeStats& s = r.stats;
    o << "{\n  \"schema\":\"arcllm.v1.runtime.result.v0.1\",\n  \"generated_token_ids\":[";
    for (std::size_t i = 0; i < r.generated_token_ids.size(); ++i) o << (i ? "," : "") << r.generated_token_ids[i];
    o << "],\n  \"stats\":{"
      << "\"prefill_dispatches\":" << s.prefill_dispatches << ",\"prefill_submits\":" << s.prefill_submits
      << ",\"decode_dispatches_per_step\":" << s.decode_dispatches_per_step
      << ",\"decode_submits_per_step\":" << s.decode_submits_per_step << ",\"decode_steps\":" << s.decode_steps
      << ",\"route_a_steps\":" << s.route_a_steps << ",\"route_b_steps\":" << s.route_b_steps
      << ",\"acquire_events\":" << s.acquire_events << ",\"evict_events\":" << s.evict_events
      << ",\"b_allocations\":" << s.b_allocations << ",\"b_materializations\":" << s.b_materializations
      << ",\"b_validations\":" << s.b_validations << ",\"b_releases\":" << s.b_releases
      << ",\"p1_calls\":" << s.p1_calls << ",\"p3_calls\":" << s.p3_calls << ",\"p0_calls\":" << s.p0_calls
      << ",\"finite\":" << (s.finite ? "true" : "false") << "}\n}\n";
}

bool parse_bit(const std::string& v, const char* flag)
{
    if (v == "0") return false;
    if (v == "1") return true;
    throw std::runtime_error(std::string(flag) + " must be 0 or 1");
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        rt::RunRequest req;
        std::string tokens, out;
        bool have_profile = false, have_scope = false;
        for (int i = 1; i < argc; ++i) {
            const std::string a = argv[i];
            auto value = [&]() -> std::string {
                if (i + 1 >= argc) throw std::runtime_error("missing value for " + a);
                return argv[++i];
            };
            if (a == "--model") req.model_path = value();
            else if (a == "--shader-dir") req.shader_dir = value();
            else if (a == "--sidecar") req.sidecar_path = value();
            else if (a == "--tokens") tokens = value();
            else if (a == "--max-new") req.max_new_tokens = static_cast<std::uint32_t>(std::stoul(value()));
            else if (a == "--profile") {
                req.evidence_profile = parse_bit(value(), "--profile") ? rt::EvidenceProfile::PROFILE_1
                                                                       : rt::EvidenceProfile::PROFILE_0;
                have_profile = true;
            } else if (a == "--within-validated-domain") {
                req.request_within_validated_domain = parse_bit(value(), "--within-validated-domain");
                have_scope = true;
            } else if (a == "--out") out = value();
            else throw std::runtime_error("unknown argument: " + a);
        }
        if (req.model_path.empty() || req.shader_dir.empty() || tokens.empty() || !have_profile || !have_scope)
            throw std::runtime_error(
                "required: --model --shader-dir --tokens --max-new --profile --within-validated-domain");
        req.input_token_ids = parse_token_list(tokens);
        const rt::RunResult result = rt::generate(req);
        if (out.empty()) {
            emit(std::cout, result);
        } else {
            std::ofstream f(out, std::ios::binary | std::ios::trunc);
            if (!f) throw std::runtime_error("cannot open --out path");
            emit(f, result);
        }
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "ArcLLM runtime error: " << e.what() << "\n";
        return 2;
    }
}
