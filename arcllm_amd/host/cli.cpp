// cli.cpp -- command-line front end of generate(), with the reference CLI's
// flags, messages, result schema and exit status (src/arcllm_v1_runtime_cli.cpp:9-103):
//   arcllm_runtime --model M.gguf --shader-dir D --tokens 1,2,3 --max-new N
//                  --profile 0|1 --within-validated-domain 0|1
//                  [--sidecar S] [--out result.json]
// Prints {"schema":"arcllm.v1.runtime.result.v0.1", "generated_token_ids":
// [...], "stats":{...}} to stdout or --out; errors go to stderr with exit
// status 2.
//
// The flags are one table (kOptions): each entry names its flag, whether the
// run needs it, and how its value lands in the request.  The result is
// written from a second table (kStatFields) of the statistics in schema order.
#include "../../include/arcllm/v1/runtime.h"

#include <cstdint>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

namespace rt = arcllm::v1::runtime;

[[noreturn]] void refuse(const std::string& why) { throw std::runtime_error(why); }

// What the command line fills in before the request is complete.
struct Invocation {
    rt::RunRequest req;
    std::string token_csv;
    std::string out_path;  // empty: stdout
};

bool flag_bit(const std::string& v, const char* flag)
{
    if (v != "0" && v != "1") refuse(std::string(flag) + " must be 0 or 1");
    return v == "1";
}

struct Option {
    const char* flag;
    bool needed;  // the run is refused unless the flag came with a nonempty value
    void (*store)(Invocation&, const std::string&);
};

const Option kOptions[] = {
    {"--model", true, [](Invocation& c, const std::string& v) { c.req.model_path = v; }},
    {"--shader-dir", true, [](Invocation& c, const std::string& v) { c.req.shader_dir = v; }},
    {"--sidecar", false, [](Invocation& c, const std::string& v) { c.req.sidecar_path = v; }},
    {"--tokens", true, [](Invocation& c, const std::string& v) { c.token_csv = v; }},
    {"--max-new", false,
     [](Invocation& c, const std::string& v) { c.req.max_new_tokens = static_cast<std::uint32_t>(std::stoul(v)); }},
    {"--profile", true,
     [](Invocation& c, const std::string& v) {
         c.req.evidence_profile =
             flag_bit(v, "--profile") ? rt::EvidenceProfile::PROFILE_1 : rt::EvidenceProfile::PROFILE_0;
     }},
    {"--within-validated-domain", true,
     [](Invocation& c, const std::string& v) {
         c.req.request_within_validated_domain = flag_bit(v, "--within-validated-domain");
     }},
    {"--out", false, [](Invocation& c, const std::string& v) { c.out_path = v; }},
};
constexpr std::size_t kOptionCount = sizeof(kOptions) / sizeof(kOptions[0]);

Invocation read_command_line(int argc, char** argv)
{
    Invocation c;
    bool given[kOptionCount] = {};
    for (int i = 1; i < argc; ++i) {
        const std::string flag = argv[i];
        std::size_t k = 0;
        while (k < kOptionCount && flag != kOptions[k].flag) ++k;
        if (k == kOptionCount) refuse("unknown argument: " + flag);
        if (i + 1 == argc) refuse("missing value for " + flag);
        const std::string value = argv[++i];
        kOptions[k].store(c, value);
        given[k] = !value.empty();
    }
    for (std::size_t k = 0; k < kOptionCount; ++k)
        if (kOptions[k].needed && !given[k])
            refuse("required: --model --shader-dir --tokens --max-new --profile --within-validated-domain");
    return c;
}

// Comma-separated decimal ids, each within uint32.
std::vector<std::uint32_t> token_ids(const std::string& csv)
{
    std::vector<std::uint32_t> ids;
    std::string::size_type at = 0;
    for (;;) {
        const std::string::size_type end = csv.find(',', at);
        const std::string item = csv.substr(at, end == std::string::npos ? std::string::npos : end - at);
        if (item.empty() || item.find_first_not_of("0123456789") != std::string::npos)
            refuse("bad token in --tokens: '" + item + "'");
        const unsigned long long id = std::stoull(item);
        if (id > 0xffffffffull) refuse("token exceeds uint32");
        ids.push_back(static_cast<std::uint32_t>(id));
        if (end == std::string::npos) return ids;
        at = end + 1;
    }
}

// ---------------------------------------------------------------- result
struct StatField {
    const char* key;
    std::uint64_t (*read)(const rt::RuntimeStats&);
};

#define ARC_STAT(member) {#member, [](const rt::RuntimeStats& s) { return std::uint64_t(s.member); }}
const StatField kStatFields[] = {
    ARC_STAT(prefill_dispatches), ARC_STAT(prefill_submits), ARC_STAT(decode_dispatches_per_step),
    ARC_STAT(decode_submits_per_step), ARC_STAT(decode_steps), ARC_STAT(route_a_steps), ARC_STAT(route_b_steps),
    ARC_STAT(acquire_events), ARC_STAT(evict_events), ARC_STAT(b_allocations), ARC_STAT(b_materializations),
    ARC_STAT(b_validations), ARC_STAT(b_releases), ARC_STAT(p1_calls), ARC_STAT(p3_calls), ARC_STAT(p0_calls),
};
#undef ARC_STAT

void write_result(std::ostream& o, const rt::RunResult& r)
{
    o << "{\n  \"schema\":\"arcllm.v1.runtime.result.v0.1\",\n  \"generated_token_ids\":[";
    const char* sep = "";
    for (std::uint32_t id : r.generated_token_ids) {
        o << sep << id;
        sep = ",";
    }
    o << "],\n  \"stats\":{";
    for (const StatField& f : kStatFields) o << '"' << f.key << "\":" << f.read(r.stats) << ',';
    o << "\"finite\":" << (r.stats.finite ? "true" : "false") << "}\n}\n";
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        Invocation c = read_command_line(argc, argv);
        c.req.input_token_ids = token_ids(c.token_csv);
        const rt::RunResult result = rt::generate(c.req);
        if (c.out_path.empty()) {
            write_result(std::cout, result);
            return 0;
        }
        std::ofstream file(c.out_path, std::ios::binary | std::ios::trunc);
        if (!file) refuse("cannot open --out path");
        write_result(file, result);
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "ArcLLM runtime error: " << e.what() << "\n";
        return 2;
    }
}
