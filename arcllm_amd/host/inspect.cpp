// inspect.cpp -- C entry point describing a GGUF file as JSON (no device
// needed): the runtime library's container checks made testable from any
// language.  Declared in include/arcllm_runtime.h.
#include "../../include/arcllm_runtime.h"
#include "gguf.h"

#include <cstdio>
#include <cstring>
#include <sstream>
#include <stdexcept>
#include <string>

namespace {

std::string json_escape(const std::string& s)
{
    std::string o;
    for (char c : s) {
        const unsigned char u = static_cast<unsigned char>(c);
        if (c == '"' || c == '\\') {
            o += '\\';
            o += c;
        } else if (u < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof(buf), "\\u%04x", u);
            o += buf;
        } else {
            o += c;
        }
    }
    return o;
}

std::string value_json(const arcllm::gguf::Value& v)
{
    using namespace arcllm::gguf;
    std::ostringstream o;
    o.precision(17);
    switch (v.type) {
    case kString: o << '"' << json_escape(v.s) << '"'; break;
    case kArray: o << "{\"array_type\":" << v.array_type << ",\"len\":" << v.array_len << "}"; break;
    case kF32: case kF64: o << v.f; break;
    case kBool: o << (v.u ? "true" : "false"); break;
    case kI8: case kI16: case kI32: case kI64: o << v.i; break;
    default: o << v.u; break;
    }
    return o.str();
}

}  // namespace

extern "C" int arcllm_gguf_describe(const char* path, char* out, size_t cap)
{
    std::string text;
    int rc = 0;
    try {
        const arcllm::gguf::File f(path ? path : "");
        std::ostringstream o;
        o << "{\"version\":" << f.version() << ",\"alignment\":" << f.alignment()
          << ",\"data_offset\":" << f.data_offset() << ",\"file_size\":" << f.file_size() << ",\"metadata\":{";
        bool first = true;
        for (const auto& kv : f.metadata()) {
            o << (first ? "" : ",") << '"' << json_escape(kv.first) << "\":" << value_json(kv.second);
            first = false;
        }
        o << "},\"tensors\":[";
        first = true;
        for (const auto& t : f.tensors()) {
            o << (first ? "" : ",") << "{\"name\":\"" << json_escape(t.name) << "\",\"type\":" << t.type
              << ",\"dims\":[";
            for (size_t d = 0; d < t.dims.size(); ++d) o << (d ? "," : "") << t.dims[d];
            o << "],\"offset\":" << t.offset << ",\"nbytes\":" << t.nbytes << "}";
            first = false;
        }
        o << "]}";
        text = o.str();
    } catch (const std::exception& e) {
        text = e.what();
        rc = 1;
    }
    if (out && cap) {
        const size_t n = text.size() < cap - 1 ? text.size() : cap - 1;
        std::memcpy(out, text.data(), n);
        out[n] = '\0';
    }
    if (!rc && text.size() >= cap) return 2;  // truncated
    return rc;
}
