// qwen2_binding.cpp -- bind_qwen2 (see qwen2_binding.h).
#include "qwen2_binding.h"

#include <stdexcept>
#include <string>

namespace arcllm::v1::runtime {

namespace {

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error("ArcLLM runtime: " + what); }

uint32_t meta_u32(const gguf::File& f, const std::string& key, uint32_t fallback)
{
    const gguf::Value* v = f.find_value(key);
    if (!v) return fallback;
    const uint64_t x = v->as_u64();
    if (x > 0xffffffffull) fail("metadata " + key + " out of range");
    return uint32_t(x);
}

float meta_f32(const gguf::File& f, const std::string& key, float fallback)
{
    const gguf::Value* v = f.find_value(key);
    return v ? float(v->as_f64()) : fallback;
}

const gguf::Tensor& need(const gguf::File& f, const std::string& name)
{
    const gguf::Tensor* t = f.find_tensor(name);
    if (!t) fail("missing tensor " + name);
    return *t;
}

std::string layer_name(uint32_t l, const char* suffix) { return "blk." + std::to_string(l) + "." + suffix; }

}  // namespace

Qwen2Binding bind_qwen2(const gguf::File& f)
{
    Qwen2Binding b;
    arc_model_dims& d = b.dims;
    const gguf::Value* arch = f.find_value("general.architecture");
    if (arch && arch->type == gguf::kString && arch->s != "qwen2") fail("unsupported architecture " + arch->s);
    d.layers = meta_u32(f, "qwen2.block_count", 0);
    if (d.layers == 0 || d.layers > ARC_MAX_LAYERS) fail("block count mismatch");
    const gguf::Tensor& emb = need(f, "token_embd.weight");
    if (emb.dims.size() != 2) fail("token_embd.weight must be 2-D");
    d.hidden = meta_u32(f, "qwen2.embedding_length", uint32_t(emb.dims[0]));
    d.vocab = uint32_t(emb.dims[1]);
    d.q_heads = meta_u32(f, "qwen2.attention.head_count", 0);
    d.kv_heads = meta_u32(f, "qwen2.attention.head_count_kv", d.q_heads);
    d.head_dim = d.q_heads ? d.hidden / d.q_heads : 0;
    d.ffn = meta_u32(f, "qwen2.feed_forward_length", 0);
    d.rms_eps = meta_f32(f, "qwen2.attention.layer_norm_rms_epsilon", 1e-6f);
    d.rope_theta = meta_f32(f, "qwen2.rope.freq_base", 1000000.0f);
    const size_t expect = 3 + size_t(d.layers) * 12;
    if (f.tensors().size() != expect)
        fail("tensor census mismatch: " + std::to_string(f.tensors().size()) + " tensors, expected " +
             std::to_string(expect));
    for (uint32_t l = 0; l < d.layers; ++l) {
        const gguf::Tensor& v = need(f, layer_name(l, "attn_v.weight"));
        const gguf::Tensor& dn = need(f, layer_name(l, "ffn_down.weight"));
        if ((v.type != gguf::kTypeQ4K && v.type != gguf::kTypeQ6K) ||
            (dn.type != gguf::kTypeQ4K && dn.type != gguf::kTypeQ6K))
            fail("mixed-quant layer obstruction: " + std::to_string(l));
        d.v_type[l] = int32_t(v.type);
        d.down_type[l] = int32_t(dn.type);
    }

    static const char* const kGlobal[ARC_T_GLOBAL_COUNT] = {"token_embd.weight", "output.weight",
                                                             "output_norm.weight"};
    static const char* const kLayer[ARC_T_LAYER_COUNT] = {
        "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q.bias",     "attn_k.bias",
        "attn_v.bias",      "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
        "ffn_down.weight"};
    auto bind_one = [&](int layer, int slot, const std::string& name) {
        int qtype = 0;
        uint32_t rows = 0, K = 0;
        uint64_t bytes = 0;
        if (arc_model_tensor_info(&d, layer, slot, &qtype, &rows, &K, &bytes) != ARC_OK)
            fail(std::string("model dims: ") + arc_last_error());
        const gguf::Tensor& t = need(f, name);
        const bool vec = qtype == 0;
        const uint32_t want_type = vec ? gguf::kTypeF32 : uint32_t(qtype);
        const bool shape_ok = vec ? (t.dims.size() == 1 && t.dims[0] == K)
                                  : (t.dims.size() == 2 && t.dims[0] == K && t.dims[1] == rows);
        if (t.type != want_type || !shape_ok || t.nbytes != bytes) fail("tensor " + name + " has an unexpected type or shape");
        b.ptrs.push_back(t.data);
    };
    for (int s = 0; s < ARC_T_GLOBAL_COUNT; ++s) bind_one(-1, s, kGlobal[s]);
    for (uint32_t l = 0; l < d.layers; ++l)
        for (int s = 0; s < ARC_T_LAYER_COUNT; ++s) bind_one(int(l), s, layer_name(l, kLayer[s]));
    return b;
}


}  // namespace arcllm::v1::runtime
