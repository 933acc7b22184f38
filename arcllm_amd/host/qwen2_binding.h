// qwen2_binding.h -- the GGUF -> tensor-slot binding of a Qwen2-architecture
// model: dims from the metadata (with the reference's eps/theta defaults),
// the tensor census, the per-layer attn_v / ffn_down quantisation, and every
// tensor checked against its slot's expected type, shape and size
// (arc_model_tensor_info).  The reference's model contract checks of
// src/arcllm_v1_runtime.cpp:164-300.  Errors throw std::runtime_error.
#pragma once

#include "../../include/arcllm_hip.h"
#include "gguf.h"

#include <vector>

namespace arcllm::v1::runtime {

struct Qwen2Binding {
    arc_model_dims dims{};
    // tensors[ARC_T_GLOBAL_COUNT + layer * ARC_T_LAYER_COUNT + slot], pointers
    // into the file's mapping (valid while the gguf::File lives)
    std::vector<const void*> ptrs;
};

Qwen2Binding bind_qwen2(const gguf::File& file);

}  // namespace arcllm::v1::runtime
