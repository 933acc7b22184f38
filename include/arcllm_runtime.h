/* arcllm_runtime.h -- C entry points of the host runtime library
 * (libarcllm_runtime.so, which also exports the C++ API of
 * include/arcllm/v1/runtime.h).
 */
#ifndef ARCLLM_RUNTIME_H
#define ARCLLM_RUNTIME_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Maps and checks a GGUF file (the checks generate() applies before binding
 * a model: magic, version 2/3, metadata and tensor table in bounds, tensor
 * data aligned, inside the file, non-overlapping, F32/Q4_K/Q6_K only) and
 * writes a JSON description {version, alignment, data_offset, file_size,
 * metadata{key: value}, tensors[{name, type, dims, offset, nbytes}]} to out.
 * Returns 0, 1 on a rejected file (out = the error message) or 2 when out was
 * too small (out holds a truncated prefix).  No device is used.  Mirrors the
 * reference's GgufReader::read (src/gguf.cpp:108-152) and TensorStore::inspect
 * (src/tensor_store.cpp:130-239). */
int arcllm_gguf_describe(const char *path, char *out, size_t cap);

#ifdef __cplusplus
}
#endif
#endif /* ARCLLM_RUNTIME_H */
