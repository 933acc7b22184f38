// gguf.h -- read-only GGUF (v2/v3) container over a POSIX memory map.
//
// The runtime reads model tensors in place: the file is mapped once, the
// header, metadata and tensor table are parsed with bounds checks against the
// mapping, and each tensor is exposed as a pointer into the mapped bytes
// (zero-copy; the packed Q4_K/Q6_K super-blocks are uploaded verbatim).
//
// Format and checks follow the reference reader (src/gguf.cpp:108-152) and
// its TensorStore invariants (src/tensor_store.cpp: bounds, overlap,
// supported types, row sizes).  Errors throw std::runtime_error.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace arcllm::gguf {

enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

enum TensorType : uint32_t { kTypeF32 = 0, kTypeQ4K = 12, kTypeQ6K = 14 };

// One metadata value.  Scalars keep their numeric value in the matching
// field; arrays record their element type and length (elements skipped).
struct Value {
    uint32_t type = 0;
    uint64_t u = 0;      // unsigned integers and bool
    int64_t i = 0;       // signed integers
    double f = 0.0;      // floats
    std::string s;       // strings
    uint32_t array_type = 0;
    uint64_t array_len = 0;

    bool is_integer() const;
    bool is_float() const;
    uint64_t as_u64() const;  // throws unless a non-negative integer
    double as_f64() const;    // integers and floats
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;  // dims[0] = row length (innermost)
    uint32_t type = 0;
    uint64_t offset = 0;         // relative to the data section
    uint64_t nbytes = 0;
    uint64_t row_bytes = 0;
    uint64_t rows = 0;
    const uint8_t* data = nullptr;  // into the mapping
};

class File {
public:
    explicit File(const std::string& path);  // maps, parses and validates
    ~File();
    File(const File&) = delete;
    File& operator=(const File&) = delete;

    uint32_t version() const { return version_; }
    uint64_t alignment() const { return alignment_; }
    uint64_t data_offset() const { return data_offset_; }
    uint64_t file_size() const { return size_; }
    const std::map<std::string, Value>& metadata() const { return meta_; }
    const std::vector<Tensor>& tensors() const { return tensors_; }

    const Value* find_value(const std::string& key) const;
    const Tensor* find_tensor(const std::string& name) const;

private:
    void parse();
    void validate();

    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    uint64_t size_ = 0;
    uint32_t version_ = 0;
    uint64_t alignment_ = 32;
    uint64_t data_offset_ = 0;
    std::map<std::string, Value> meta_;
    std::vector<Tensor> tensors_;
};

// Bytes per row of `type` with row length ne0 (throws on unsupported types or
// a row length that is not a whole number of 256-weight super-blocks).
uint64_t row_bytes(uint32_t type, uint64_t ne0);

}  // namespace arcllm::gguf
