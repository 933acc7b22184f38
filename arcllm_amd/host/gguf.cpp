// gguf.cpp -- GGUF container over mmap (see gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace arcllm::gguf {

namespace {

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error("GGUF: " + what); }

uint64_t mul_checked(uint64_t a, uint64_t b)
{
    if (a && b > std::numeric_limits<uint64_t>::max() / a) fail("tensor size overflow");
    return a * b;
}

uint64_t align_up(uint64_t x, uint64_t a) { return a ? (x + a - 1) / a * a : x; }

// Bounds-checked little-endian reader over the mapping.
class Cursor {
public:
    Cursor(const uint8_t* p, uint64_t n) : p_(p), n_(n) {}
    uint64_t pos() const { return at_; }

    template <typename T>
    T pod()
    {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + at_, sizeof(T));
        at_ += sizeof(T);
        return v;
    }
    std::string str()
    {
        const uint64_t len = pod<uint64_t>();
        if (len > (1ull << 31)) fail("string too large");
        need(len);
        std::string s(reinterpret_cast<const char*>(p_ + at_), size_t(len));
        at_ += len;
        return s;
    }
    void skip(uint64_t n)
    {
        need(n);
        at_ += n;
    }

private:
    void need(uint64_t n) const
    {
        if (n > n_ || at_ > n_ - n) fail("unexpected end of file");
    }
    const uint8_t* p_;
    uint64_t n_;
    uint64_t at_ = 0;
};

uint64_t scalar_size(uint32_t t)
{
    switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

void read_value(Cursor& c, uint32_t type, Value& v, int depth)
{
    v.type = type;
    switch (type) {
    case kU8: v.u = c.pod<uint8_t>(); break;
    case kI8: v.i = c.pod<int8_t>(); break;
    case kU16: v.u = c.pod<uint16_t>(); break;
    case kI16: v.i = c.pod<int16_t>(); break;
    case kU32: v.u = c.pod<uint32_t>(); break;
    case kI32: v.i = c.pod<int32_t>(); break;
    case kF32: v.f = c.pod<float>(); break;
    case kBool: v.u = c.pod<uint8_t>() ? 1 : 0; break;
    case kString: v.s = c.str(); break;
    case kU64: v.u = c.pod<uint64_t>(); break;
    case kI64: v.i = c.pod<int64_t>(); break;
    case kF64: v.f = c.pod<double>(); break;
    case kArray: {
        if (depth > 4) fail("nested arrays too deep");
        v.array_type = c.pod<uint32_t>();
        v.array_len = c.pod<uint64_t>();
        if (v.array_len > (1ull << 32)) fail("array too large");
        const uint64_t es = scalar_size(v.array_type);
        if (es) {
            c.skip(mul_checked(es, v.array_len));
        } else {
            Value e;
            for (uint64_t k = 0; k < v.array_len; ++k) read_value(c, v.array_type, e, depth + 1);
        }
        break;
    }
    default: fail("unsupported metadata type " + std::to_string(type));
    }
}

}  // namespace

bool Value::is_integer() const
{
    return type == kU8 || type == kI8 || type == kU16 || type == kI16 || type == kU32 || type == kI32 ||
           type == kU64 || type == kI64 || type == kBool;
}

bool Value::is_float() const { return type == kF32 || type == kF64; }

uint64_t Value::as_u64() const
{
    if (type == kI8 || type == kI16 || type == kI32 || type == kI64) {
        if (i < 0) fail("negative value where a count was expected");
        return uint64_t(i);
    }
    if (!is_integer()) fail("integer value expected");
    return u;
}

double Value::as_f64() const
{
    if (is_float()) return f;
    if (type == kI8 || type == kI16 || type == kI32 || type == kI64) return double(i);
    if (is_integer()) return double(u);
    fail("numeric value expected");
}

uint64_t row_bytes(uint32_t type, uint64_t ne0)
{
    switch (type) {
    case kTypeF32: return mul_checked(ne0, 4);
    case kTypeQ4K:
        if (ne0 % 256) fail("Q4_K row length not a multiple of 256");
        return mul_checked(ne0 / 256, 144);
    case kTypeQ6K:
        if (ne0 % 256) fail("Q6_K row length not a multiple of 256");
        return mul_checked(ne0 / 256, 210);
    default: fail("unsupported tensor type " + std::to_string(type));
    }
}

File::File(const std::string& path)
{
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) fail("cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd_, &st) != 0 || st.st_size < 0) {
        ::close(fd_);
        fail("cannot stat " + path);
    }
    size_ = uint64_t(st.st_size);
    if (size_ < 24) {
        ::close(fd_);
        fail("file too small: " + path);
    }
    void* m = ::mmap(nullptr, size_t(size_), PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
        ::close(fd_);
        fail("mmap failed: " + path);
    }
    base_ = static_cast<const uint8_t*>(m);
    try {
        parse();
        validate();
    } catch (...) {
        ::munmap(const_cast<uint8_t*>(base_), size_t(size_));
        ::close(fd_);
        throw;
    }
}

File::~File()
{
    if (base_) ::munmap(const_cast<uint8_t*>(base_), size_t(size_));
    if (fd_ >= 0) ::close(fd_);
}

void File::parse()
{
    Cursor c(base_, size_);
    if (std::memcmp(base_, "GGUF", 4) != 0) fail("bad magic");
    c.skip(4);
    version_ = c.pod<uint32_t>();
    if (version_ < 2 || version_ > 3) fail("unsupported version " + std::to_string(version_));
    const uint64_t n_tensors = c.pod<uint64_t>();
    const uint64_t n_meta = c.pod<uint64_t>();
    if (n_tensors > (1ull << 24) || n_meta > (1ull << 24)) fail("implausible header counts");

    for (uint64_t k = 0; k < n_meta; ++k) {
        std::string key = c.str();
        const uint32_t type = c.pod<uint32_t>();
        Value v;
        read_value(c, type, v, 0);
        if (key == "general.alignment") {
            alignment_ = v.as_u64();
            if (alignment_ == 0 || (alignment_ & (alignment_ - 1))) fail("alignment must be a power of two");
        }
        meta_[std::move(key)] = std::move(v);
    }

    tensors_.reserve(size_t(n_tensors));
    for (uint64_t k = 0; k < n_tensors; ++k) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.pod<uint32_t>();
        if (nd == 0 || nd > 4) fail("tensor " + t.name + ": unsupported rank " + std::to_string(nd));
        for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.pod<uint64_t>());
        t.type = c.pod<uint32_t>();
        t.offset = c.pod<uint64_t>();
        tensors_.push_back(std::move(t));
    }
    data_offset_ = align_up(c.pos(), alignment_);
}

void File::validate()
{
    // every tensor: supported type, whole rows, inside the file, aligned,
    // and no two tensors overlap
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    std::map<std::string, int> seen;
    for (Tensor& t : tensors_) {
        if (seen[t.name]++) fail("duplicate tensor " + t.name);
        t.row_bytes = row_bytes(t.type, t.dims[0]);
        t.rows = 1;
        for (size_t d = 1; d < t.dims.size(); ++d) t.rows = mul_checked(t.rows, t.dims[d]);
        t.nbytes = mul_checked(t.row_bytes, t.rows);
        if (t.offset % alignment_) fail("tensor " + t.name + " is not aligned");
        const uint64_t start = data_offset_ + t.offset;
        if (start < data_offset_ || start > size_ || t.nbytes > size_ - start)
            fail("tensor " + t.name + " extends past the end of the file");
        t.data = base_ + start;
        spans.emplace_back(start, start + t.nbytes);
    }
    std::sort(spans.begin(), spans.end());
    for (size_t k = 1; k < spans.size(); ++k)
        if (spans[k].first < spans[k - 1].second) fail("tensor data regions overlap");
}

const Value* File::find_value(const std::string& key) const
{
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const Tensor* File::find_tensor(const std::string& name) const
{
    for (const Tensor& t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}

}  // namespace arcllm::gguf
