// arc_synth.cpp -- deterministic host-side generators for seeded synthetic
// packed Q4_K/Q6_K tensors and normal vectors (random-init weights for the
// synthetic model and the benchmarks; no GPU involved).
//
// Counter-based: super-block b of (seed, stream) draws from
// splitmix64(mix(seed, stream, b)), element i of a normal vector from
// mix(seed, stream, i), so slices can be generated in parallel or alone and
// always reproduce the same bytes.
#include "../../include/arcllm_hip.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace arc {
int set_error(int code, const char* fmt, ...);

namespace {

inline uint64_t splitmix64(uint64_t& x)
{
    uint64_t z = (x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t mix3(uint64_t seed, uint64_t stream, uint64_t idx)
{
    uint64_t s = seed ^ 0x6172636c6c6d3335ull;
    uint64_t a = splitmix64(s) ^ stream;
    uint64_t b = splitmix64(a) ^ idx;
    return splitmix64(b);
}

// Standard normal from two 53-bit uniforms (Box-Muller, cosine branch).
inline double normal(uint64_t& st)
{
    const double u1 = (double((splitmix64(st) >> 11)) + 1.0) * (1.0 / 9007199254740992.0);  // (0, 1]
    const double u2 = double(splitmix64(st) >> 11) * (1.0 / 9007199254740992.0);            // [0, 1)
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925 * u2);
}

inline uint16_t f16_bits(float f)
{
    const _Float16 h = static_cast<_Float16>(f);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

template <class F>
void parallel_for(uint64_t n, F&& f)
{
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < 4096) nt = 1;
    std::vector<std::thread> th;
    const uint64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const uint64_t b = t * chunk, e = b + chunk < n ? b + chunk : n;
        if (b >= e) break;
        th.emplace_back([=, &f] {
            for (uint64_t i = b; i < e; ++i) f(i);
        });
    }
    for (auto& t : th) t.join();
}

}  // namespace
}  // namespace arc

using namespace arc;

extern "C" int arc_synth_packed(int qtype, uint64_t seed, uint64_t stream, uint32_t rows, uint32_t K, float d_sigma,
                                float dmin_sigma, void* out)
{
    if (!out) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    if (qtype != ARC_Q4_K && qtype != ARC_Q6_K) return set_error(ARC_ERR_UNSUPPORTED, "unsupported qtype %d", qtype);
    if (rows == 0 || K == 0 || K % 256u) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad shape");
    const uint64_t blocks = uint64_t(rows) * (K / 256u);
    uint8_t* o = static_cast<uint8_t*>(out);
    if (qtype == ARC_Q4_K) {
        parallel_for(blocks, [=](uint64_t b) {
            uint64_t st = mix3(seed, stream, b);
            uint8_t* p = o + b * 144u;
            const uint16_t d = f16_bits(float(std::fabs(normal(st) * d_sigma)));
            const uint16_t dm = f16_bits(float(std::fabs(normal(st) * dmin_sigma)));
            p[0] = uint8_t(d);
            p[1] = uint8_t(d >> 8);
            p[2] = uint8_t(dm);
            p[3] = uint8_t(dm >> 8);
            for (int i = 4; i < 144; i += 8) {
                const uint64_t r = splitmix64(st);
                std::memcpy(p + i, &r, (144 - i) < 8 ? size_t(144 - i) : size_t(8));
            }
        });
    } else {
        parallel_for(blocks, [=](uint64_t b) {
            uint64_t st = mix3(seed, stream, b);
            uint8_t* p = o + b * 210u;
            for (int i = 0; i < 192; i += 8) {
                const uint64_t r = splitmix64(st);
                std::memcpy(p + i, &r, 8);
            }
            const uint64_t r0 = splitmix64(st), r1 = splitmix64(st);
            for (int i = 0; i < 16; ++i) {
                const uint64_t r = i < 8 ? r0 : r1;
                const int v = int((r >> (8 * (i & 7))) & 63u) - 32;  // uniform in [-32, 31]
                p[192 + i] = uint8_t(int8_t(v));
            }
            const uint16_t d = f16_bits(float(std::fabs(normal(st) * d_sigma)));
            p[208] = uint8_t(d);
            p[209] = uint8_t(d >> 8);
        });
    }
    (void)dmin_sigma;
    return ARC_OK;
}

extern "C" int arc_synth_normal(uint64_t seed, uint64_t stream, size_t n, float mean, float sigma, float* out)
{
    if (!out && n) return set_error(ARC_ERR_INVALID_ARGUMENT, "null output");
    parallel_for(n, [=](uint64_t i) {
        uint64_t st = mix3(seed, stream ^ 0x4e4f524dull, i);
        out[i] = float(double(mean) + double(sigma) * normal(st));
    });
    return ARC_OK;
}
