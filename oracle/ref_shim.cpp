// ref_shim.cpp -- extern "C" entry points over the reference's own portable,
// header-only CPU code, so tests can pin the oracle against it.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/ with the
// reference headers taken from where they lie in the reference tree
// (-I <reference>/src); nothing from the reference is copied here.  Wrapped:
//   src/q6cb_q6_reference.hpp       half_to_float :20-36, decode_q6_element :49-91,
//                                   arm_r64 :118-132, arm_s32 :134-148, arm_t32_cpu :160-175
//   src/q6cb_fixture_generator.hpp  generate_fixture :160-192, verify_semantic_invariant :196-228
//   src/q4_down_exec148_materializer.h  validator_source_tuple, materialize_block, Sha256
#include "q6cb_q6_reference.hpp"
#include "q6cb_fixture_generator.hpp"
#include "q4_down_exec148_materializer.h"

#include <cstdint>
#include <cstring>
#include <exception>

extern "C" {

float ref_half_to_float(uint16_t h) { return q6cb::half_to_float(h); }

// Decode all 256 elements of one Q6_K block.
void ref_q6_decode_block(const uint8_t* blk, int32_t* q, int32_t* scale, float* value)
{
    for (uint32_t k = 0; k < 256; ++k) {
        const q6cb::CanonicalQ6Element e = q6cb::decode_q6_element(blk, k);
        q[k] = e.q;
        scale[k] = e.scale;
        value[k] = e.value;
    }
}

// The reference's Q6CB fixture generator.  Returns 0 on success, -1 if the
// reference rejects the spec.
int ref_q6_fixture(uint32_t n, uint32_t rows, uint64_t seed, int stratum,
                   uint8_t* packed, float* x, int8_t* expected_q, int8_t* expected_scale)
{
    try {
        q6cb::FixtureSpec s;
        s.id = "golden";
        s.n = n;
        s.rows = rows;
        s.seed = seed;
        s.stratum = static_cast<q6cb::ConditioningStratum>(stratum);
        const q6cb::Fixture f = q6cb::generate_fixture(s);
        std::memcpy(packed, f.packed.data(), f.packed.size());
        std::memcpy(x, f.x.data(), f.x.size() * sizeof(float));
        std::memcpy(expected_q, f.expected_q.data(), f.expected_q.size());
        std::memcpy(expected_scale, f.expected_scale.data(), f.expected_scale.size());
        const q6cb::SemanticInvariant inv = q6cb::verify_semantic_invariant(f);
        return inv.pass ? 0 : -2;
    } catch (const std::exception&) {
        return -1;
    }
}

// R64 / S32 / T32 GEMV arms of the reference over a packed Q6_K tensor.
int ref_q6_arms(const uint8_t* packed, size_t packed_bytes, uint32_t n, uint32_t rows,
                const float* x, double* r64, float* s32, float* t32)
{
    try {
        std::vector<uint8_t> p(packed, packed + packed_bytes);
        const std::vector<float> ex = q6cb::expand_q6_rows(p, n, rows);
        const std::vector<float> xv(x, x + n);
        const std::vector<double> a = q6cb::arm_r64(ex, xv, n, rows);
        const std::vector<float> b = q6cb::arm_s32(ex, xv, n, rows);
        const std::vector<float> c = q6cb::arm_t32_cpu(ex, xv, n, rows);
        std::memcpy(r64, a.data(), a.size() * sizeof(double));
        std::memcpy(s32, b.data(), b.size() * sizeof(float));
        std::memcpy(t32, c.data(), c.size() * sizeof(float));
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Canonical 276-byte tuple of a Q4_K block: d,dmin bytes; (sc,mn) x 8; 256 codes.
void ref_q4_source_tuple(const uint8_t* blk, uint8_t* out276)
{
    std::array<uint8_t, arcllm_exec148::kCanonicalBytes> t{};
    arcllm_exec148::validator_source_tuple(blk, t);
    std::memcpy(out276, t.data(), t.size());
}

void ref_exec148_materialize_block(const uint8_t* src144, uint8_t* dst148)
{
    arcllm_exec148::materialize_block(src144, dst148);
}

void ref_sha256(const uint8_t* p, size_t n, uint8_t* out32)
{
    arcllm_exec148::Sha256 h;
    h.update(p, n);
    const std::array<uint8_t, 32> d = h.final();
    std::memcpy(out32, d.data(), 32);
}

} // extern "C"
