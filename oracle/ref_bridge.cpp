// Bridge that exposes a few CPU routines of the reference (carloshgsilva/evk)
// to the oracle tests.  TEST INFRASTRUCTURE ONLY: it is compiled by
// oracle/Makefile straight from the reference's own headers where they lie
// (/root/reference/evk_ai.h, /root/reference/example/tests.h) into
// oracle/_ref/libevkref.so, which is never shipped or linked by the product.
//
// Exposed (reference file:line):
//   float16_t::float_to_float16 / float16_to_float   evk_ai.h:52-158
//   cpu_matmul_nn / cpu_matmul_tn                     example/tests.h:52-86
//   gelu_approx_cpu                                   example/tests.h:9-15
// tests.h also defines GPU test functions; they are hidden and unreferenced,
// so --gc-sections drops them together with their references to evk::ai.
// evk.h uses std::memcpy without including <cstring> (MSVC pulls it in
// transitively); the standard header is included first for g++.
#include <cstring>
#include <evk_ai.h>
#include <example/tests.h>

#define REF_EXPORT extern "C" __attribute__((visibility("default")))

REF_EXPORT uint16_t ref_f32_to_f16(float f) { return float16_t::float_to_float16(f); }
REF_EXPORT float ref_f16_to_f32(uint16_t h) { return float16_t::float16_to_float(h); }
// Bit pattern of the conversion (keeps signalling-NaN payloads intact).
REF_EXPORT uint32_t ref_f16_to_f32_bits(uint16_t h) {
    float f = float16_t::float16_to_float(h);
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

REF_EXPORT void ref_cpu_matmul_nn(const float* a, const float* b, float* c,
                                  uint32_t rows, uint32_t inner, uint32_t cols) {
    std::vector<float> av(a, a + size_t(rows) * inner), bv(b, b + size_t(inner) * cols), cv;
    cpu_matmul_nn(av, bv, cv, rows, inner, cols);
    std::copy(cv.begin(), cv.end(), c);
}

REF_EXPORT void ref_cpu_matmul_tn(const float* a, const float* b, float* c,
                                  uint32_t rows, uint32_t inner, uint32_t cols) {
    std::vector<float> av(a, a + size_t(rows) * inner), bv(b, b + size_t(rows) * cols), cv;
    cpu_matmul_tn(av, bv, cv, rows, inner, cols);
    std::copy(cv.begin(), cv.end(), c);
}

REF_EXPORT float ref_gelu(float x) { return gelu_approx_cpu(x); }
