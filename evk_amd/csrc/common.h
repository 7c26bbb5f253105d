// Shared definitions for the gfx950 kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "../../include/evkhip.h"

typedef _Float16 f16;
typedef f16 half8 __attribute__((ext_vector_type(8)));
typedef f16 half4 __attribute__((ext_vector_type(4)));
typedef f16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DEV __device__ __forceinline__

// ---------------------------------------------------------------------------
// Error reporting (host)
// ---------------------------------------------------------------------------
namespace evkhip {
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
hipStream_t as_stream(void* s);
int device_cu_count();
}  // namespace evkhip

#define EVK_RETURN_IF(cond, code, ...)                  \
    do {                                                \
        if (cond) return evkhip::set_error(code, __VA_ARGS__); \
    } while (0)

#define EVK_HIP(expr)                                                   \
    do {                                                                \
        hipError_t _e = (expr);                                         \
        if (_e != hipSuccess) return evkhip::check_hip(_e, #expr);      \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
// v_mfma_f32_32x32x16_f16: D(32x32) = A(32x16) B(16x32) + C, wave64.
// Operand lane l holds 8 halves of row (A) / column (B) l%32 for k-group
// l/32; the k mapping is the same for A and B, so callers only rely on:
//   A: row = l%32, B: col = l%32, both with the same (l/32, slot) -> k.
//   D: element j of lane l is row 8*(j/4) + 4*(l/32) + (j%4), col l%32.
DEV floatx16 mfma32(const half8& a, const half8& b, const floatx16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

DEV uint32_t pack_h2(float lo, float hi) {
    half2_t v = {(f16)lo, (f16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

DEV half8 as_half8(const u32x4& v) { return __builtin_bit_cast(half8, v); }
DEV u32x4 as_u32x4(const half8& v) { return __builtin_bit_cast(u32x4, v); }

// Byte permute: result bytes chosen from {hi:lo} (v_perm_b32).
DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// (lo half of x) | (lo half of y) << 16
DEV uint32_t pack_lo(uint32_t x, uint32_t y) { return perm_b32(y, x, 0x05040100u); }
// (hi half of x) | (hi half of y) << 16
DEV uint32_t pack_hi(uint32_t x, uint32_t y) { return perm_b32(y, x, 0x07060302u); }

// Transpose an 8x8 block of halves held as 8 rows of 16 bytes.
// in[r] holds elements (r, 0..7); out[c] receives elements (0..7, c).
DEV void transpose8x8(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {  // column pair (2*c2, 2*c2+1) lives in dword c2
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int r2 = 0; r2 < 4; ++r2) {
            uint32_t x = in[2 * r2][c2], y = in[2 * r2 + 1][c2];
            lo[r2] = pack_lo(x, y);  // column 2*c2, rows 2r2, 2r2+1
            hi[r2] = pack_hi(x, y);  // column 2*c2+1
        }
        out[2 * c2] = u32x4{lo[0], lo[1], lo[2], lo[3]};
        out[2 * c2 + 1] = u32x4{hi[0], hi[1], hi[2], hi[3]};
    }
}

DEV floatx4 mfma16(const half8& a, const half8& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 over a row-major 16-bit LDS tile: in each group of 16
// lanes, lane i passes the address of row i / 4, columns 4 (i % 4) .. +3 of a
// 4-row x 16-column block and receives column i of the block (its 4 rows).
DEV half4 lds_read_tr(const f16* p) {
    fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (__attribute__((address_space(3))) fp16x4_t*)(p));
    return __builtin_bit_cast(half4, v);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <class F, int... S>
DEV void static_for_impl(F&& f, std::integer_sequence<int, S...>) {
    (f(std::integral_constant<int, S>{}), ...);
}
template <int N, class F>
DEV void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

DEV half8 cat4(const half4& a, const half4& b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Values handed between workgroups of one launch.  Every value handed over
// is written and read with an agent-scope atomic store / load; on gfx950
// those carry the sc1 cache policy: a store is written through to the
// device coherence point and the wave's vmcnt counts it done only once it
// is there, and a load is served from that point (never from a stale line
// of another XCD's L2).  arrive_last therefore orders the handoff in the
// hardware, without an agent-scope release/acquire fence pair:
//   1. every wave waits for its own stores to complete (s_waitcnt 0),
//   2. the workgroup meets at a barrier,
//   3. one thread increments the counter (an atomic at the coherence point,
//      issued after 1-2, so every handed-over store precedes it there),
//   4. the last arrival reads the values with agent-scope atomic loads.
// The formal fences are not used because they are costly here: an
// agent-scope release writes back the XCD's whole L2 (buffer_wbl2), and
// with one per workgroup the skinny GEMV (1376 workgroups) measured 175 us
// instead of 16 us on MI355X.
DEV void st_ag(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV float ld_ag(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void st_ag(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV uint32_t ld_ag(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// The last of `total` arrivals gets true and resets the counter for the
// next launch.
DEV bool arrive_last(unsigned* cnt, unsigned total) {
    __shared__ unsigned s_last;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev + 1 == total);
        if (s_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    return s_last;
}

// Raw buffer loads: a descriptor over [base, base + bytes); a 16-byte load
// at byte offset voff + soff past the end returns zeros.
DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
DEV float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}
DEV float buf_load_f16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return (float)__builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0));
}
// An offset no descriptor covers (descriptors span < 2^31 bytes): a load at
// it returns zeros, so predicated loads need no branch.
DEV uint32_t oob_or(bool ok, uint32_t off) { return ok ? off : 0x80000000u; }

DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// tanh GELU of gelu.comp (evk_ai.cpp:679-699)
DEV float gelu_f(float x) {
    const float ka = 0.7978845608028654f, kb = 0.044715f;
    float u = ka * (x + kb * x * x * x);
    return 0.5f * x * (1.0f + tanhf(u));
}

// greedy_sample.comp's winner is the maximum under the total order
// (value desc, bitrev8(j mod 256) asc, j asc); rank encodes the last two.
DEV uint32_t greedy_rank(uint32_t j) {
    return ((__builtin_bitreverse32(j & 255u) >> 24) << 16) | (j >> 8);
}
DEV uint32_t greedy_index(uint32_t rank) {
    return ((rank & 0xFFFFu) << 8) | (__builtin_bitreverse32(rank >> 16) >> 24);
}
DEV bool greedy_better(float va, uint32_t ra, float vb, uint32_t rb) {
    return va > vb || (va == vb && ra < rb);
}

DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }

// ---------------------------------------------------------------------------
// Host-side tensor helpers
// ---------------------------------------------------------------------------
namespace evkhip {
inline uint64_t numel(const evkhip_tensor* t) {
    uint64_t n = 1;
    for (uint32_t i = 0; i < t->rank; ++i) n *= t->dims[i];
    return n;
}
inline uint32_t dim_at(const evkhip_tensor* t, int i) {  // negative = from the end
    return t->dims[i < 0 ? (int)t->rank + i : i];
}
inline uint64_t batch_of(const evkhip_tensor* t, uint32_t inner) {  // Shape::batch_size
    uint64_t b = 1;
    for (uint32_t i = 0; i + inner < t->rank; ++i) b *= t->dims[i];
    return b;
}
int check_tensor(const evkhip_tensor* t, const char* name, uint32_t min_rank, uint32_t max_rank);
bool aligned16(const void* p);
}  // namespace evkhip
