// evk::ai, HIP edition: fp16 tensors on one MI355X and the AI hot-path ops
// (matmul, flash attention forward/backward, single-query decode attention,
// and the decode-step elementwise ops), implemented in libevk.so over the
// C ABI of evkhip.h (hand-written gfx950 kernels in libevkhip.so).
//
// Mirrors /root/reference/evk_ai.h: float16_t (:18-159), Shape (:161-219),
// GradStats (:221-235), Tensor (:242-472) and the evk::ai declarations
// (:474-611) that lie on the hot path.  Extensions, all trailing and
// defaulted so every reference call site compiles unchanged:
//   * flash_attention / flash_attention_bwd: `bool causal`, `Tensor* lse`
//   * rope: `uint32_t position_offset`, `uint32_t head_dim`
//   * single_query_attention: the host entry the reference's
//     single_query_attention.comp never had
// Errors: the reference asserts (evk_ai.cpp) and exits; here every op checks
// the C ABI's status and, on failure, prints the library's message and aborts.
#pragma once

#include <evk.h>

#include <algorithm>
#include <cassert>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <memory>
#include <vector>

namespace evk::ai {
evk::Cmd& GetCmd();
uint64_t SubmitCmd(bool wait = true);
}  // namespace evk::ai

// IEEE binary16 storage with the reference's host conversions
// (evk_ai.h:52-158): fp32 -> fp16 rounds to nearest even for normals,
// rounds half-up (no sticky bits) into the subnormal range and flushes
// |x| < 2^-24 to zero; fp16 -> fp32 is exact.  Token ids reuse `value` as a
// raw uint16.
struct float16_t {
    uint16_t value;

    float16_t() = default;
    float16_t(float f) { value = float_to_float16(f); }
    float16_t(const float16_t& other) = default;
    float16_t& operator=(const float16_t& other) = default;
    operator float() const { return float16_to_float(value); }

    float16_t& operator+=(const float16_t& other) {
        *this = float16_t(float(*this) + float(other));
        return *this;
    }
    float16_t& operator/=(const float16_t& other) {
        *this = float16_t(float(*this) / float(other));
        return *this;
    }

    static uint16_t float_to_float16(float f) {
        uint32_t x;
        std::memcpy(&x, &f, 4);
        const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
        const uint32_t biased = (x >> 23) & 0xFFu;
        const uint32_t frac = x & 0x7FFFFFu;
        if (biased == 0xFFu) {  // inf / nan (payload kept, never turned into inf)
            if (frac == 0) return sign | 0x7C00u;
            const uint32_t p = (frac >> 13) & 0x3FFu;
            return uint16_t(sign | 0x7C00u | (p ? p : 1u));
        }
        const int e = int(biased) - 127;
        if (e > 15) return sign | 0x7C00u;
        if (e >= -14) {  // normal: round to nearest even on the 13 dropped bits
            uint32_t h = (uint32_t(e + 15) << 10) | (frac >> 13);
            const uint32_t dropped = frac & 0x1FFFu;
            if (dropped > 0x1000u || (dropped == 0x1000u && (h & 1u))) ++h;  // carries into the exponent
            return uint16_t(sign | (h >= 0x7C00u ? 0x7C00u : h));
        }
        if (e < -24) return sign;
        // subnormal: shift the implicit-one significand, add the first dropped bit
        const uint32_t sig = frac | 0x800000u;
        const int sh = 13 + (-14 - e);
        const uint32_t m = (sig >> sh) + ((sig >> (sh - 1)) & 1u);
        return uint16_t(sign | (m & 0x3FFu));
    }

    static float float16_to_float(uint16_t h) {
        const uint32_t sign = uint32_t(h & 0x8000u) << 16;
        const uint32_t e = (h >> 10) & 0x1Fu;
        const uint32_t m = h & 0x3FFu;
        uint32_t x;
        if (e == 0x1Fu) {
            x = sign | 0x7F800000u | (m << 13);
        } else if (e != 0) {
            x = sign | ((e + 112u) << 23) | (m << 13);
        } else {
            const float v = float(m) * (1.0f / 16777216.0f);  // m * 2^-24, exact
            std::memcpy(&x, &v, 4);
            x |= sign;
        }
        float f;
        std::memcpy(&f, &x, 4);
        return f;
    }
};

// Up to 8 dimensions; operator[] accepts negative indices (from the back);
// batch_size(n) = product of every dimension except the last n
// (evk_ai.h:161-219).
struct Shape {
    static constexpr uint32_t MAX_DIMENSIONS = 8;
    uint32_t values[MAX_DIMENSIONS] = {};
    uint32_t size = 0;

    Shape() = default;
    Shape(std::initializer_list<uint32_t> dims) {
        assert(dims.size() <= MAX_DIMENSIONS);
        for (uint32_t d : dims) values[size++] = d;
    }

    uint32_t operator[](int index) const {
        const int i = index < 0 ? int(size) + index : index;
        assert(i >= 0 && i < int(size));
        return values[i];
    }
    uint32_t rank() const { return size; }
    uint32_t number_of_elements(uint32_t index = 0) const {
        assert(index < size);
        uint32_t n = 1;
        for (uint32_t i = index; i < size; ++i) n *= values[i];
        return n;
    }
    uint32_t count() const {
        uint32_t n = 1;
        for (uint32_t i = 0; i < size; ++i) n *= values[i];
        return n;
    }
    uint32_t batch_size(uint32_t element_count) const {
        assert(element_count <= size);
        uint32_t n = 1;
        for (uint32_t i = 0; i + element_count < size; ++i) n *= values[i];
        return n;
    }
};

struct GradStats {
    float min_val = 1e9f;
    float max_val = -1e9f;
    float mean = 0.0f;
    float rms = 0.0f;
    uint32_t nan_count = 0;
    uint32_t inf_count = 0;
    uint32_t zero_count = 0;

    void print(const char* name) const {
        std::printf("    %s: min=%.6f, max=%.6f, mean=%.6f, rms=%.6f, nan=%u, inf=%u, zero=%u\n", name,
                    min_val, max_val, mean, rms, nan_count, inf_count, zero_count);
    }
};

enum class VarianceScaleMode {
    FanIn,
    FanOut,
    FanAverage,
};

// An fp16 tensor in HBM (`buffer`, shape.count()*2 bytes) with a lazily
// created pinned host mirror (`cpu_buffer`).  cpu_upload/cpu_download enqueue
// a copy on the library stream and, by default, submit and wait
// (evk_ai.h:279-294).
struct Tensor {
    evk::Buffer buffer;
    evk::Buffer cpu_buffer;
    std::unique_ptr<Tensor> grad_tensor;
    Shape shape = {};

    std::function<void()> forward_fn;
    std::function<void()> backward_fn;

    Tensor() = default;
    Tensor(const Shape& s) : shape(s) {
        buffer = evk::CreateBuffer({
            .size = uint64_t(s.count()) * sizeof(float16_t),
            .usage = evk::BufferUsage::Storage,
        });
    }

    static Tensor alias(const Shape& s, const evk::Buffer& existing) {
        Tensor t;
        t.shape = s;
        t.buffer = existing;
        return t;
    }

    Tensor& grad() {
        if (!grad_tensor) grad_tensor = std::make_unique<Tensor>(shape);
        return *grad_tensor;
    }

    // Device address of the fp16 data (what the kernels read and write).
    void* device_ptr() { return reinterpret_cast<void*>(buffer.GetReference()); }

    float16_t* cpu() {
        if (!cpu_buffer) {
            cpu_buffer = evk::CreateBuffer({
                .size = uint64_t(shape.count()) * sizeof(float16_t),
                .usage = evk::BufferUsage::TransferDst | evk::BufferUsage::TransferSrc,
                .memoryType = evk::MemoryType::CPU,
            });
        }
        return static_cast<float16_t*>(cpu_buffer.GetPtr());
    }
    void cpu_upload(bool submit = true) {
        cpu();
        evk::ai::GetCmd().copy(cpu_buffer, buffer, uint64_t(shape.count()) * sizeof(float16_t));
        if (submit) evk::ai::SubmitCmd(true);
    }
    void cpu_download(bool submit = true) {
        cpu();
        evk::ai::GetCmd().copy(buffer, cpu_buffer, uint64_t(shape.count()) * sizeof(float16_t));
        if (submit) evk::ai::SubmitCmd(true);
    }

    // Flat index i is on the diagonal when i % (shape[0]+1) == 0
    // (evk_ai.h:306-313: an identity for square matrices).
    Tensor& identity(float16_t val = float16_t(1.0f)) {
        float16_t* h = cpu();
        const uint32_t n = shape.count(), stride = shape[0] + 1;
        for (uint32_t i = 0; i < n; ++i) h[i] = (i % stride == 0) ? val : float16_t(0.0f);
        cpu_upload();
        return *this;
    }
    // Uniform [0,1] from the platform rand() (evk_ai.h:314-320).
    Tensor& random(float16_t = float16_t(0.0f)) {
        float16_t* h = cpu();
        for (uint32_t i = 0; i < shape.count(); ++i) h[i] = float16_t(float(std::rand()) / float(RAND_MAX));
        cpu_upload();
        return *this;
    }
    Tensor& fill(float16_t val = float16_t(0.0f)) {
        float16_t* h = cpu();
        std::fill(h, h + shape.count(), val);
        cpu_upload();
        return *this;
    }
    // N(0, stddev^2) by Box-Muller over the platform rand() (evk_ai.h:326-344).
    Tensor& random_init(float stddev = 0.1f) {
        float16_t* h = cpu();
        for (uint32_t i = 0; i < shape.count(); ++i) {
            const float u1 = float(std::rand() + 1) / float(RAND_MAX + 1.0);
            const float u2 = float(std::rand()) / float(RAND_MAX);
            h[i] = float16_t(stddev * std::sqrt(-2.0f * std::log(u1)) * std::cos(6.28318531f * u2));
        }
        cpu_upload();
        return *this;
    }

    float16_t item() {
        assert(shape.count() == 1);
        cpu_download();
        return cpu()[0];
    }

    void print(uint32_t max_elements = 8, uint32_t max_batch = 4) {
        std::printf("Tensor (");
        for (uint32_t i = 0; i < shape.rank(); ++i) std::printf(i ? ", %u" : "%u", shape[int(i)]);
        std::printf("):\n");
        cpu_download();
        const float16_t* h = cpu();
        auto row = [&](const float16_t* r, uint32_t n) {
            std::printf("[");
            for (uint32_t c = 0; c < std::min(n, max_elements); ++c) std::printf(c ? ", %g" : "%g", float(r[c]));
            if (n > max_elements) std::printf(", ...");
            std::printf("]");
        };
        if (shape.rank() < 2) {
            row(h, shape.count());
            std::printf("\n");
            return;
        }
        const uint32_t rows = shape[-2], cols = shape[-1], batch = shape.batch_size(2);
        for (uint32_t b = 0; b < std::min(batch, max_batch); ++b) {
            std::printf(b ? ",\n[\n" : "[\n");
            for (uint32_t r = 0; r < std::min(rows, max_elements); ++r) {
                std::printf(r ? ",\n  " : "  ");
                row(h + (uint64_t(b) * rows + r) * cols, cols);
            }
            if (rows > max_elements) {
                std::printf(",\n  ...,\n  ");
                row(h + (uint64_t(b) * rows + rows - 1) * cols, cols);
            }
            std::printf("]");
        }
        std::printf(batch > max_batch ? ",\n...\n]\n" : "\n]\n");
    }

    GradStats stats() {
        cpu_download();
        const float16_t* h = cpu();
        GradStats s;
        double sum = 0.0, sq = 0.0;
        uint32_t valid = 0;
        for (uint32_t i = 0; i < shape.count(); ++i) {
            const float v = float(h[i]);
            if (std::isnan(v)) {
                ++s.nan_count;
            } else if (std::isinf(v)) {
                ++s.inf_count;
            } else {
                s.zero_count += (v == 0.0f);
                s.min_val = std::min(s.min_val, v);
                s.max_val = std::max(s.max_val, v);
                sum += v;
                sq += double(v) * v;
                ++valid;
            }
        }
        if (valid) {
            s.mean = float(sum / valid);
            s.rms = float(std::sqrt(sq / valid));
        }
        return s;
    }
};

namespace evk::ai {

// Brings up the evk runtime on HIP device 0 when InitializeEVK was not
// called, and the kernel library (evkhip_init).
void initialize();
// Releases the kernel library's workspace and the runtime.
void shutdown();

// C (+)= op(A) . op(B), fp32 accumulation, fp16 output (evk_ai.h:489-495).
// (...,M,N) = (...,M,K) . (...,K,N); transpose_a reads A stored (...,K,M),
// transpose_b reads B stored (...,N,K); an operand with batch 1 broadcasts.
// TILE_M/TILE_N are the reference's tile hints (multiples of 16): accepted,
// while the MFMA kernels choose their own tiling, so M, N and K need not be
// multiples of them.
void matmul(Tensor& a, Tensor& b, Tensor& c, bool transpose_a = false, bool transpose_b = false,
            bool acc_c = false, uint8_t TILE_M = 80u, uint8_t TILE_N = 80u);

// Multi-query flash attention forward (evk_ai.h:497-501).
// Q, O: (B, N, D), D = H*Dh; K, V: (B, N, Dh) shared by the H heads; scale
// 1/sqrt(Dh).  causal masks keys j > i.  lse, when given, receives the fp32
// log-sum-exp of each (b, h, i) row: B*H*N fp32 values, so its fp16 element
// count must be 2*B*H*N (e.g. shape (B, H, N, 2)).
void flash_attention(Tensor& q, Tensor& k, Tensor& v, Tensor& o, bool causal = false, Tensor* lse = nullptr);

// Backward (evk_ai.h:503): dQ (B,N,D); dK, dV (B,N,Dh) summed over heads.
// heads != 0 must equal D/Dh.  With lse from the forward pass the row
// statistics are not recomputed and D_i is taken as rowsum(dO_i * O_i).
void flash_attention_bwd(Tensor& q, Tensor& k, Tensor& v, Tensor& o, Tensor& dO, Tensor& dQ, Tensor& dK,
                         Tensor& dV, uint32_t heads = 0, bool causal = false, Tensor* lse = nullptr);

// Decode-step attention of one query over a KV cache:
// out[h] = softmax(q[h] . K[0:L, h]^T / sqrt(dh)) . V[0:L, h]
// q, out: (heads*dh); k_cache, v_cache: (max_len, heads*dh) row-major.
void single_query_attention(Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& out,
                            uint32_t current_length, uint32_t heads = 1);

// c = a + b (evk_ai.h:521).
void add(Tensor& a, Tensor& b, Tensor& c);

// out = 0.5 x (1 + tanh(0.79788456 (x + 0.044715 x^3))) (evk_ai.h:540).
void gelu(Tensor& in, Tensor& out);

// out[i] = embeddings[indices[i]], indices raw uint16 (evk_ai.h:552-558).
void embed(Tensor& embeddings, Tensor& indices, Tensor& out);

// argmax over logits[b, position, token_base : token_base+token_count]
// written as raw uint16 (evk_ai.h:560-566).
void greedy_sample(Tensor& logits, Tensor& out_tokens, uint32_t position, uint16_t token_base,
                   uint16_t token_count);

// Rotary encoding of interleaved pairs over the last dimension
// (evk_ai.h:585-591).  position_offset shifts t; head_dim > 0 rotates each
// head_dim-wide slice independently.
void rope(Tensor& input, Tensor& out, uint32_t batch_size, uint32_t seq_len, uint32_t embed_dim,
          float rotary_base = 10000.0f, uint32_t position_offset = 0, uint32_t head_dim = 0);

// out = x / sqrt(mean(x^2) + eps) over the last dimension (evk_ai.h:605-610).
void rms_norm(Tensor& input, Tensor& output, float eps = 1e-4f);

// tensor = 0 (evk_ai.h:602).
void zero(Tensor& tensor);

}  // namespace evk::ai
