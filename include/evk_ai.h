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
#include <unordered_map>
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
// Whether the flash kernels for this head size run on the matrix cores (no
// reference counterpart: the reference's shader has one code path).
bool flash_has_mfma(uint32_t head_dim);

// Backward (evk_ai.h:503): dQ (B,N,D); dK, dV (B,N,Dh) summed over heads.
// heads != 0 must equal D/Dh.  With lse from the forward pass the row
// statistics are not recomputed and D_i is taken as rowsum(dO_i * O_i).
void flash_attention_bwd(Tensor& q, Tensor& k, Tensor& v, Tensor& o, Tensor& dO, Tensor& dQ, Tensor& dK,
                         Tensor& dV, uint32_t heads = 0, bool causal = false, Tensor* lse = nullptr);

// Decode-step attention of one query over a KV cache:
// out[h] = softmax(q[h] . K[0:L, h]^T / sqrt(dh)) . V[0:L, h]
// q, out: (heads*dh); k_cache, v_cache: (max_len, heads*dh) row-major.
// Batched: k_cache, v_cache (B, max_len, heads*dh) with B > 1 and q, out
// (B, heads*dh) or (B, 1, heads*dh): sequence b attends over its own cache.
void single_query_attention(Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& out,
                            uint32_t current_length, uint32_t heads = 1);

// KV-cache append: rows [pos0, pos0+n) of each sequence's cache
// (B, max_seq, D) take the rows of src (B, n, D).
void kv_cache_write(Tensor& src, Tensor& cache, uint32_t pos0);

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

// ---- training ops (evk_ai.h:476-614).  *_backward ops accumulate into
// their grad_in, as the reference's shaders do. ----

// Adam state of one parameter tensor (evk_ai.h:476-487): fp16 first moment
// divided by the RMS of the second moment, and log2 of that RMS plus 41
// (0 meaning RMS 0); t counts the steps taken.
struct AdamState {
    evk::Buffer m_buffer;
    evk::Buffer v_buffer;
    uint32_t t = 0;

    void init(uint32_t num_elements);  // zeroed state, t = 0
    void reset();                      // releases the state
};

// result[0] = mean((predicted - target)^2); predGrad = 2 (predicted - target) / n
// (evk_ai.h:505-507).
void mse_loss(Tensor& predicted, Tensor& target, Tensor& predGrad, Tensor& result);

// param -= learning_rate * gradient (evk_ai.h:509-510).
void sgd(Tensor& param, Tensor& gradient, float learning_rate);

// One Adam step; the state is created on first use and t advances by one
// (evk_ai.h:512-518).
void adam(Tensor& param, Tensor& gradient, AdamState& state, float learning_rate = 0.001f, float beta1 = 0.9f,
          float beta2 = 0.999f, float epsilon = 1e-4f);

// Softmax over the last dimension of in * input_scale; entries <= -65504 are
// masked to probability 0 (evk_ai.h:523-525).
void softmax(Tensor& in, Tensor& out, float input_scale = 1.0f);

// grad_in += probs * (grad_out - dot(grad_out, probs)) * scale_factor per row
// (evk_ai.h:527-529).
void softmax_backward(Tensor& probs, Tensor& grad_out, Tensor& grad_in, float scale_factor = 1.0f);

// out = max(0, in); grad_in += (in > 0 ? grad_out : 0) (evk_ai.h:531-536).
void relu(Tensor& in, Tensor& out);
void relu_backward(Tensor& grad_out, Tensor& in, Tensor& grad_in);

// grad_in += grad_out * gelu'(in) (evk_ai.h:542-543).
void gelu_backward(Tensor& grad_out, Tensor& in, Tensor& grad_in);

// logits (B*N, V), targets (B*N) raw uint16 (0 = ignore): grad = (softmax -
// one_hot) / n_valid, zero rows for ignored targets; result[0] = mean loss
// over the valid rows (evk_ai.h:545-552).
void cross_entropy_loss(Tensor& logits, Tensor& targets, Tensor& grad, Tensor& result);

// grad_embeddings[indices[i]] += grad_out[i] (evk_ai.h:568-572).
void embed_backward(Tensor& grad_out, Tensor& indices, Tensor& grad_embeddings);

// scores (..., N, N): entries j > i set to -65504 (evk_ai.h:574-577).
void apply_causal_mask(Tensor& scores);

// out = input + pos_emb broadcast over the batch; backward: grad_input +=
// grad_out, grad_pos += sum over the batch (evk_ai.h:579-585).
void position_add(Tensor& input, Tensor& pos_emb, Tensor& out, uint32_t batch_size, uint32_t seq_len,
                  uint32_t embed_dim);
void position_add_backward(Tensor& grad_out, Tensor& grad_input, Tensor& grad_pos, uint32_t batch_size,
                           uint32_t seq_len, uint32_t embed_dim);

// grad_input += the transposed rotation of grad_out (evk_ai.h:593-596).
void rope_backward(Tensor& grad_out, Tensor& grad_input, uint32_t batch_size, uint32_t seq_len,
                   uint32_t embed_dim, float rotary_base = 10000.0f);

// tensor *= scale_factor in place (evk_ai.h:598-599).
void scale(Tensor& tensor, float scale_factor);

// output[i] += sum_b input[b * size_per_batch + i] (evk_ai.h:604-605).
void sum_batch(Tensor& input, Tensor& output, uint32_t batch_count, uint32_t size_per_batch);

// grad_input += (g - y dot(g, y) / D) / rms per row (evk_ai.h:612-614).
void rms_norm_backward(Tensor& input, Tensor& grad_out, Tensor& grad_input, float eps = 1e-4f);

}  // namespace evk::ai

// A define-by-run graph with reverse-mode gradients (evk_ai.h:616-1074).
// Ops append nodes whose forward_fn / backward_fn record work on the
// library stream; eval() runs them in order (and the backward functions in
// reverse), step()/step_adam() update the parameters.  Gradient buffers
// accumulate, and eval(true) zeroes them first, as in the reference.
// causal_attention runs the fused causal flash attention (forward with the
// saved log-sum-exp, backward from it) instead of materialising the N x N
// scores and probabilities; a non-default scale takes the unfused
// matmul / mask / softmax / matmul chain.
struct Graph {
    std::vector<std::unique_ptr<Tensor>> nodes;
    std::vector<Tensor*> params;
    std::unordered_map<Tensor*, evk::ai::AdamState> adam_states;
    std::unique_ptr<Tensor> scratch;

    Tensor& get_scratch(const Shape& shape) {
        if (!scratch || scratch->shape.count() < shape.count()) {
            scratch = std::make_unique<Tensor>(shape);
        } else {
            scratch->shape = shape;
        }
        return *scratch;
    }

    Tensor& tensor(Shape shape, bool param = false) {
        Tensor& t = node(shape);
        if (param) params.push_back(&t);
        return t;
    }

    // Same elements under another shape (a copy of the buffer each eval).
    Tensor& view(Tensor& a, Shape new_shape) {
        assert(a.shape.count() == new_shape.count() && "view requires the same number of elements");
        Tensor& out = node(new_shape);
        const uint64_t bytes = uint64_t(a.shape.count()) * sizeof(float16_t);
        out.forward_fn = [&a, &out, bytes]() { evk::ai::GetCmd().copy(a.buffer, out.buffer, bytes); };
        out.backward_fn = [&a, &out, bytes]() { evk::ai::GetCmd().copy(out.grad().buffer, a.grad().buffer, bytes); };
        return out;
    }

    // (M,K)@(K,N), (B,M,K)@(K,N), (M,K)@(B,K,N) and (B,M,K)@(B,K,N).
    Tensor& matmul(Tensor& a, Tensor& b, uint8_t tile_m = 16, uint8_t tile_n = 16) {
        const uint32_t ra = a.shape.rank(), rb = b.shape.rank();
        Shape out_shape;
        if (ra == 2 && rb == 2) {
            out_shape = Shape({a.shape[0], b.shape[1]});
        } else if (ra == 3 && rb == 2) {
            out_shape = Shape({a.shape[0], a.shape[1], b.shape[1]});
        } else if (ra == 2 && rb == 3) {
            out_shape = Shape({b.shape[0], a.shape[0], b.shape[2]});
        } else if (ra == 3 && rb == 3) {
            out_shape = Shape({a.shape[0], a.shape[1], b.shape[2]});
        } else {
            assert(false && "Graph::matmul: unsupported ranks");
        }
        Tensor& c = node(out_shape);
        c.forward_fn = [&a, &b, &c, tile_m, tile_n]() {
            evk::ai::matmul(a, b, c, false, false, false, tile_m, tile_n);
        };
        c.backward_fn = [this, &a, &b, &c, tile_m, tile_n]() {
            // dA += dC B^T
            evk::ai::matmul(c.grad(), b, a.grad(), false, true, true, tile_m, tile_n);
            // dB += A^T dC; a batched A against a shared B sums the batch
            if (a.shape.rank() == 3 && b.shape.rank() == 2) {
                const uint32_t B = a.shape[0], K = a.shape[2], N = b.shape[1];
                Tensor& per_batch = get_scratch(Shape({B, K, N}));
                evk::ai::matmul(a, c.grad(), per_batch, true, false, false, tile_m, tile_n);
                evk::ai::sum_batch(per_batch, b.grad(), B, K * N);
            } else {
                evk::ai::matmul(a, c.grad(), b.grad(), true, false, true, tile_m, tile_n);
            }
        };
        return c;
    }

    Tensor& add(Tensor& a, Tensor& b) {
        Tensor& c = node(a.shape);
        c.forward_fn = [&a, &b, &c]() { evk::ai::add(a, b, c); };
        c.backward_fn = [&a, &b, &c]() {
            evk::ai::add(a.grad(), c.grad(), a.grad());
            evk::ai::add(b.grad(), c.grad(), b.grad());
        };
        return c;
    }

    // Scalar loss; the forward pass also writes predicted's gradient.
    Tensor& mse_loss(Tensor& predicted, Tensor& target) {
        assert(predicted.shape.rank() == target.shape.rank() && "mse_loss: ranks differ");
        Tensor& loss = node(Shape({1}));
        loss.forward_fn = [&predicted, &target, &loss]() {
            evk::ai::mse_loss(predicted, target, predicted.grad(), loss);
        };
        return loss;
    }

    Tensor& relu(Tensor& a) {
        Tensor& out = node(a.shape);
        out.forward_fn = [&a, &out]() { evk::ai::relu(a, out); };
        out.backward_fn = [&a, &out]() { evk::ai::relu_backward(out.grad(), a, a.grad()); };
        return out;
    }

    Tensor& gelu(Tensor& a) {
        Tensor& out = node(a.shape);
        out.forward_fn = [&a, &out]() { evk::ai::gelu(a, out); };
        out.backward_fn = [&a, &out]() { evk::ai::gelu_backward(out.grad(), a, a.grad()); };
        return out;
    }

    Tensor& scale(Tensor& a, float factor) {
        Tensor& out = node(a.shape);
        const uint64_t bytes = uint64_t(a.shape.count()) * sizeof(float16_t);
        out.forward_fn = [&a, &out, factor, bytes]() {
            evk::ai::GetCmd().copy(a.buffer, out.buffer, bytes);
            evk::ai::scale(out, factor);
        };
        out.backward_fn = [&a, &out, factor]() {
            // out's consumers have all run their backward functions by now
            evk::ai::scale(out.grad(), factor);
            evk::ai::add(a.grad(), out.grad(), a.grad());
        };
        return out;
    }

    Tensor& rms_norm(Tensor& input, float eps = 1e-4f) {
        assert(input.shape.rank() >= 2 && "rms_norm expects at least 2D tensor");
        Tensor& out = node(input.shape);
        out.forward_fn = [&input, &out, eps]() { evk::ai::rms_norm(input, out, eps); };
        out.backward_fn = [&input, &out, eps]() { evk::ai::rms_norm_backward(input, out.grad(), input.grad(), eps); };
        return out;
    }

    // input (B, N, D) + pos_emb (N, D) broadcast over the batch.
    Tensor& add_position_embedding(Tensor& input, Tensor& pos_emb, uint32_t batch_size, uint32_t seq_len) {
        const uint32_t dim = pos_emb.shape[1];
        assert(input.shape.rank() == 3 && input.shape[0] == batch_size && input.shape[1] == seq_len &&
               input.shape[2] == dim && pos_emb.shape[0] == seq_len && "add_position_embedding: shapes");
        Tensor& out = node(input.shape);
        out.forward_fn = [&input, &pos_emb, &out, batch_size, seq_len, dim]() {
            evk::ai::position_add(input, pos_emb, out, batch_size, seq_len, dim);
        };
        out.backward_fn = [&input, &pos_emb, &out, batch_size, seq_len, dim]() {
            evk::ai::position_add_backward(out.grad(), input.grad(), pos_emb.grad(), batch_size, seq_len, dim);
        };
        return out;
    }

    Tensor& rope(Tensor& input, float rotary_base = 10000.0f) {
        assert(input.shape.rank() == 3 && input.shape[2] % 2 == 0 && "rope expects (B, N, D), D even");
        const uint32_t B = input.shape[0], N = input.shape[1], D = input.shape[2];
        Tensor& out = node(input.shape);
        out.forward_fn = [&input, &out, B, N, D, rotary_base]() { evk::ai::rope(input, out, B, N, D, rotary_base); };
        out.backward_fn = [&input, &out, B, N, D, rotary_base]() {
            evk::ai::rope_backward(out.grad(), input.grad(), B, N, D, rotary_base);
        };
        return out;
    }

    // embeddings (V, D), indices (B, N) raw uint16 -> (B, N, D).
    Tensor& embed(Tensor& embeddings, Tensor& indices) {
        assert(indices.shape.rank() == 2 && "indices must be (B, N)");
        Tensor& out = node(Shape({indices.shape[0], indices.shape[1], embeddings.shape[1]}));
        out.forward_fn = [&embeddings, &indices, &out]() { evk::ai::embed(embeddings, indices, out); };
        out.backward_fn = [&embeddings, &indices, &out]() {
            evk::ai::embed_backward(out.grad(), indices, embeddings.grad());
        };
        return out;
    }

    // logits (B, N, V), targets (B, N) raw uint16, target 0 ignored -> scalar
    // mean loss over the other positions.
    Tensor& cross_entropy_loss(Tensor& logits, Tensor& targets) {
        assert(logits.shape.rank() == 3 && targets.shape.rank() == 2 && "cross_entropy_loss: shapes");
        const uint32_t rows = logits.shape[0] * logits.shape[1], V = logits.shape[2];
        Tensor& flat_grad = node(Shape({rows, V}));
        Tensor& loss = node(Shape({1}));
        auto run = [&logits, &targets, &flat_grad, &loss, rows, V]() {
            Tensor flat_logits = Tensor::alias(Shape({rows, V}), logits.buffer);
            Tensor flat_targets = Tensor::alias(Shape({rows}), targets.buffer);
            evk::ai::cross_entropy_loss(flat_logits, flat_targets, flat_grad, loss);
        };
        loss.forward_fn = run;
        loss.backward_fn = [run, &logits, &flat_grad]() {
            run();
            evk::ai::GetCmd().copy(flat_grad.buffer, logits.grad().buffer,
                                   uint64_t(logits.shape.count()) * sizeof(float16_t));
        };
        return loss;
    }

    Tensor& softmax(Tensor& input, float input_scale = 1.0f) {
        Tensor& out = node(input.shape);
        out.forward_fn = [&input, &out, input_scale]() { evk::ai::softmax(input, out, input_scale); };
        out.backward_fn = [&input, &out, input_scale]() {
            evk::ai::softmax_backward(out, out.grad(), input.grad(), input_scale);
        };
        return out;
    }

    // Causal self-attention of q, k, v (B, N, D): softmax(q k^T * scale with
    // keys j > i masked) v; scale 0 means 1/sqrt(D).
    Tensor& causal_attention(Tensor& q, Tensor& k, Tensor& v, float scale = 0.0f) {
        assert(q.shape.rank() == 3 && k.shape.rank() == 3 && v.shape.rank() == 3 && "causal_attention: (B, N, D)");
        const uint32_t B = q.shape[0], N = q.shape[1], D = q.shape[2];
        const float default_scale = 1.0f / std::sqrt(float(D));
        if (scale > 0.0f && scale != default_scale) return causal_attention_unfused(q, k, v, scale);
        // the fused route needs a head size with MFMA flash kernels; other
        // sizes keep the reference's matmul + mask + softmax chain (on MFMA)
        if (!evk::ai::flash_has_mfma(D)) return causal_attention_unfused(q, k, v, scale);
        Tensor& lse = node(Shape({B, 1, N, 2}));  // fp32 log-sum-exp per row
        Tensor& dq = node(q.shape);
        Tensor& dk = node(k.shape);
        Tensor& dv = node(v.shape);
        Tensor& out = node(Shape({B, N, D}));
        out.forward_fn = [&q, &k, &v, &out, &lse]() { evk::ai::flash_attention(q, k, v, out, true, &lse); };
        out.backward_fn = [&q, &k, &v, &out, &lse, &dq, &dk, &dv]() {
            evk::ai::flash_attention_bwd(q, k, v, out, out.grad(), dq, dk, dv, 1, true, &lse);
            evk::ai::add(q.grad(), dq, q.grad());
            evk::ai::add(k.grad(), dk, k.grad());
            evk::ai::add(v.grad(), dv, v.grad());
        };
        return out;
    }

    // The reference's composition: scores = q k^T, mask, softmax(scale), @ v.
    Tensor& causal_attention_unfused(Tensor& q, Tensor& k, Tensor& v, float scale = 0.0f) {
        const uint32_t B = q.shape[0], N = q.shape[1], D = q.shape[2];
        const float s = scale > 0.0f ? scale : 1.0f / std::sqrt(float(D));
        Tensor& scores = node(Shape({B, N, N}));
        Tensor& probs = node(Shape({B, N, N}));
        Tensor& out = node(Shape({B, N, D}));
        out.forward_fn = [&q, &k, &v, &scores, &probs, &out, s]() {
            evk::ai::matmul(q, k, scores, false, true, false, 16, 16);
            evk::ai::apply_causal_mask(scores);
            evk::ai::softmax(scores, probs, s);
            evk::ai::matmul(probs, v, out, false, false, false, 16, 16);
        };
        out.backward_fn = [&q, &k, &v, &scores, &probs, &out, s]() {
            evk::ai::matmul(out.grad(), v, probs.grad(), false, true, false, 16, 16);
            evk::ai::matmul(probs, out.grad(), v.grad(), true, false, true, 16, 16);
            evk::ai::softmax_backward(probs, probs.grad(), scores.grad(), s);
            evk::ai::matmul(scores.grad(), k, q.grad(), false, false, true, 16, 16);
            evk::ai::matmul(scores.grad(), q, k.grad(), true, false, true, 16, 16);
        };
        return out;
    }

    Tensor& residual(Tensor& a, Tensor& b) { return add(a, b); }

    // Forward functions in order; with backward, gradients are zeroed first
    // and the backward functions run in reverse order.
    void eval(bool backward = false, bool submit = true, bool wait = true) {
        evk::ai::GetCmd();
        if (backward)
            for (auto& n : nodes) evk::ai::zero(n->grad());
        for (auto& n : nodes)
            if (n->forward_fn) n->forward_fn();
        if (backward)
            for (auto it = nodes.rbegin(); it != nodes.rend(); ++it)
                if ((*it)->backward_fn) (*it)->backward_fn();
        if (submit) evk::ai::SubmitCmd(wait);
    }

    void step(float lr = 0.001f) {
        for (Tensor* p : params) {
            assert(p->grad_tensor && "Graph::step: parameter without a gradient");
            evk::ai::sgd(*p, p->grad(), lr);
        }
    }

    void step_adam(float lr = 0.001f, float beta1 = 0.9f, float beta2 = 0.999f, float epsilon = 1e-4f) {
        for (Tensor* p : params) evk::ai::adam(*p, p->grad(), adam_states[p], lr, beta1, beta2, epsilon);
    }

    void reset_adam() {
        for (auto& kv : adam_states) kv.second.reset();
        adam_states.clear();
    }

private:
    Tensor& node(const Shape& shape) {
        nodes.push_back(std::make_unique<Tensor>(shape));
        return *nodes.back();
    }
};

namespace evk::ai {

// Weights of one CausalAttentionBlock (example/main_llm.cpp:494-547): the
// Graph's own parameter tensors, read in place.
struct DecoderLayer {
    Tensor* w_q;  // (D, D)
    Tensor* w_k;  // (D, D)
    Tensor* w_v;  // (D, D)
    Tensor* w_o;  // (D, D)
    Tensor* w1;   // (D, hidden)
    Tensor* w2;   // (hidden, D)
};

// The fused decode step of KVCacheDecoder (no reference counterpart): one
// launch runs one position of every sequence through all layers and writes
// the logits (B, 1, V), with the op-by-op step's fp16 rounding points.
// Returns false, having done nothing, when the shapes need the op-by-op
// step (evkhip_kv_decode_step lists its limits).
bool kv_decode_step(Tensor& token_emb, Tensor& w_out, const std::vector<DecoderLayer>& layers,
                    const std::vector<std::unique_ptr<Tensor>>& k_cache,
                    const std::vector<std::unique_ptr<Tensor>>& v_cache, Tensor& ids, uint32_t pos, Tensor& logits,
                    float rope_base, float eps);

// KV-cached decoding of the model example/main_llm.cpp builds with Graph
// ops (MeshTokenModel, :549-620): embed, then per layer
// CausalAttentionBlock::forward (:528-546) -- rms_norm, the q/k/v
// projections, rope over the full width with position = sequence index,
// single-head causal attention, the output projection and residual,
// rms_norm, W1, gelu, W2 and residual -- then rms_norm and the output
// projection.  It replaces the full recompute of sample_autoregressive
// (:622-654) for B sequences decoded together:
//   prefill(tokens)  runs the prompt (B, n) once (MFMA GEMMs, causal flash
//                    attention) and writes every layer's rope'd keys and
//                    values into per-layer caches (B, max_seq, D);
//   step(ids)        feeds one token per sequence at position cached():
//                    single-query attention over the caches, logits (B,1,V)
//                    of that position; evk::ai::greedy_sample(logits(), out,
//                    0, token_base, token_count) then picks the next ids
//                    with the reference's token sub-range.
// The rounding points are those of the Graph (every op output fp16), so the
// greedy ids match a full recompute except at near-ties of the logits.
class KVCacheDecoder {
public:
    KVCacheDecoder(Tensor& token_emb, Tensor& w_out, std::vector<DecoderLayer> layers, uint32_t batch,
                   uint32_t max_seq, float rope_base = 10000.0f, float eps = 1e-4f)
        : emb_(token_emb), w_out_(w_out), layers_(std::move(layers)), B_(batch), S_(max_seq), base_(rope_base),
          eps_(eps) {
        D_ = token_emb.shape[1];
        V_ = w_out.shape[1];
        assert(!layers_.empty() && layers_[0].w1 && "KVCacheDecoder: no layers");
        H_ = layers_[0].w1->shape[1];
        assert(w_out.shape[0] == D_ && D_ % 2 == 0 && "KVCacheDecoder: shapes");
        for (size_t l = 0; l < layers_.size(); ++l) {
            k_cache_.emplace_back(std::make_unique<Tensor>(Shape({B_, S_, D_})));
            v_cache_.emplace_back(std::make_unique<Tensor>(Shape({B_, S_, D_})));
        }
        // prefill work tensors at their largest shape, aliased down per call
        for (auto* t : {&px_, &ph_, &pq_, &pk_, &pv_, &pqr_, &pkr_, &po_, &pt_, &px1_})
            *t = std::make_unique<Tensor>(Shape({B_, S_, D_}));
        pu_ = std::make_unique<Tensor>(Shape({B_, S_, H_}));
        pg_ = std::make_unique<Tensor>(Shape({B_, S_, H_}));
        for (auto* t : {&sx_, &sh_, &sq_, &sk_, &sv_, &sqr_, &skr_, &so_, &st_})
            *t = std::make_unique<Tensor>(Shape({B_, D_}));
        su_ = std::make_unique<Tensor>(Shape({B_, H_}));
        sg_ = std::make_unique<Tensor>(Shape({B_, H_}));
        logits_ = std::make_unique<Tensor>(Shape({B_, 1, V_}));
    }

    uint32_t cached() const { return len_; }
    // step() runs the fused one-launch step (kv_decode_step) where the
    // shapes allow it; false keeps the op-by-op step (for comparisons)
    void set_fused(bool on) { fused_ = on; }
    Tensor& logits() { return *logits_; }
    Tensor& k_cache(uint32_t layer) { return *k_cache_[layer]; }
    Tensor& v_cache(uint32_t layer) { return *v_cache_[layer]; }
    void reset() { len_ = 0; }

    // tokens (B, n) raw uint16 ids of positions [0, n); the caches must be
    // empty (reset() discards what they hold).
    void prefill(Tensor& tokens) {
        assert(tokens.shape.rank() == 2 && tokens.shape[0] == B_ && "prefill: tokens (B, n)");
        const uint32_t n = tokens.shape[1];
        assert(len_ == 0 && n > 0 && n <= S_ && "prefill: from an empty cache, n <= max_seq");
        auto a = [&](std::unique_ptr<Tensor>& t, uint32_t w) { return Tensor::alias(Shape({B_, n, w}), t->buffer); };
        Tensor x = a(px_, D_), h = a(ph_, D_), q = a(pq_, D_), k = a(pk_, D_), v = a(pv_, D_);
        Tensor qr = a(pqr_, D_), kr = a(pkr_, D_), o = a(po_, D_), t = a(pt_, D_), x1 = a(px1_, D_);
        Tensor u = a(pu_, H_), g = a(pg_, H_);
        embed(emb_, tokens, x);
        for (size_t l = 0; l < layers_.size(); ++l) {
            const DecoderLayer& w = layers_[l];
            rms_norm(x, h, eps_);
            matmul(h, *w.w_q, q);
            matmul(h, *w.w_k, k);
            matmul(h, *w.w_v, v);
            rope(q, qr, B_, n, D_, base_);
            rope(k, kr, B_, n, D_, base_);
            kv_cache_write(kr, *k_cache_[l], 0);
            kv_cache_write(v, *v_cache_[l], 0);
            flash_attention(qr, kr, v, o, /*causal=*/true);
            layer_tail(w, x, o, t, x1, h, u, g);
        }
        len_ = n;
    }

    // ids (B) or (B, 1) raw uint16: the token of every sequence at position
    // cached().  Returns logits() (B, 1, V) of that position.
    Tensor& step(Tensor& ids) {
        assert(ids.shape.count() == B_ && "step: one id per sequence");
        assert(len_ < S_ && "step: the caches are full");
        const uint32_t pos = len_;
        if (fused_ && kv_decode_step(emb_, w_out_, layers_, k_cache_, v_cache_, ids, pos, *logits_, base_, eps_)) {
            len_ = pos + 1;
            return *logits_;
        }
        Tensor krow = Tensor::alias(Shape({B_, 1, D_}), skr_->buffer);
        Tensor vrow = Tensor::alias(Shape({B_, 1, D_}), sv_->buffer);
        embed(emb_, ids, *sx_);
        for (size_t l = 0; l < layers_.size(); ++l) {
            const DecoderLayer& w = layers_[l];
            rms_norm(*sx_, *sh_, eps_);
            matmul(*sh_, *w.w_q, *sq_);
            matmul(*sh_, *w.w_k, *sk_);
            matmul(*sh_, *w.w_v, *sv_);
            rope(*sq_, *sqr_, B_, 1, D_, base_, pos);
            rope(*sk_, *skr_, B_, 1, D_, base_, pos);
            kv_cache_write(krow, *k_cache_[l], pos);
            kv_cache_write(vrow, *v_cache_[l], pos);
            single_query_attention(*sqr_, *k_cache_[l], *v_cache_[l], *so_, pos + 1, 1);
            layer_tail(w, *sx_, *so_, *st_, *sx_, *sh_, *su_, *sg_);
        }
        rms_norm(*sx_, *sh_, eps_);
        Tensor flat = Tensor::alias(Shape({B_, V_}), logits_->buffer);
        matmul(*sh_, w_out_, flat);
        len_ = pos + 1;
        return *logits_;
    }

private:
    // attention output o -> x1 = x + o Wo; x = x1 + gelu(rms_norm(x1) W1) W2
    void layer_tail(const DecoderLayer& w, Tensor& x, Tensor& o, Tensor& t, Tensor& x1, Tensor& h, Tensor& u,
                    Tensor& g) {
        matmul(o, *w.w_o, t);
        add(x, t, x1);
        rms_norm(x1, h, eps_);
        matmul(h, *w.w1, u);
        gelu(u, g);
        matmul(g, *w.w2, t);
        add(x1, t, x);
    }

    Tensor& emb_;
    Tensor& w_out_;
    std::vector<DecoderLayer> layers_;
    uint32_t B_, S_, D_ = 0, V_ = 0, H_ = 0;
    float base_, eps_;
    uint32_t len_ = 0;
    bool fused_ = true;
    std::vector<std::unique_ptr<Tensor>> k_cache_, v_cache_;
    std::unique_ptr<Tensor> px_, ph_, pq_, pk_, pv_, pqr_, pkr_, po_, pt_, px1_, pu_, pg_;
    std::unique_ptr<Tensor> sx_, sh_, sq_, sk_, sv_, sqr_, skr_, so_, st_, su_, sg_;
    std::unique_ptr<Tensor> logits_;
};

}  // namespace evk::ai
