// evk::ai over the gfx950 kernel library: each op turns its Tensors into
// evkhip_tensor descriptors and calls the C ABI on the runtime's stream.
//
// Replaces /root/reference/evk_ai.cpp for the hot path: GetCmd/SubmitCmd
// (:13-28), initialize/shutdown (:211-252), matmul (:254-330),
// flash_attention (:332-369), flash_attention_bwd (:371-473), add
// (:568-591), gelu (:679-699), embed (:782-806), greedy_sample (:808-837),
// rope (:945-966), zero (:1010-1025), rms_norm (:1045-1067), and the
// training ops with AdamState (:181-209,475-566,593-780,839-943,968-1043,
// 1072-1093).  Shape checks
// live in the C ABI (they run on the host before any launch); a failed check
// prints the library's message and aborts, as the reference's asserts do.
#include <evk_ai.h>
#include <evkhip.h>

#include <hip/hip_runtime_api.h>

namespace evk::ai {
namespace {

evk::Cmd* g_cmd = nullptr;

evkhip_tensor desc(Tensor& t) {
    evkhip_tensor d{};
    d.data = t.device_ptr();
    d.rank = t.shape.rank();
    for (uint32_t i = 0; i < d.rank; ++i) d.dims[i] = t.shape.values[i];
    return d;
}

void check(int status, const char* op) {
    if (status != EVKHIP_OK) {
        std::fprintf(stderr, "evk::ai::%s failed (status %d): %s\n", op, status, evkhip_last_error());
        std::abort();
    }
}

void* stream() {
    return GetCmd().stream();
}

// The fp32 LSE of B*H*N rows lives in an fp16 tensor of 2*B*H*N elements.
float* lse_ptr(Tensor* lse, Tensor& q, Tensor& k, const char* op) {
    if (!lse) return nullptr;
    if (q.shape.rank() != 3 || k.shape.rank() != 3 || k.shape[2] == 0) return nullptr;  // the C ABI reports it
    const uint64_t rows = uint64_t(q.shape[0]) * (q.shape[2] / k.shape[2]) * q.shape[1];
    if (uint64_t(lse->shape.count()) != 2 * rows) {
        std::fprintf(stderr, "evk::ai::%s: lse holds %u fp16 slots, needs %llu (B*H*N fp32)\n", op,
                     lse->shape.count(), (unsigned long long)(2 * rows));
        std::abort();
    }
    return static_cast<float*>(lse->device_ptr());
}

}  // namespace

evk::Cmd& GetCmd() {
    if (!g_cmd) g_cmd = &evk::CmdBegin(evk::Queue::Graphics);
    return *g_cmd;
}

uint64_t SubmitCmd(bool wait) {
    evk::Cmd& cmd = GetCmd();
    const uint64_t idx = cmd.submit();
    g_cmd = nullptr;
    if (wait) evk::CmdWait(idx);
    return idx;
}

void initialize() {
    if (!evk::IsInitialized() && !evk::InitializeEVK(evk::EvkDesc{})) {
        std::fprintf(stderr, "evk::ai::initialize: no usable gfx950 device\n");
        std::abort();
    }
    check(evkhip_init(), "initialize");
}

void shutdown() {
    if (g_cmd) SubmitCmd(true);
    check(evkhip_shutdown(), "shutdown");
    evk::Shutdown();
}

void matmul(Tensor& a, Tensor& b, Tensor& c, bool transpose_a, bool transpose_b, bool acc_c, uint8_t TILE_M,
            uint8_t TILE_N) {
    evkhip_tensor A = desc(a), B = desc(b), C = desc(c);
    check(evkhip_matmul(&A, &B, &C, transpose_a, transpose_b, acc_c, TILE_M, TILE_N, stream()), "matmul");
}

bool flash_has_mfma(uint32_t head_dim) { return evkhip_flash_has_mfma(head_dim) != 0; }

void flash_attention(Tensor& q, Tensor& k, Tensor& v, Tensor& o, bool causal, Tensor* lse) {
    evkhip_tensor Q = desc(q), K = desc(k), V = desc(v), O = desc(o);
    float* L = lse_ptr(lse, q, k, "flash_attention");
    check(evkhip_flash_attention(&Q, &K, &V, &O, causal, L, stream()), "flash_attention");
}

void flash_attention_bwd(Tensor& q, Tensor& k, Tensor& v, Tensor& o, Tensor& dO, Tensor& dQ, Tensor& dK,
                         Tensor& dV, uint32_t heads, bool causal, Tensor* lse) {
    evkhip_tensor Q = desc(q), K = desc(k), V = desc(v), O = desc(o), G = desc(dO);
    evkhip_tensor DQ = desc(dQ), DK = desc(dK), DV = desc(dV);
    float* L = lse_ptr(lse, q, k, "flash_attention_bwd");
    check(evkhip_flash_attention_bwd(&Q, &K, &V, &O, &G, &DQ, &DK, &DV, heads, causal, L, stream()),
          "flash_attention_bwd");
}

void single_query_attention(Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& out, uint32_t current_length,
                            uint32_t heads) {
    evkhip_tensor Q = desc(q), K = desc(k_cache), V = desc(v_cache), O = desc(out);
    check(evkhip_single_query_attention(&Q, &K, &V, &O, current_length, heads, stream()),
          "single_query_attention");
}

bool kv_decode_step(Tensor& token_emb, Tensor& w_out, const std::vector<DecoderLayer>& layers,
                    const std::vector<std::unique_ptr<Tensor>>& k_cache,
                    const std::vector<std::unique_ptr<Tensor>>& v_cache, Tensor& ids, uint32_t pos, Tensor& logits,
                    float rope_base, float eps) {
    if (layers.empty() || layers.size() > EVKHIP_KV_MAX_LAYERS || k_cache.size() != layers.size() ||
        v_cache.size() != layers.size() || token_emb.shape.rank() != 2 || w_out.shape.rank() != 2 ||
        k_cache[0]->shape.rank() != 3)
        return false;
    evkhip_kv_model m{};
    m.batch = k_cache[0]->shape[0];
    m.max_seq = k_cache[0]->shape[1];
    m.d = token_emb.shape[1];
    m.vocab = w_out.shape[1];
    m.hidden = layers[0].w1->shape[1];
    m.layers = uint32_t(layers.size());
    m.eps = eps;
    m.rope_base = rope_base;
    if (ids.shape.count() != m.batch || logits.shape.count() != m.batch * m.vocab || w_out.shape[0] != m.d)
        return false;
    m.emb = token_emb.device_ptr();
    m.w_out = w_out.device_ptr();
    for (size_t l = 0; l < layers.size(); ++l) {
        const DecoderLayer& w = layers[l];
        Tensor* t[6] = {w.w_q, w.w_k, w.w_v, w.w_o, w.w1, w.w2};
        for (int i = 0; i < 6; ++i) m.w[l][i] = t[i]->device_ptr();
        m.k_cache[l] = k_cache[l]->device_ptr();
        m.v_cache[l] = v_cache[l]->device_ptr();
    }
    const int rc = evkhip_kv_decode_step(&m, static_cast<const uint16_t*>(ids.device_ptr()), pos,
                                         logits.device_ptr(), stream());
    if (rc == EVKHIP_ERR_UNSUPPORTED) return false;
    check(rc, "kv_decode_step");
    return true;
}

void kv_cache_write(Tensor& src, Tensor& cache, uint32_t pos0) {
    evkhip_tensor S = desc(src), C = desc(cache);
    check(evkhip_kv_cache_write(&S, &C, pos0, stream()), "kv_cache_write");
}

void add(Tensor& a, Tensor& b, Tensor& c) {
    evkhip_tensor A = desc(a), B = desc(b), C = desc(c);
    check(evkhip_add(&A, &B, &C, stream()), "add");
}

void gelu(Tensor& in, Tensor& out) {
    evkhip_tensor I = desc(in), O = desc(out);
    check(evkhip_gelu(&I, &O, stream()), "gelu");
}

void embed(Tensor& embeddings, Tensor& indices, Tensor& out) {
    evkhip_tensor E = desc(embeddings), I = desc(indices), O = desc(out);
    check(evkhip_embed(&E, &I, &O, stream()), "embed");
}

void greedy_sample(Tensor& logits, Tensor& out_tokens, uint32_t position, uint16_t token_base,
                   uint16_t token_count) {
    evkhip_tensor L = desc(logits), T = desc(out_tokens);
    check(evkhip_greedy_sample(&L, &T, position, token_base, token_count, stream()), "greedy_sample");
}

void rope(Tensor& input, Tensor& out, uint32_t batch_size, uint32_t seq_len, uint32_t embed_dim, float rotary_base,
          uint32_t position_offset, uint32_t head_dim) {
    evkhip_tensor I = desc(input), O = desc(out);
    check(evkhip_rope(&I, &O, batch_size, seq_len, embed_dim, rotary_base, position_offset, head_dim, stream()),
          "rope");
}

void rms_norm(Tensor& input, Tensor& output, float eps) {
    evkhip_tensor I = desc(input), O = desc(output);
    check(evkhip_rms_norm(&I, &O, eps, stream()), "rms_norm");
}

void zero(Tensor& tensor) {
    const uint64_t bytes = uint64_t(tensor.shape.count()) * sizeof(float16_t);
    if (bytes == 0) return;
    check(evkhip_fill(tensor.device_ptr(), bytes, 0u, stream()), "zero");
}

// ---- training ops (evk_ai.cpp:475-566,593-780,839-943,968-1043,1072-1093) ----

void AdamState::init(uint32_t num_elements) {
    const uint64_t bytes = uint64_t(num_elements) * sizeof(float16_t);
    m_buffer = evk::CreateBuffer({.size = bytes, .usage = evk::BufferUsage::Storage | evk::BufferUsage::TransferDst});
    v_buffer = evk::CreateBuffer({.size = bytes, .usage = evk::BufferUsage::Storage | evk::BufferUsage::TransferDst});
    if (bytes) {
        GetCmd().fill(m_buffer, 0u, bytes);
        GetCmd().fill(v_buffer, 0u, bytes);
    }
    t = 0;
}

void AdamState::reset() {
    m_buffer = {};
    v_buffer = {};
    t = 0;
}

void mse_loss(Tensor& predicted, Tensor& target, Tensor& predGrad, Tensor& result) {
    evkhip_tensor P = desc(predicted), T = desc(target), G = desc(predGrad), R = desc(result);
    check(evkhip_mse_loss(&P, &T, &G, &R, stream()), "mse_loss");
}

void sgd(Tensor& param, Tensor& gradient, float learning_rate) {
    evkhip_tensor P = desc(param), G = desc(gradient);
    check(evkhip_sgd(&P, &G, learning_rate, stream()), "sgd");
}

void adam(Tensor& param, Tensor& gradient, AdamState& state, float learning_rate, float beta1, float beta2,
          float epsilon) {
    const uint32_t n = param.shape.count();
    if (!state.m_buffer) state.init(n);
    state.t++;
    const float c1 = 1.0f / (1.0f - std::pow(beta1, float(state.t)));
    const float c2 = 1.0f / (1.0f - std::pow(beta2, float(state.t)));
    evkhip_tensor P = desc(param), G = desc(gradient);
    evkhip_tensor M{}, V{};
    M.data = reinterpret_cast<void*>(state.m_buffer.GetReference());
    V.data = reinterpret_cast<void*>(state.v_buffer.GetReference());
    M.rank = V.rank = 1;
    M.dims[0] = V.dims[0] = n;
    check(evkhip_adam(&P, &G, &M, &V, learning_rate, beta1, beta2, c1, c2, epsilon, stream()), "adam");
}

void softmax(Tensor& in, Tensor& out, float input_scale) {
    evkhip_tensor I = desc(in), O = desc(out);
    check(evkhip_softmax(&I, &O, input_scale, stream()), "softmax");
}

void softmax_backward(Tensor& probs, Tensor& grad_out, Tensor& grad_in, float scale_factor) {
    evkhip_tensor P = desc(probs), G = desc(grad_out), I = desc(grad_in);
    check(evkhip_softmax_backward(&P, &G, &I, scale_factor, stream()), "softmax_backward");
}

void relu(Tensor& in, Tensor& out) {
    evkhip_tensor I = desc(in), O = desc(out);
    check(evkhip_relu(&I, &O, stream()), "relu");
}

void relu_backward(Tensor& grad_out, Tensor& in, Tensor& grad_in) {
    evkhip_tensor G = desc(grad_out), I = desc(in), D = desc(grad_in);
    check(evkhip_relu_backward(&G, &I, &D, stream()), "relu_backward");
}

void gelu_backward(Tensor& grad_out, Tensor& in, Tensor& grad_in) {
    evkhip_tensor G = desc(grad_out), I = desc(in), D = desc(grad_in);
    check(evkhip_gelu_backward(&G, &I, &D, stream()), "gelu_backward");
}

void cross_entropy_loss(Tensor& logits, Tensor& targets, Tensor& grad, Tensor& result) {
    evkhip_tensor L = desc(logits), T = desc(targets), G = desc(grad), R = desc(result);
    check(evkhip_cross_entropy_loss(&L, &T, &G, &R, stream()), "cross_entropy_loss");
}

void embed_backward(Tensor& grad_out, Tensor& indices, Tensor& grad_embeddings) {
    evkhip_tensor G = desc(grad_out), I = desc(indices), E = desc(grad_embeddings);
    check(evkhip_embed_backward(&G, &I, &E, stream()), "embed_backward");
}

void apply_causal_mask(Tensor& scores) {
    evkhip_tensor S = desc(scores);
    check(evkhip_apply_causal_mask(&S, stream()), "apply_causal_mask");
}

void position_add(Tensor& input, Tensor& pos_emb, Tensor& out, uint32_t batch_size, uint32_t seq_len,
                  uint32_t embed_dim) {
    evkhip_tensor I = desc(input), P = desc(pos_emb), O = desc(out);
    check(evkhip_position_add(&I, &P, &O, batch_size, seq_len, embed_dim, stream()), "position_add");
}

void position_add_backward(Tensor& grad_out, Tensor& grad_input, Tensor& grad_pos, uint32_t batch_size,
                           uint32_t seq_len, uint32_t embed_dim) {
    evkhip_tensor G = desc(grad_out), I = desc(grad_input), P = desc(grad_pos);
    check(evkhip_position_add_backward(&G, &I, &P, batch_size, seq_len, embed_dim, stream()),
          "position_add_backward");
}

void rope_backward(Tensor& grad_out, Tensor& grad_input, uint32_t batch_size, uint32_t seq_len, uint32_t embed_dim,
                   float rotary_base) {
    evkhip_tensor G = desc(grad_out), I = desc(grad_input);
    check(evkhip_rope_backward(&G, &I, batch_size, seq_len, embed_dim, rotary_base, stream()), "rope_backward");
}

void scale(Tensor& tensor, float scale_factor) {
    evkhip_tensor T = desc(tensor);
    check(evkhip_scale(&T, scale_factor, stream()), "scale");
}

void sum_batch(Tensor& input, Tensor& output, uint32_t batch_count, uint32_t size_per_batch) {
    evkhip_tensor I = desc(input), O = desc(output);
    check(evkhip_sum_batch(&I, &O, batch_count, size_per_batch, stream()), "sum_batch");
}

void rms_norm_backward(Tensor& input, Tensor& grad_out, Tensor& grad_input, float eps) {
    evkhip_tensor I = desc(input), G = desc(grad_out), D = desc(grad_input);
    check(evkhip_rms_norm_backward(&I, &G, &D, eps, stream()), "rms_norm_backward");
}

}  // namespace evk::ai
