// evk::ai over the gfx950 kernel library: each op turns its Tensors into
// evkhip_tensor descriptors and calls the C ABI on the runtime's stream.
//
// Replaces /root/reference/evk_ai.cpp for the hot path: GetCmd/SubmitCmd
// (:13-28), initialize/shutdown (:211-252), matmul (:254-330),
// flash_attention (:332-369), flash_attention_bwd (:371-473), add
// (:568-591), gelu (:679-699), embed (:782-806), greedy_sample (:808-837),
// rope (:945-966), zero (:1010-1025), rms_norm (:1045-1067).  Shape checks
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
    const hipError_t e = hipMemsetAsync(tensor.device_ptr(), 0, bytes, static_cast<hipStream_t>(stream()));
    if (e != hipSuccess) {
        std::fprintf(stderr, "evk::ai::zero failed: %s\n", hipGetErrorString(e));
        std::abort();
    }
}

}  // namespace evk::ai
