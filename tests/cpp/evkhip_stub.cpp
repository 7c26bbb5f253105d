// Recording stand-in for the evkhip C ABI; see evkhip_stub.h.
#include "evkhip_stub.h"

#include <evk_ai.h>  // float16_t

#include <cstring>

namespace {
StubCall g_last;
int g_count = 0;
std::vector<std::string> g_log;
int g_fail_status = 0;
std::string g_fail_msg, g_error;

uint64_t elems(const evkhip_tensor* t) {
    uint64_t n = 1;
    for (uint32_t i = 0; i < t->rank; ++i) n *= t->dims[i];
    return n;
}

int record(const char* name, std::initializer_list<const evkhip_tensor*> ts, std::initializer_list<long long> ints,
           std::initializer_list<double> floats, void* stream, const void* ptr = nullptr) {
    ++g_count;
    g_log.push_back(name);
    g_last = StubCall{};
    g_last.name = name;
    for (const evkhip_tensor* t : ts) {
        g_last.tensors.push_back(*t);
        if (t->data && !mock_stream_access(t->data, elems(t) * 2)) return EVKHIP_ERR_INVALID_ARG;
    }
    g_last.ints = ints;
    g_last.floats = floats;
    g_last.stream = stream;
    g_last.ptr = ptr;
    if (g_fail_status) {
        const int s = g_fail_status;
        g_fail_status = 0;
        g_error = g_fail_msg;
        return s;
    }
    return EVKHIP_OK;
}
}  // namespace

const StubCall& stub_last_call() {
    return g_last;
}
int stub_call_count() {
    return g_count;
}
const std::vector<std::string>& stub_call_log() {
    return g_log;
}
void stub_clear_log() {
    g_log.clear();
}
void stub_fail_next(int status, const char* msg) {
    g_fail_status = status;
    g_fail_msg = msg;
}

extern "C" {

const char* evkhip_version(void) {
    return "evkhip stub";
}
const char* evkhip_last_error(void) {
    return g_error.c_str();
}
int evkhip_init(void) {
    return record("init", {}, {}, {}, nullptr);
}
int evkhip_shutdown(void) {
    return record("shutdown", {}, {}, {}, nullptr);
}

int evkhip_matmul(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, int ta, int tb, int acc,
                  uint32_t tm, uint32_t tn, void* stream) {
    return record("matmul", {a, b, c}, {ta, tb, acc, tm, tn}, {}, stream);
}
// The fill really fills (the mock's device memory is host memory), so the
// evk core's Cmd::fill and evk::ai::zero can be checked by reading back.
int evkhip_fill(void* data, uint64_t bytes, uint32_t pattern, void* stream) {
    const int rc = record("fill", {}, {(long long)bytes, (long long)pattern}, {}, stream, data);
    if (rc) return rc;
    if (bytes & 1) return EVKHIP_ERR_INVALID_ARG;
    if (bytes && !mock_stream_access(data, bytes)) return EVKHIP_ERR_INVALID_ARG;
    uint16_t* p = static_cast<uint16_t*>(data);
    for (uint64_t i = 0; i < bytes / 2; ++i) p[i] = uint16_t((i & 1) ? pattern >> 16 : pattern);
    return EVKHIP_OK;
}
int evkhip_flash_has_mfma(uint32_t head_dim) {
    return head_dim % 16 == 0 && head_dim >= 16 && head_dim <= 256;
}
int evkhip_flash_attention(const evkhip_tensor* q, const evkhip_tensor* k, const evkhip_tensor* v,
                           const evkhip_tensor* o, int causal, float* lse, void* stream) {
    return record("flash_attention", {q, k, v, o}, {causal}, {}, stream, lse);
}
int evkhip_flash_attention_bwd(const evkhip_tensor* q, const evkhip_tensor* k, const evkhip_tensor* v,
                               const evkhip_tensor* o, const evkhip_tensor* dO, const evkhip_tensor* dQ,
                               const evkhip_tensor* dK, const evkhip_tensor* dV, uint32_t heads, int causal,
                               const float* lse, void* stream) {
    return record("flash_attention_bwd", {q, k, v, o, dO, dQ, dK, dV}, {heads, causal}, {}, stream, lse);
}
int evkhip_single_query_attention(const evkhip_tensor* q, const evkhip_tensor* kc, const evkhip_tensor* vc,
                                  const evkhip_tensor* out, uint32_t L, uint32_t heads, void* stream) {
    return record("single_query_attention", {q, kc, vc, out}, {L, heads}, {}, stream);
}
int evkhip_kv_decode_step(const evkhip_kv_model* m, const uint16_t* ids, uint32_t pos, void* logits, void* stream) {
    // the host mock has no kernels: report the shape as unsupported, so the
    // decoder takes its op-by-op step (which the stub records)
    (void)record("kv_decode_step", {}, {m ? (long long)m->layers : 0, pos}, {}, stream, ids);
    (void)logits;
    return EVKHIP_ERR_UNSUPPORTED;
}
int evkhip_kv_cache_write(const evkhip_tensor* src, const evkhip_tensor* cache, uint32_t pos0, void* stream) {
    return record("kv_cache_write", {src, cache}, {pos0}, {}, stream);
}
int evkhip_rms_norm(const evkhip_tensor* in, const evkhip_tensor* out, float eps, void* stream) {
    return record("rms_norm", {in, out}, {}, {eps}, stream);
}
int evkhip_rope(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t b, uint32_t n, uint32_t d, float base,
                uint32_t pos, uint32_t hd, void* stream) {
    return record("rope", {in, out}, {b, n, d, pos, hd}, {base}, stream);
}
int evkhip_gelu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream) {
    return record("gelu", {in, out}, {}, {}, stream);
}
// training ops: recorded only
int evkhip_scale(const evkhip_tensor* t, float factor, void* stream) {
    return record("scale", {t}, {}, {factor}, stream);
}
int evkhip_relu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream) {
    return record("relu", {in, out}, {}, {}, stream);
}
int evkhip_relu_backward(const evkhip_tensor* go, const evkhip_tensor* in, const evkhip_tensor* gi, void* stream) {
    return record("relu_backward", {go, in, gi}, {}, {}, stream);
}
int evkhip_gelu_backward(const evkhip_tensor* go, const evkhip_tensor* in, const evkhip_tensor* gi, void* stream) {
    return record("gelu_backward", {go, in, gi}, {}, {}, stream);
}
int evkhip_mse_loss(const evkhip_tensor* p, const evkhip_tensor* t, const evkhip_tensor* g, const evkhip_tensor* r,
                    void* stream) {
    return record("mse_loss", {p, t, g, r}, {}, {}, stream);
}
int evkhip_sgd(const evkhip_tensor* p, const evkhip_tensor* g, float lr, void* stream) {
    return record("sgd", {p, g}, {}, {lr}, stream);
}
int evkhip_adam(const evkhip_tensor* p, const evkhip_tensor* g, const evkhip_tensor* m, const evkhip_tensor* v,
                float lr, float b1, float b2, float c1, float c2, float eps, void* stream) {
    return record("adam", {p, g, m, v}, {}, {lr, b1, b2, c1, c2, eps}, stream);
}
int evkhip_softmax(const evkhip_tensor* in, const evkhip_tensor* out, float scale, void* stream) {
    return record("softmax", {in, out}, {}, {scale}, stream);
}
int evkhip_softmax_backward(const evkhip_tensor* p, const evkhip_tensor* go, const evkhip_tensor* gi, float scale,
                            void* stream) {
    return record("softmax_backward", {p, go, gi}, {}, {scale}, stream);
}
int evkhip_rms_norm_backward(const evkhip_tensor* in, const evkhip_tensor* go, const evkhip_tensor* gi, float eps,
                             void* stream) {
    return record("rms_norm_backward", {in, go, gi}, {}, {eps}, stream);
}
int evkhip_cross_entropy_loss(const evkhip_tensor* l, const evkhip_tensor* t, const evkhip_tensor* g,
                              const evkhip_tensor* r, void* stream) {
    return record("cross_entropy_loss", {l, t, g, r}, {}, {}, stream);
}
int evkhip_sum_batch(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t b, uint32_t n, void* stream) {
    return record("sum_batch", {in, out}, {b, n}, {}, stream);
}
int evkhip_apply_causal_mask(const evkhip_tensor* s, void* stream) {
    return record("apply_causal_mask", {s}, {}, {}, stream);
}
int evkhip_position_add(const evkhip_tensor* in, const evkhip_tensor* pos, const evkhip_tensor* out, uint32_t b,
                        uint32_t n, uint32_t d, void* stream) {
    return record("position_add", {in, pos, out}, {b, n, d}, {}, stream);
}
int evkhip_position_add_backward(const evkhip_tensor* go, const evkhip_tensor* gi, const evkhip_tensor* gp,
                                 uint32_t b, uint32_t n, uint32_t d, void* stream) {
    return record("position_add_backward", {go, gi, gp}, {b, n, d}, {}, stream);
}
int evkhip_rope_backward(const evkhip_tensor* go, const evkhip_tensor* gi, uint32_t b, uint32_t n, uint32_t d,
                         float base, void* stream) {
    return record("rope_backward", {go, gi}, {b, n, d}, {base}, stream);
}
int evkhip_embed_backward(const evkhip_tensor* go, const evkhip_tensor* idx, const evkhip_tensor* ge, void* stream) {
    return record("embed_backward", {go, idx, ge}, {}, {}, stream);
}
// add is computed (fp32 sum rounded to fp16) so data round trips can be checked
int evkhip_add(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, void* stream) {
    const int s = record("add", {a, b, c}, {}, {}, stream);
    if (s != EVKHIP_OK) return s;
    const uint64_t n = elems(c);
    if (elems(a) != n || elems(b) != n) return EVKHIP_ERR_SHAPE;
    const float16_t* x = static_cast<const float16_t*>(a->data);
    const float16_t* y = static_cast<const float16_t*>(b->data);
    float16_t* z = static_cast<float16_t*>(c->data);
    for (uint64_t i = 0; i < n; ++i) z[i] = float16_t(float(x[i]) + float(y[i]));
    return EVKHIP_OK;
}
int evkhip_embed(const evkhip_tensor* e, const evkhip_tensor* idx, const evkhip_tensor* out, void* stream) {
    return record("embed", {e, idx, out}, {}, {}, stream);
}
int evkhip_greedy_sample(const evkhip_tensor* logits, const evkhip_tensor* out, uint32_t position, uint16_t base,
                         uint16_t count, void* stream) {
    return record("greedy_sample", {logits, out}, {position, base, count}, {}, stream);
}

}  // extern "C"
