// KV-cached greedy decode of the reference transformer block
// (example/main_llm.cpp:528-546, MeshTokenModel :598-606) on the device.
// The reference samples by re-running the whole graph for every position
// (main_llm.cpp:622-654); this runtime keeps a per-layer K/V cache and runs
// one token per step: embed -> [rms_norm, x.Wqkv, rope(q,k), cache append,
// single-query attention, x.Wo + residual, rms_norm, gelu(x.W1).W2 +
// residual] x layers -> rms_norm -> x.Wout -> greedy argmax, with the next
// token id read back by the next step's embed on the device (no host sync).
#include "kernels.h"

#include <algorithm>

#define CHECK(expr)          \
    do {                     \
        int _rc = (expr);    \
        if (_rc) return _rc; \
    } while (0)

namespace evkhip {

namespace {

__global__ __launch_bounds__(256) void copy_k(const u32x4* src, u32x4* dst, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

struct ModelWs {
    f16* buf = nullptr;
    size_t elems = 0;
};
ModelWs g_ws;

struct Weights {
    const f16* E;
    const f16* Wout;
    uint64_t per_layer;
    const f16* layer(const evkhip_model_cfg& c, const f16* base, uint32_t l) const {
        return base + (uint64_t)c.vocab * c.d + l * per_layer;
    }
};

int gemv(const f16* x, const f16* W, f16* y, int K, int N, hipStream_t st) {
    GemmArgs g{};
    g.A = x;
    g.B = W;
    g.C = y;
    g.M = 1;
    g.N = N;
    g.K = K;
    g.acc = 0;
    const bool vec = (K % 8 == 0) && (N % 8 == 0) && aligned16(x) && aligned16(W) && aligned16(y);
    return gemm_dispatch(g, 1, false, false, vec, st);
}

}  // namespace

void model_free_workspace() {
    if (g_ws.buf) (void)hipFree(g_ws.buf);
    g_ws = ModelWs{};
}

}  // namespace evkhip

using namespace evkhip;

extern "C" {

uint64_t evkhip_model_weight_elems(const evkhip_model_cfg* c) {
    if (!c) return 0;
    const uint64_t d = c->d;
    const uint64_t per = d * 3 * d + d * d + d * c->hidden + (uint64_t)c->hidden * d;
    return (uint64_t)c->vocab * d + c->layers * per + d * c->vocab;
}

uint64_t evkhip_model_cache_elems(const evkhip_model_cfg* c) {
    if (!c) return 0;
    return (uint64_t)c->layers * 2 * c->max_seq * c->d;
}

}  // extern "C"

namespace evkhip {
namespace {

// Validates cfg/buffers and runs n tokens.  feed != null: token s is feed[s],
// only the last step runs the LM head (into ids[0]); otherwise token s is
// ids[s] and every step writes ids[s+1].
int run_tokens(const evkhip_model_cfg* cfg, const void* weights, void* cache, const uint16_t* feed,
               uint16_t* ids, uint32_t n, uint32_t pos0, void* logits, hipStream_t st) {
    EVK_RETURN_IF(!cfg || !weights || !cache || !ids || !logits, EVKHIP_ERR_INVALID_ARG,
                  "model: null argument");
    const evkhip_model_cfg c = *cfg;
    EVK_RETURN_IF(c.vocab == 0 || c.vocab > 65536 || c.d == 0 || c.heads == 0 || c.layers == 0 || c.hidden == 0,
                  EVKHIP_ERR_INVALID_ARG, "model: empty model dimension");
    EVK_RETURN_IF(c.heads * c.dh != c.d || c.dh % 2, EVKHIP_ERR_SHAPE, "model: d=%u != heads*dh (%u*%u)",
                  c.d, c.heads, c.dh);
    EVK_RETURN_IF((uint64_t)pos0 + n > c.max_seq, EVKHIP_ERR_SHAPE,
                  "model: positions %u..%u exceed max_seq %u", pos0, pos0 + n, c.max_seq);
    EVK_RETURN_IF(c.d % 8 || c.hidden % 8 || c.vocab % 8 || !aligned16(weights) || !aligned16(cache) ||
                      !aligned16(logits),
                  EVKHIP_ERR_UNSUPPORTED, "model: needs 16-byte aligned buffers and d, hidden, vocab "
                  "multiples of 8");
    if (n == 0) return EVKHIP_OK;
    const uint32_t d = c.d, hid = c.hidden;
    // workspace: x, h, att, tmp (d each), qkv (3d), qr (d), hid, hidg
    const size_t need = (size_t)d * 8 + 2 * (size_t)hid + 64;
    if (need > g_ws.elems) {
        if (g_ws.buf) EVK_HIP(hipFree(g_ws.buf));
        g_ws.buf = nullptr;
        EVK_HIP(hipMalloc(&g_ws.buf, need * sizeof(f16)));
        g_ws.elems = need;
    }
    f16* x = g_ws.buf;
    f16* h = x + d;
    f16* att = h + d;
    f16* tmp = att + d;
    f16* qkv = tmp + d;
    f16* qr = qkv + 3 * d;
    f16* hh = qr + d;
    f16* hg = hh + hid;

    Weights W{};
    W.E = (const f16*)weights;
    W.per_layer = (uint64_t)d * 3 * d + (uint64_t)d * d + (uint64_t)d * hid + (uint64_t)hid * d;
    W.Wout = W.E + (uint64_t)c.vocab * d + c.layers * W.per_layer;
    f16* cache_h = (f16*)cache;

    for (uint32_t s = 0; s < n; ++s) {
        const uint32_t pos = pos0 + s;
        const uint16_t* tok = feed ? feed + s : ids + s;
        CHECK(embed_launch(W.E, tok, x, 1, (int)d, (int)c.vocab, st));
        for (uint32_t l = 0; l < c.layers; ++l) {
            const f16* Wqkv = W.layer(c, W.E, l);
            const f16* Wo = Wqkv + (uint64_t)d * 3 * d;
            const f16* W1 = Wo + (uint64_t)d * d;
            const f16* W2 = W1 + (uint64_t)d * hid;
            f16* Kc = cache_h + (uint64_t)l * 2 * c.max_seq * d;
            f16* Vc = Kc + (uint64_t)c.max_seq * d;
            CHECK(rms_norm_launch(x, h, 1, (int)d, c.eps, st));
            CHECK(gemv(h, Wqkv, qkv, (int)d, (int)(3 * d), st));
            CHECK(rope_launch(qkv, qr, 1, 1, (int)d, c.rope_base, (int)pos, (int)c.dh, st));
            CHECK(rope_launch(qkv + d, Kc + (uint64_t)pos * d, 1, 1, (int)d, c.rope_base, (int)pos, (int)c.dh, st));
            hipLaunchKernelGGL(copy_k, dim3((d / 8 + 255) / 256), dim3(256), 0, st,
                               reinterpret_cast<const u32x4*>(qkv + 2 * d),
                               reinterpret_cast<u32x4*>(Vc + (uint64_t)pos * d), (int64_t)(d / 8));
            CHECK(sq_attention_launch(qr, Kc, Vc, att, (int64_t)d, (int)c.heads, (int)c.dh, (int)(pos + 1), true,
                                      st));
            CHECK(gemv(att, Wo, tmp, (int)d, (int)d, st));
            CHECK(add_launch(x, tmp, x, d, st));
            CHECK(rms_norm_launch(x, h, 1, (int)d, c.eps, st));
            CHECK(gemv(h, W1, hh, (int)d, (int)hid, st));
            CHECK(gelu_launch(hh, hg, hid, st));
            CHECK(gemv(hg, W2, tmp, (int)hid, (int)d, st));
            CHECK(add_launch(x, tmp, x, d, st));
        }
        if (!feed || s + 1 == n) {
            uint16_t* out_id = feed ? ids : ids + s + 1;
            CHECK(rms_norm_launch(x, h, 1, (int)d, c.eps, st));
            CHECK(gemv(h, W.Wout, (f16*)logits, (int)d, (int)c.vocab, st));
            CHECK(greedy_launch((const f16*)logits, out_id, 1, 1, (int)c.vocab, 0, 0, (int)c.vocab, st));
        }
    }
    EVK_HIP(hipGetLastError());
    return EVKHIP_OK;
}

}  // namespace
}  // namespace evkhip

extern "C" {

int evkhip_model_prefill(const evkhip_model_cfg* cfg, const void* weights, void* cache, const uint16_t* tokens,
                         uint32_t n_tokens, uint32_t pos0, uint16_t* next_id, void* logits, void* stream) {
    EVK_RETURN_IF(!tokens && n_tokens, EVKHIP_ERR_INVALID_ARG, "model_prefill: null tokens");
    return run_tokens(cfg, weights, cache, tokens, next_id, n_tokens, pos0, logits, as_stream(stream));
}

int evkhip_model_decode(const evkhip_model_cfg* cfg, const void* weights, void* cache, uint16_t* token_io,
                        uint32_t n_steps, uint32_t pos0, void* logits, void* stream) {
    return run_tokens(cfg, weights, cache, nullptr, token_io, n_steps, pos0, logits, as_stream(stream));
}

}  // extern "C"
