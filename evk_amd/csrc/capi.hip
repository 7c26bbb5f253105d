// C ABI entry points (include/evkhip.h): argument and shape validation on the
// host, then dispatch to the gfx950 kernels.  Validation mirrors the asserts
// of the reference wrappers (evk_ai.cpp) but reports a status code instead of
// aborting, and relaxes the tile-divisibility rules (matmul accepts any M, N,
// K; flash attention any N).
#include "kernels.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <initializer_list>

namespace evkhip {


// ---------------------------------------------------------------------------
static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char* what) {
    return set_error(EVKHIP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int device_cu_count() {
    static int cached_dev = -1, cached_cus = 256;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return cached_cus;
    if (dev != cached_dev) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            cached_cus = cus;
        cached_dev = dev;
    }
    return cached_cus;
}

int check_tensor(const evkhip_tensor* t, const char* name, uint32_t min_rank, uint32_t max_rank) {
    if (!t) return set_error(EVKHIP_ERR_INVALID_ARG, "%s: null tensor descriptor", name);
    if (t->rank < min_rank || t->rank > max_rank)
        return set_error(EVKHIP_ERR_SHAPE, "%s: rank %u not in [%u,%u]", name, t->rank, min_rank, max_rank);
    if (numel(t) > 0 && !t->data) return set_error(EVKHIP_ERR_INVALID_ARG, "%s: null data pointer", name);
    return EVKHIP_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static bool same_shape(const evkhip_tensor* a, const evkhip_tensor* b) {
    if (a->rank != b->rank) return false;
    for (uint32_t i = 0; i < a->rank; ++i)
        if (a->dims[i] != b->dims[i]) return false;
    return true;
}

}  // namespace evkhip

using namespace evkhip;

#define CHECK(expr)                 \
    do {                            \
        int _rc = (expr);           \
        if (_rc) return _rc;        \
    } while (0)

extern "C" {

const char* evkhip_version(void) { return "evkhip 0.1 gfx950"; }

const char* evkhip_last_error(void) { return g_err; }

int evkhip_init(void) {
    int dev = 0;
    EVK_HIP(hipGetDevice(&dev));
    (void)device_cu_count();
    GemvScratch s{};
    return noalloc_scratch(&s);  // the static scratch's address on this device
}

int evkhip_shutdown(void) {
    gemm_free_workspace();
    flash_free_workspace();
    decode_ops_free_workspace();
    model_free_workspace();
    decode_persist_free_workspace();
    train_ops_free_workspace();
    kv_step_free_workspace();
    return EVKHIP_OK;
}

int evkhip_device_status(uint32_t* flags, int clear) {
    EVK_RETURN_IF(!flags, EVKHIP_ERR_INVALID_ARG, "device_status: null flags");
    uint32_t f = 0, g = 0;
    int rc = flash_status(&f, clear != 0);
    if (rc != EVKHIP_OK) return rc;
    rc = decode_status(&g, clear != 0);
    if (rc != EVKHIP_OK) return rc;
    uint32_t k = 0;
    rc = kv_step_status(&k, clear != 0);
    if (rc != EVKHIP_OK) return rc;
    *flags = f | g | k;
    return EVKHIP_OK;
}

int evkhip_debug_set_spin_limit(uint32_t iterations) {
    flash_set_spin_limit(iterations);
    return EVKHIP_OK;
}

static int matmul_impl(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, int transpose_a,
                       int transpose_b, int acc_c, uint32_t tile_m, uint32_t tile_n, void* stream,
                       const GemvScratch* fixed) {
    CHECK(check_tensor(a, "matmul: a", 2, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(b, "matmul: b", 2, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(c, "matmul: c", 2, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF((tile_m % 16) || (tile_n % 16), EVKHIP_ERR_INVALID_ARG,
                  "matmul: tile hints must be multiples of 16 (got %u, %u)", tile_m, tile_n);
    // evk_ai.cpp:261-268: batch = max, inputs may broadcast, C must match
    const uint64_t bA = a->rank >= 3 ? batch_of(a, 2) : 1, bB = b->rank >= 3 ? batch_of(b, 2) : 1;
    const uint64_t bC = c->rank >= 3 ? batch_of(c, 2) : 1;
    const uint64_t batch = std::max({bA, bB, bC});
    EVK_RETURN_IF(!(bA == batch || bA == 1) || !(bB == batch || bB == 1) || bC != batch, EVKHIP_ERR_SHAPE,
                  "matmul: batch mismatch (a %llu, b %llu, c %llu)", (unsigned long long)bA,
                  (unsigned long long)bB, (unsigned long long)bC);
    // evk_ai.cpp:273-288: logical dims from the transpose flags
    const uint32_t M = transpose_a ? dim_at(a, -1) : dim_at(a, -2);
    const uint32_t K = transpose_a ? dim_at(a, -2) : dim_at(a, -1);
    const uint32_t Kb = transpose_b ? dim_at(b, -1) : dim_at(b, -2);
    const uint32_t N = transpose_b ? dim_at(b, -2) : dim_at(b, -1);
    EVK_RETURN_IF(K != Kb, EVKHIP_ERR_SHAPE, "matmul: inner dims differ (%u vs %u)", K, Kb);
    EVK_RETURN_IF(dim_at(c, -2) != M || dim_at(c, -1) != N, EVKHIP_ERR_SHAPE,
                  "matmul: c is (%u,%u), expected (%u,%u)", dim_at(c, -2), dim_at(c, -1), M, N);
    EVK_RETURN_IF(batch > 65535 || M > (1u << 30) || N > (1u << 30), EVKHIP_ERR_UNSUPPORTED,
                  "matmul: sizes beyond the kernel's grid limits");
    if (batch == 0 || M == 0 || N == 0) return EVKHIP_OK;
    GemmArgs g{};
    g.A = (const f16*)a->data;
    g.B = (const f16*)b->data;
    g.C = (f16*)c->data;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.sA = (bA == 1 && batch > 1) ? 0 : (int64_t)dim_at(a, -2) * dim_at(a, -1);
    g.sB = (bB == 1 && batch > 1) ? 0 : (int64_t)dim_at(b, -2) * dim_at(b, -1);
    g.sC = (int64_t)M * N;
    g.acc = acc_c ? 1 : 0;
    const bool vec_ok = aligned16(a->data) && aligned16(b->data) && aligned16(c->data) &&
                        (dim_at(a, -1) % 8 == 0) && (dim_at(b, -1) % 8 == 0) && (N % 8 == 0) &&
                        (K % 8 == 0) && (M % 8 == 0 || !transpose_a) && (g.sA % 8 == 0) &&
                        (g.sB % 8 == 0);
    if (K == 0) {
        // C = 0 (or unchanged with acc): a GEMM with an empty contraction
        if (acc_c) return EVKHIP_OK;
        return fill_launch(c->data, 0u, (int64_t)numel(c), aligned16(c->data), as_stream(stream));
    }
    return gemm_dispatch(g, (int)batch, transpose_a != 0, transpose_b != 0, vec_ok, as_stream(stream), fixed);
}

int evkhip_matmul(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, int transpose_a,
                  int transpose_b, int acc_c, uint32_t tile_m, uint32_t tile_n, void* stream) {
    return matmul_impl(a, b, c, transpose_a, transpose_b, acc_c, tile_m, tile_n, stream, nullptr);
}

int evkhip_matmul_noalloc(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, int transpose_a,
                          int transpose_b, int acc_c, uint32_t tile_m, uint32_t tile_n, void* stream) {
    GemvScratch s{};
    CHECK(noalloc_scratch(&s));
    return matmul_impl(a, b, c, transpose_a, transpose_b, acc_c, tile_m, tile_n, stream, &s);
}

static int flash_shapes(const evkhip_tensor* q, const evkhip_tensor* k, const evkhip_tensor* v,
                        const char* op, uint32_t* B, uint32_t* N, uint32_t* D, uint32_t* Dh) {
    CHECK(check_tensor(q, "flash: q", 3, 3));
    CHECK(check_tensor(k, "flash: k", 3, 3));
    CHECK(check_tensor(v, "flash: v", 3, 3));
    *B = q->dims[0];
    *N = q->dims[1];
    *D = q->dims[2];
    *Dh = k->dims[2];
    EVK_RETURN_IF(k->dims[0] != *B || k->dims[1] != *N, EVKHIP_ERR_SHAPE, "%s: k must be (B,N,Dh)", op);
    EVK_RETURN_IF(!same_shape(k, v), EVKHIP_ERR_SHAPE, "%s: v must match k", op);
    EVK_RETURN_IF(*Dh == 0 || *D % *Dh != 0, EVKHIP_ERR_SHAPE, "%s: D=%u not a multiple of Dh=%u", op, *D, *Dh);
    EVK_RETURN_IF(*Dh > 256, EVKHIP_ERR_UNSUPPORTED, "%s: Dh=%u > 256", op, *Dh);
    EVK_RETURN_IF((uint64_t)*N * (*D / *Dh) > (1u << 30), EVKHIP_ERR_UNSUPPORTED, "%s: N*H too large", op);
    EVK_RETURN_IF(*B > 65535, EVKHIP_ERR_UNSUPPORTED, "%s: B too large", op);
    return EVKHIP_OK;
}

int evkhip_flash_has_mfma(uint32_t head_dim) { return flash_mfma_head(head_dim) ? 1 : 0; }

int evkhip_flash_kernel_path(uint32_t n, uint32_t heads, uint32_t head_dim) {
    if (head_dim == 0 || heads == 0 || !flash_mfma_head(head_dim)) return EVKHIP_FLASH_PATH_SCALAR;
    if (flash_wide_head(head_dim))
        return flash_wide_fits(n, heads, head_dim) ? EVKHIP_FLASH_PATH_WIDE : EVKHIP_FLASH_PATH_SCALAR;
    return EVKHIP_FLASH_PATH_MFMA;
}

int evkhip_flash_attention(const evkhip_tensor* q, const evkhip_tensor* k, const evkhip_tensor* v,
                           const evkhip_tensor* o, int causal, float* lse, void* stream) {
    uint32_t B, N, D, Dh;
    CHECK(flash_shapes(q, k, v, "flash_attention", &B, &N, &D, &Dh));
    CHECK(check_tensor(o, "flash_attention: o", 3, 3));
    EVK_RETURN_IF(!same_shape(q, o), EVKHIP_ERR_SHAPE, "flash_attention: o must match q");
    if (B == 0 || N == 0) return EVKHIP_OK;
    const bool mfma = flash_mfma_head(Dh) && aligned16(q->data) && aligned16(k->data) &&
                      aligned16(v->data) && aligned16(o->data);
    FlashArgs a{};
    a.q = (const f16*)q->data;
    a.k = (const f16*)k->data;
    a.v = (const f16*)v->data;
    a.out = (f16*)o->data;
    a.lse = lse;
    a.B = (int)B;
    a.H = (int)(D / Dh);
    a.N = (int)N;
    return flash_forward(a, (int)Dh, mfma, causal != 0, as_stream(stream));
}

int evkhip_flash_attention_bwd(const evkhip_tensor* q, const evkhip_tensor* k, const evkhip_tensor* v,
                               const evkhip_tensor* o, const evkhip_tensor* dO, const evkhip_tensor* dQ,
                               const evkhip_tensor* dK, const evkhip_tensor* dV, uint32_t heads, int causal,
                               const float* lse, void* stream) {
    uint32_t B, N, D, Dh;
    CHECK(flash_shapes(q, k, v, "flash_attention_bwd", &B, &N, &D, &Dh));
    CHECK(check_tensor(dO, "flash_attention_bwd: dO", 3, 3));
    CHECK(check_tensor(dQ, "flash_attention_bwd: dQ", 3, 3));
    CHECK(check_tensor(dK, "flash_attention_bwd: dK", 3, 3));
    CHECK(check_tensor(dV, "flash_attention_bwd: dV", 3, 3));
    EVK_RETURN_IF(!same_shape(q, dO) || !same_shape(q, dQ), EVKHIP_ERR_SHAPE,
                  "flash_attention_bwd: dO and dQ must match q");
    EVK_RETURN_IF(!same_shape(k, dK) || !same_shape(k, dV), EVKHIP_ERR_SHAPE,
                  "flash_attention_bwd: dK and dV must match k");
    const uint32_t H = D / Dh;
    EVK_RETURN_IF(heads != 0 && heads != H, EVKHIP_ERR_SHAPE, "flash_attention_bwd: heads=%u but D/Dh=%u", heads,
                  H);
    if (lse) {
        CHECK(check_tensor(o, "flash_attention_bwd: o", 3, 3));
        EVK_RETURN_IF(!same_shape(q, o), EVKHIP_ERR_SHAPE, "flash_attention_bwd: o must match q");
    }
    if (B == 0 || N == 0) return EVKHIP_OK;
    bool mfma = flash_mfma_head(Dh);
    for (const evkhip_tensor* t : {q, k, v, dO, dQ, dK, dV}) mfma = mfma && aligned16(t->data);
    if (lse) mfma = mfma && aligned16(o->data);
    FlashArgs a{};
    a.q = (const f16*)q->data;
    a.k = (const f16*)k->data;
    a.v = (const f16*)v->data;
    a.o = lse ? (const f16*)o->data : nullptr;
    a.dO = (const f16*)dO->data;
    a.out = (f16*)dQ->data;
    a.dK = (f16*)dK->data;
    a.dV = (f16*)dV->data;
    a.lse = const_cast<float*>(lse);
    a.B = (int)B;
    a.H = (int)H;
    a.N = (int)N;
    return flash_backward(a, (int)Dh, mfma, causal != 0, as_stream(stream));
}

int evkhip_single_query_attention(const evkhip_tensor* q, const evkhip_tensor* k_cache,
                                  const evkhip_tensor* v_cache, const evkhip_tensor* out, uint32_t current_length,
                                  uint32_t heads, void* stream) {
    CHECK(check_tensor(q, "single_query_attention: q", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(k_cache, "single_query_attention: k_cache", 2, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(v_cache, "single_query_attention: v_cache", 2, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "single_query_attention: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(heads == 0, EVKHIP_ERR_INVALID_ARG, "single_query_attention: heads must be >= 1");
    // batched form: caches (B, max_len, D) with B > 1 and q, out holding B*D
    const uint64_t cache_batch = k_cache->rank >= 3 ? batch_of(k_cache, 2) : 1;
    if (cache_batch > 1) {
        const uint64_t Dc = dim_at(k_cache, -1), max_len = dim_at(k_cache, -2);
        EVK_RETURN_IF(!same_shape(k_cache, v_cache), EVKHIP_ERR_SHAPE, "single_query_attention: caches differ");
        EVK_RETURN_IF(numel(q) != cache_batch * Dc || numel(out) != cache_batch * Dc, EVKHIP_ERR_SHAPE,
                      "single_query_attention: %llu cached sequences of %llu values need q and out of %llu values",
                      (unsigned long long)cache_batch, (unsigned long long)Dc,
                      (unsigned long long)(cache_batch * Dc));
        EVK_RETURN_IF(Dc % heads, EVKHIP_ERR_SHAPE, "single_query_attention: %llu values not divisible by %u heads",
                      (unsigned long long)Dc, heads);
        EVK_RETURN_IF(current_length > max_len, EVKHIP_ERR_SHAPE,
                      "single_query_attention: current_length %u exceeds the %llu cached rows", current_length,
                      (unsigned long long)max_len);
        EVK_RETURN_IF(cache_batch > 65535 / heads, EVKHIP_ERR_UNSUPPORTED, "single_query_attention: too many sequences");
        const bool alb = aligned16(q->data) && aligned16(k_cache->data) && aligned16(v_cache->data) &&
                         aligned16(out->data);
        return sq_attention_launch((const f16*)q->data, (const f16*)k_cache->data, (const f16*)v_cache->data,
                                   (f16*)out->data, (int64_t)Dc, (int)heads, (int)(Dc / heads),
                                   (int)current_length, alb, as_stream(stream), (int)cache_batch,
                                   (int64_t)(max_len * Dc));
    }
    const uint64_t D = numel(q);
    EVK_RETURN_IF(D == 0 || D % heads, EVKHIP_ERR_SHAPE, "single_query_attention: q size %llu not divisible by %u heads",
                  (unsigned long long)D, heads);
    EVK_RETURN_IF(numel(out) != D, EVKHIP_ERR_SHAPE, "single_query_attention: out must have q's size");
    EVK_RETURN_IF(!same_shape(k_cache, v_cache), EVKHIP_ERR_SHAPE, "single_query_attention: caches differ");
    EVK_RETURN_IF(dim_at(k_cache, -1) != D, EVKHIP_ERR_SHAPE,
                  "single_query_attention: cache rows hold %u values, q has %llu", dim_at(k_cache, -1),
                  (unsigned long long)D);
    const uint64_t rows = numel(k_cache) / D;
    EVK_RETURN_IF(current_length > rows, EVKHIP_ERR_SHAPE,
                  "single_query_attention: current_length %u exceeds the %llu cached rows", current_length,
                  (unsigned long long)rows);
    const uint32_t dh = (uint32_t)(D / heads);
    const bool al = aligned16(q->data) && aligned16(k_cache->data) && aligned16(v_cache->data);
    return sq_attention_launch((const f16*)q->data, (const f16*)k_cache->data, (const f16*)v_cache->data,
                               (f16*)out->data, (int64_t)D, (int)heads, (int)dh, (int)current_length, al,
                               as_stream(stream));
}

int evkhip_kv_cache_write(const evkhip_tensor* src, const evkhip_tensor* cache, uint32_t pos0, void* stream) {
    CHECK(check_tensor(src, "kv_cache_write: src", 2, 3));
    CHECK(check_tensor(cache, "kv_cache_write: cache", 2, 3));
    const uint32_t B = src->rank == 3 ? src->dims[0] : 1, n = dim_at(src, -2), D = dim_at(src, -1);
    const uint32_t Bc = cache->rank == 3 ? cache->dims[0] : 1, max_seq = dim_at(cache, -2);
    EVK_RETURN_IF(Bc != B || dim_at(cache, -1) != D, EVKHIP_ERR_SHAPE,
                  "kv_cache_write: src (%u,%u,%u) does not match cache (%u,%u,%u)", B, n, D, Bc, max_seq,
                  dim_at(cache, -1));
    EVK_RETURN_IF((uint64_t)pos0 + n > max_seq, EVKHIP_ERR_SHAPE,
                  "kv_cache_write: rows %u..%u exceed the cache's %u", pos0, pos0 + n, max_seq);
    return kv_cache_write_launch((const f16*)src->data, (f16*)cache->data, (int)B, (int)n, (int)D, (int)max_seq,
                                 (int)pos0, as_stream(stream));
}

int evkhip_rms_norm(const evkhip_tensor* in, const evkhip_tensor* out, float eps, void* stream) {
    CHECK(check_tensor(in, "rms_norm: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "rms_norm: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(in, out), EVKHIP_ERR_SHAPE, "rms_norm: shapes differ");
    const uint32_t D = dim_at(in, -1);
    if (D == 0) return EVKHIP_OK;
    return rms_norm_launch((const f16*)in->data, (f16*)out->data, (int64_t)(numel(in) / D), (int)D, eps,
                           as_stream(stream));
}

int evkhip_rope(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t batch_size, uint32_t seq_len,
                uint32_t embed_dim, float rotary_base, uint32_t position_offset, uint32_t head_dim, void* stream) {
    CHECK(check_tensor(in, "rope: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "rope: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(embed_dim % 2, EVKHIP_ERR_SHAPE, "rope: embed_dim %u must be even", embed_dim);
    const uint32_t hd = head_dim ? head_dim : embed_dim;
    EVK_RETURN_IF(hd == 0 || hd % 2 || embed_dim % hd, EVKHIP_ERR_SHAPE,
                  "rope: head_dim %u must be even and divide embed_dim %u", hd, embed_dim);
    const uint64_t n = (uint64_t)batch_size * seq_len * embed_dim;
    EVK_RETURN_IF(numel(in) < n || numel(out) < n, EVKHIP_ERR_SHAPE, "rope: tensors hold fewer than B*S*D values");
    return rope_launch((const f16*)in->data, (f16*)out->data, (int)batch_size, (int)seq_len, (int)embed_dim,
                       rotary_base, (int)position_offset, (int)hd, as_stream(stream));
}

int evkhip_gelu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream) {
    CHECK(check_tensor(in, "gelu: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "gelu: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(in, out), EVKHIP_ERR_SHAPE, "gelu: shapes differ");
    return gelu_launch((const f16*)in->data, (f16*)out->data, (int64_t)numel(in), as_stream(stream));
}

int evkhip_add(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c, void* stream) {
    CHECK(check_tensor(a, "add: a", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(b, "add: b", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(c, "add: c", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(a, b) || !same_shape(a, c), EVKHIP_ERR_SHAPE, "add: shapes differ");
    return add_launch((const f16*)a->data, (const f16*)b->data, (f16*)c->data, (int64_t)numel(a),
                      as_stream(stream));
}

int evkhip_embed(const evkhip_tensor* embeddings, const evkhip_tensor* indices, const evkhip_tensor* out,
                 void* stream) {
    CHECK(check_tensor(embeddings, "embed: embeddings", 2, 2));
    CHECK(check_tensor(indices, "embed: indices", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "embed: out", 1, EVKHIP_MAX_DIMS));
    const uint32_t vocab = embeddings->dims[0], dim = embeddings->dims[1];
    const uint64_t n_idx = numel(indices);
    EVK_RETURN_IF(numel(out) != n_idx * dim, EVKHIP_ERR_SHAPE, "embed: out must hold indices*embed_dim values");
    EVK_RETURN_IF(vocab == 0 && n_idx > 0, EVKHIP_ERR_SHAPE, "embed: empty table");
    return embed_launch((const f16*)embeddings->data, (const uint16_t*)indices->data, (f16*)out->data,
                        (int64_t)n_idx, (int)dim, (int)vocab, as_stream(stream));
}

int evkhip_greedy_sample(const evkhip_tensor* logits, const evkhip_tensor* out_tokens, uint32_t position,
                         uint16_t token_base, uint16_t token_count, void* stream) {
    CHECK(check_tensor(logits, "greedy_sample: logits", 3, 3));
    CHECK(check_tensor(out_tokens, "greedy_sample: out_tokens", 1, 1));
    const uint32_t B = logits->dims[0], S = logits->dims[1], V = logits->dims[2];
    EVK_RETURN_IF(out_tokens->dims[0] != B, EVKHIP_ERR_SHAPE, "greedy_sample: out_tokens must be (B)");
    EVK_RETURN_IF(position >= S, EVKHIP_ERR_SHAPE, "greedy_sample: position %u >= seq_len %u", position, S);
    EVK_RETURN_IF((uint32_t)token_base + token_count > V, EVKHIP_ERR_SHAPE,
                  "greedy_sample: token range exceeds vocab");
    return greedy_launch((const f16*)logits->data, (uint16_t*)out_tokens->data, (int)B, (int)S, (int)V,
                         (int)position, token_base, token_count, as_stream(stream));
}

// ---- training ops ----

static bool all_aligned(std::initializer_list<const evkhip_tensor*> ts) {
    for (const evkhip_tensor* x : ts)
        if (!aligned16(x->data)) return false;
    return true;
}

int evkhip_fill(void* data, uint64_t bytes, uint32_t pattern, void* stream) {
    EVK_RETURN_IF(bytes & 1, EVKHIP_ERR_INVALID_ARG, "fill: %llu bytes is not a whole number of 16-bit words",
                  (unsigned long long)bytes);
    EVK_RETURN_IF(bytes && (!data || (reinterpret_cast<uintptr_t>(data) & 1)), EVKHIP_ERR_INVALID_ARG,
                  "fill: null or odd data pointer");
    return fill_launch(data, pattern, (int64_t)(bytes / 2), aligned16(data), as_stream(stream));
}

int evkhip_scale(const evkhip_tensor* t, float factor, void* stream) {
    CHECK(check_tensor(t, "scale: tensor", 1, EVKHIP_MAX_DIMS));
    return scale_launch((f16*)t->data, factor, (int64_t)numel(t), all_aligned({t}), as_stream(stream));
}

int evkhip_relu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream) {
    CHECK(check_tensor(in, "relu: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "relu: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(in, out), EVKHIP_ERR_SHAPE, "relu: shapes differ");
    return relu_launch((const f16*)in->data, (f16*)out->data, (int64_t)numel(in), all_aligned({in, out}),
                       as_stream(stream));
}

int evkhip_relu_backward(const evkhip_tensor* grad_out, const evkhip_tensor* in, const evkhip_tensor* grad_in,
                         void* stream) {
    CHECK(check_tensor(grad_out, "relu_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(in, "relu_backward: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "relu_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    const uint64_t n = numel(in);
    EVK_RETURN_IF(numel(grad_out) != n || numel(grad_in) != n, EVKHIP_ERR_SHAPE,
                  "relu_backward: element counts differ");
    return relu_bwd_launch((const f16*)grad_out->data, (const f16*)in->data, (f16*)grad_in->data, (int64_t)n,
                           all_aligned({grad_out, in, grad_in}), as_stream(stream));
}

int evkhip_gelu_backward(const evkhip_tensor* grad_out, const evkhip_tensor* in, const evkhip_tensor* grad_in,
                         void* stream) {
    CHECK(check_tensor(grad_out, "gelu_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(in, "gelu_backward: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "gelu_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    const uint64_t n = numel(in);
    EVK_RETURN_IF(numel(grad_out) != n || numel(grad_in) != n, EVKHIP_ERR_SHAPE,
                  "gelu_backward: element counts differ");
    return gelu_bwd_launch((const f16*)grad_out->data, (const f16*)in->data, (f16*)grad_in->data, (int64_t)n,
                           all_aligned({grad_out, in, grad_in}), as_stream(stream));
}

int evkhip_mse_loss(const evkhip_tensor* predicted, const evkhip_tensor* target, const evkhip_tensor* pred_grad,
                    const evkhip_tensor* result, void* stream) {
    CHECK(check_tensor(predicted, "mse_loss: predicted", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(target, "mse_loss: target", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(pred_grad, "mse_loss: pred_grad", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(result, "mse_loss: result", 1, 1));
    EVK_RETURN_IF(!same_shape(predicted, target), EVKHIP_ERR_SHAPE, "mse_loss: predicted and target differ");
    EVK_RETURN_IF(numel(pred_grad) != numel(predicted), EVKHIP_ERR_SHAPE, "mse_loss: pred_grad size");
    EVK_RETURN_IF(result->dims[0] < 1, EVKHIP_ERR_SHAPE, "mse_loss: result must hold one value");
    return mse_loss_launch((const f16*)predicted->data, (const f16*)target->data, (f16*)pred_grad->data,
                           (f16*)result->data, (int64_t)numel(predicted), as_stream(stream));
}

int evkhip_sgd(const evkhip_tensor* param, const evkhip_tensor* gradient, float learning_rate, void* stream) {
    CHECK(check_tensor(param, "sgd: param", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(gradient, "sgd: gradient", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(param, gradient), EVKHIP_ERR_SHAPE, "sgd: param and gradient differ");
    return sgd_launch((f16*)param->data, (const f16*)gradient->data, learning_rate, (int64_t)numel(param),
                      all_aligned({param, gradient}), as_stream(stream));
}

int evkhip_adam(const evkhip_tensor* param, const evkhip_tensor* gradient, const evkhip_tensor* m_state,
                const evkhip_tensor* v_state, float learning_rate, float beta1, float beta2,
                float beta1_correction_inv, float beta2_correction_inv, float epsilon, void* stream) {
    CHECK(check_tensor(param, "adam: param", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(gradient, "adam: gradient", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(m_state, "adam: m_state", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(v_state, "adam: v_state", 1, EVKHIP_MAX_DIMS));
    const uint64_t n = numel(param);
    EVK_RETURN_IF(!same_shape(param, gradient), EVKHIP_ERR_SHAPE, "adam: param and gradient differ");
    EVK_RETURN_IF(numel(m_state) != n || numel(v_state) != n, EVKHIP_ERR_SHAPE,
                  "adam: state must hold one value per parameter");
    return adam_launch((f16*)param->data, (const f16*)gradient->data, (f16*)m_state->data, (f16*)v_state->data,
                       (int64_t)n, learning_rate, beta1, beta2, beta1_correction_inv, beta2_correction_inv, epsilon,
                       all_aligned({param, gradient, m_state, v_state}), as_stream(stream));
}

int evkhip_softmax(const evkhip_tensor* in, const evkhip_tensor* out, float input_scale, void* stream) {
    CHECK(check_tensor(in, "softmax: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "softmax: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(in, out), EVKHIP_ERR_SHAPE, "softmax: shapes differ");
    const uint32_t D = dim_at(in, -1);
    if (D == 0) return EVKHIP_OK;
    return softmax_launch((const f16*)in->data, (f16*)out->data, input_scale, (int)D, (int64_t)(numel(in) / D),
                          all_aligned({in, out}), as_stream(stream));
}

int evkhip_softmax_backward(const evkhip_tensor* probs, const evkhip_tensor* grad_out,
                            const evkhip_tensor* grad_in, float scale, void* stream) {
    CHECK(check_tensor(probs, "softmax_backward: probs", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_out, "softmax_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "softmax_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(probs, grad_out) || !same_shape(probs, grad_in), EVKHIP_ERR_SHAPE,
                  "softmax_backward: shapes differ");
    const uint32_t D = dim_at(probs, -1);
    if (D == 0) return EVKHIP_OK;
    return softmax_bwd_launch((const f16*)probs->data, (const f16*)grad_out->data, (f16*)grad_in->data, scale,
                              (int)D, (int64_t)(numel(probs) / D), as_stream(stream));
}

int evkhip_rms_norm_backward(const evkhip_tensor* in, const evkhip_tensor* grad_out,
                             const evkhip_tensor* grad_in, float eps, void* stream) {
    CHECK(check_tensor(in, "rms_norm_backward: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_out, "rms_norm_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "rms_norm_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(!same_shape(in, grad_out) || !same_shape(in, grad_in), EVKHIP_ERR_SHAPE,
                  "rms_norm_backward: shapes differ");
    const uint32_t D = dim_at(in, -1);
    if (D == 0) return EVKHIP_OK;
    return rms_norm_bwd_launch((const f16*)in->data, (const f16*)grad_out->data, (f16*)grad_in->data, eps, (int)D,
                               (int64_t)(numel(in) / D), as_stream(stream));
}

int evkhip_cross_entropy_loss(const evkhip_tensor* logits, const evkhip_tensor* targets,
                              const evkhip_tensor* grad, const evkhip_tensor* result, void* stream) {
    CHECK(check_tensor(logits, "cross_entropy_loss: logits", 2, 2));
    CHECK(check_tensor(targets, "cross_entropy_loss: targets", 1, 1));
    CHECK(check_tensor(grad, "cross_entropy_loss: grad", 2, 2));
    CHECK(check_tensor(result, "cross_entropy_loss: result", 1, 1));
    const uint32_t P = logits->dims[0], V = logits->dims[1];
    EVK_RETURN_IF(targets->dims[0] != P, EVKHIP_ERR_SHAPE, "cross_entropy_loss: targets must be (positions)");
    EVK_RETURN_IF(!same_shape(logits, grad), EVKHIP_ERR_SHAPE, "cross_entropy_loss: grad must match logits");
    EVK_RETURN_IF(result->dims[0] != 1, EVKHIP_ERR_SHAPE, "cross_entropy_loss: result must be (1)");
    EVK_RETURN_IF(V == 0 && P > 0, EVKHIP_ERR_SHAPE, "cross_entropy_loss: empty vocabulary");
    return cross_entropy_launch((const f16*)logits->data, (const uint16_t*)targets->data, (f16*)grad->data,
                                (f16*)result->data, (int64_t)P, (int)V, all_aligned({logits, grad}),
                                as_stream(stream));
}

int evkhip_sum_batch(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t batch_count,
                     uint32_t size_per_batch, void* stream) {
    CHECK(check_tensor(in, "sum_batch: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "sum_batch: out", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(numel(in) < (uint64_t)batch_count * size_per_batch || numel(out) < size_per_batch,
                  EVKHIP_ERR_SHAPE, "sum_batch: tensors hold fewer than batch_count*size_per_batch values");
    return sum_batch_launch((const f16*)in->data, (f16*)out->data, (int)batch_count, (int64_t)size_per_batch,
                            as_stream(stream));
}

int evkhip_apply_causal_mask(const evkhip_tensor* scores, void* stream) {
    CHECK(check_tensor(scores, "apply_causal_mask: scores", 2, EVKHIP_MAX_DIMS));
    const uint32_t N = dim_at(scores, -1);
    EVK_RETURN_IF(dim_at(scores, -2) != N, EVKHIP_ERR_SHAPE, "apply_causal_mask: scores must be (..., N, N)");
    if (N == 0) return EVKHIP_OK;
    return causal_mask_launch((f16*)scores->data, (int64_t)(numel(scores) / ((uint64_t)N * N)), (int)N,
                              as_stream(stream));
}

int evkhip_position_add(const evkhip_tensor* in, const evkhip_tensor* pos_emb, const evkhip_tensor* out,
                        uint32_t batch_size, uint32_t seq_len, uint32_t embed_dim, void* stream) {
    CHECK(check_tensor(in, "position_add: in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(pos_emb, "position_add: pos_emb", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(out, "position_add: out", 1, EVKHIP_MAX_DIMS));
    const uint64_t per = (uint64_t)seq_len * embed_dim, n = per * batch_size;
    EVK_RETURN_IF(numel(in) < n || numel(out) < n || numel(pos_emb) < per, EVKHIP_ERR_SHAPE,
                  "position_add: tensors hold fewer than B*N*D (pos_emb N*D) values");
    return position_add_launch((const f16*)in->data, (const f16*)pos_emb->data, (f16*)out->data, (int)batch_size,
                               (int64_t)per, as_stream(stream));
}

int evkhip_position_add_backward(const evkhip_tensor* grad_out, const evkhip_tensor* grad_in,
                                 const evkhip_tensor* grad_pos, uint32_t batch_size, uint32_t seq_len,
                                 uint32_t embed_dim, void* stream) {
    CHECK(check_tensor(grad_out, "position_add_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "position_add_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_pos, "position_add_backward: grad_pos", 1, EVKHIP_MAX_DIMS));
    const uint64_t per = (uint64_t)seq_len * embed_dim, n = per * batch_size;
    EVK_RETURN_IF(numel(grad_out) < n || numel(grad_in) < n || numel(grad_pos) < per, EVKHIP_ERR_SHAPE,
                  "position_add_backward: tensors hold fewer than B*N*D (grad_pos N*D) values");
    return position_add_bwd_launch((const f16*)grad_out->data, (f16*)grad_in->data, (f16*)grad_pos->data,
                                   (int)batch_size, (int64_t)per, as_stream(stream));
}

int evkhip_rope_backward(const evkhip_tensor* grad_out, const evkhip_tensor* grad_in, uint32_t batch_size,
                         uint32_t seq_len, uint32_t embed_dim, float rotary_base, void* stream) {
    CHECK(check_tensor(grad_out, "rope_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_in, "rope_backward: grad_in", 1, EVKHIP_MAX_DIMS));
    EVK_RETURN_IF(embed_dim % 2, EVKHIP_ERR_SHAPE, "rope_backward: embed_dim %u must be even", embed_dim);
    const uint64_t n = (uint64_t)batch_size * seq_len * embed_dim;
    EVK_RETURN_IF(numel(grad_out) < n || numel(grad_in) < n, EVKHIP_ERR_SHAPE,
                  "rope_backward: tensors hold fewer than B*S*D values");
    return rope_bwd_launch((const f16*)grad_out->data, (f16*)grad_in->data, (int)batch_size, (int)seq_len,
                           (int)embed_dim, rotary_base, as_stream(stream));
}

int evkhip_embed_backward(const evkhip_tensor* grad_out, const evkhip_tensor* indices,
                          const evkhip_tensor* grad_embeddings, void* stream) {
    CHECK(check_tensor(grad_out, "embed_backward: grad_out", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(indices, "embed_backward: indices", 1, EVKHIP_MAX_DIMS));
    CHECK(check_tensor(grad_embeddings, "embed_backward: grad_embeddings", 2, 2));
    const uint32_t vocab = grad_embeddings->dims[0], dim = grad_embeddings->dims[1];
    const uint64_t n_idx = numel(indices);
    EVK_RETURN_IF(numel(grad_out) != n_idx * dim, EVKHIP_ERR_SHAPE,
                  "embed_backward: grad_out must hold indices*embed_dim values");
    return embed_bwd_launch((const f16*)grad_out->data, (const uint16_t*)indices->data, (f16*)grad_embeddings->data,
                            (int64_t)n_idx, (int)dim, (int)vocab, as_stream(stream));
}

}  // extern "C"
