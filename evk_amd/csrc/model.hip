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
ModelWs g_ws;   // unfused path (fp16 elements)
ModelWs g_fws;  // fused path (bytes in `elems`)
// Counters of the fused kernels: their own grow-only array, zeroed when it
// grows; every launch leaves them at zero, so any configuration can reuse them.
unsigned* g_fcnt = nullptr;
size_t g_fcnt_n = 0;

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

// ---------------------------------------------------------------------------
// Fused decode step: five kernels per layer and one for the LM head.  Each
// GEMV workgroup owns a 64-column block (one 128-byte line of every weight
// row) over all K rows and runs its epilogue itself:
//   qkv  : rms_norm(x) . Wqkv -> rope(q), rope(k), cache append (layer 0
//          first takes x from the embedding row of the step's token)
//   attn : single-query attention split over the cache, merged per head
//   wo   : att . Wo, x += (residual)
//   w1   : rms_norm(x) . W1 -> gelu
//   w2   : gelu . W2, x += (residual)
//   head : rms_norm(x) . Wout -> logits, greedy argmax (shader tie order)
// Rounding points are those of the unfused op sequence (every op output is
// fp16).  Partial sums are combined in a fixed order, so results do not
// depend on which workgroup finishes last.
// Cross-workgroup values are written and read with agent-scope atomics
// (straight to the device coherence point, no L2 flush or invalidate), and
// a workgroup counts itself in only after those stores have completed.
// Counters are left at zero by the workgroup that consumes them.
// ---------------------------------------------------------------------------
constexpr int GCB = 64;   // GEMV output columns per workgroup (128 bytes of a weight row)
constexpr int ULD = 8;    // loads a thread keeps in flight

struct DecArgs {
    int d, heads, dh, hidden, vocab, max_seq;
    float eps, rope_base;
    f16* x;            // residual stream (d)
    f16* q;            // rope'd query (d)
    f16* att;          // attention output (d)
    f16* hg;           // gelu(x . W1) (hidden)
    float* cand_v;     // LM-head block winners
    uint32_t* cand_r;
    unsigned* cnt;     // counters (zero between launches)
};

DEV void st_ag(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV float ld_ag(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void st_ag(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV uint32_t ld_ag(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

DEV bool arrive_last(unsigned* cnt, unsigned total) {
    __shared__ unsigned s_last;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev + 1 == total);
        if (s_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    return s_last;
}

// sum_{k < n} p[k * stride], k ascending, with ULD loads in flight
DEV float sum_strided_ag(const float* p, int n, int64_t stride) {
    float s = 0.0f;
    for (int k0 = 0; k0 < n; k0 += ULD) {
        float v[ULD];
#pragma unroll
        for (int u = 0; u < ULD; ++u) v[u] = (k0 + u < n) ? ld_ag(p + (int64_t)(k0 + u) * stride) : 0.0f;
#pragma unroll
        for (int u = 0; u < ULD; ++u) s += v[u];
    }
    return s;
}

// Sum of squares of x (clamped to the fp16 range as rms_norm.comp does), in
// the same order in every workgroup.
template <int NT>
DEV float block_sumsq(const f16* x, int d, float* red) {
    float ss = 0.0f;
    for (int j = threadIdx.x; j < d; j += NT) {
        const float v = fminf(fmaxf((float)x[j], -65504.0f), 65504.0f);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
    for (int w = 0; w < NT / 64; ++w) ss += red[w];
    __syncthreads();
    return ss;
}

enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_EMBED_RMS = 2 };
enum { EPI_QKV = 0, EPI_RESID = 1, EPI_GELU = 2, EPI_HEAD = 3 };

struct GemvJob {
    const f16* in;    // input vector (PRO_PLAIN), or x (rms prologues)
    const f16* W;     // (K, N) row-major
    int K, N;
    // epilogue targets
    f16* Kc;          // EPI_QKV: this layer's caches
    f16* Vc;
    int pos;
    const f16* E;     // PRO_EMBED_RMS: embedding table and the step's token
    const uint16_t* tok;
    f16* logits;      // EPI_HEAD
    uint16_t* out_id;
};

// GEMV over all K rows of a block of NCB output columns (one 128-byte line of
// each weight row when NCB = 64), with a prologue on the input vector and an
// epilogue on the block's outputs in the same workgroup: no cross-workgroup
// partials on the path.  NT threads = NCB/8 column groups x row groups; a
// thread issues LD 16-byte weight loads before it waits, so that a block's
// rows are in flight at once (256 threads x 24 loads cover K = 768).  Grid:
// ceil(N / NCB); the input vector (K floats) lives in dynamic LDS.
template <int NCB, int NT, int LD, int PRO, int EPI>
__global__ __launch_bounds__(NT) void dec_gemv(DecArgs a, GemvJob j) {
    constexpr int GLD = LD;
    constexpr int CG = NCB / 8, RG = NT / CG;
    extern __shared__ float hv[];  // K input values
    __shared__ float red[RG * NCB];
    __shared__ float y[NCB];
    __shared__ float s_v[NT / 64];
    __shared__ uint32_t s_r[NT / 64];
    const int N = j.N, K = j.K;
    const int cb = blockIdx.x, c0 = cb * NCB, nc = min(NCB, N - c0);

    // The first batch of weight loads goes out before the prologue: the
    // weights do not depend on the input vector, so both latencies overlap.
    const int cg = threadIdx.x % CG, rg = threadIdx.x / CG;
    const int col = c0 + cg * 8;
    const bool col_ok = col < N;
    const f16* wp = j.W + col;
    half8 w[GLD];
    auto load_batch = [&](int i0) {
#pragma unroll
        for (int u = 0; u < GLD; ++u) {
            const int i = i0 + u * RG;
            w[u] = (col_ok && i < K) ? *reinterpret_cast<const half8*>(wp + (int64_t)i * N) : half8{};
        }
    };
    load_batch(rg);

    // ---- prologue: the input vector as fp16 values ----
    if (PRO == PRO_PLAIN) {
        for (int i = threadIdx.x; i < K; i += NT) hv[i] = (float)j.in[i];
    } else {
        const f16* x = j.in;
        if (PRO == PRO_EMBED_RMS) {
            x = j.E + (int64_t)min((int)j.tok[0], a.vocab - 1) * K;
            if (blockIdx.x == 0)
                for (int t = threadIdx.x; t < K; t += NT) a.x[t] = x[t];
        }
        const float ss = block_sumsq<NT>(x, K, red);
        const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
        for (int i = threadIdx.x; i < K; i += NT) {
            const float v = fminf(fmaxf((float)x[i], -65504.0f), 65504.0f);
            hv[i] = (float)(f16)(v * inv);
        }
    }
    __syncthreads();

    // ---- the block's dot products ----
    {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int i0 = rg; i0 < K; i0 += RG * GLD) {
            if (i0 != rg) load_batch(i0);
#pragma unroll
            for (int u = 0; u < GLD; ++u) {
                const int i = i0 + u * RG;
                const float h = (i < K) ? hv[i] : 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += h * (float)w[u][e];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) red[rg * NCB + cg * 8 + e] = acc[e];
        __syncthreads();
        for (int c = threadIdx.x; c < NCB; c += NT) {
            float s = 0.0f;
            for (int r = 0; r < RG; ++r) s += red[r * NCB + c];
            y[c] = (float)(f16)s;  // fp16 output of the product
        }
        __syncthreads();
    }

    // ---- epilogue ----
    if (EPI == EPI_QKV) {
        const int d = a.d;
        for (int c = threadIdx.x; c < nc; c += NT) {
            const int col = c0 + c;
            const int part = col / d, jj = col % d;
            if (part == 2) {
                j.Vc[(int64_t)j.pos * d + jj] = (f16)y[c];
                continue;
            }
            const float x0 = y[c & ~1], x1 = y[c | 1];
            const int pp = (jj % a.dh) / 2;
            const float inv_freq = powf(a.rope_base, -2.0f * (float)pp / (float)a.dh);
            const float ang = (float)j.pos * inv_freq;
            float sn, cs;
            sincosf(ang, &sn, &cs);
            const f16 r = (f16)((c & 1) ? (x0 * sn + x1 * cs) : (x0 * cs - x1 * sn));
            if (part == 0) a.q[jj] = r;
            else j.Kc[(int64_t)j.pos * d + jj] = r;
        }
    } else if (EPI == EPI_RESID) {
        for (int c = threadIdx.x; c < nc; c += NT)
            a.x[c0 + c] = (f16)((float)a.x[c0 + c] + y[c]);
    } else if (EPI == EPI_GELU) {
        for (int c = threadIdx.x; c < nc; c += NT) a.hg[c0 + c] = (f16)gelu_f(y[c]);
    } else {  // EPI_HEAD: logits, then the greedy winner over all blocks
        const int ncb = (N + NCB - 1) / NCB;
        float bv = -3.402823466e+38f;
        uint32_t br = 0u;
        for (int c = threadIdx.x; c < nc; c += NT) {
            const f16 lg = (f16)y[c];
            j.logits[c0 + c] = lg;
            const float v = (float)lg;
            const uint32_t r = greedy_rank((uint32_t)(c0 + c));
            if (v > -3.402823466e+38f && greedy_better(v, r, bv, br)) { bv = v; br = r; }
        }
        auto block_best = [&]() {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float v2 = __shfl_xor(bv, o, 64);
                const uint32_t r2 = __shfl_xor(br, o, 64);
                if (greedy_better(v2, r2, bv, br)) { bv = v2; br = r2; }
            }
            if ((threadIdx.x & 63) == 0) { s_v[threadIdx.x >> 6] = bv; s_r[threadIdx.x >> 6] = br; }
            __syncthreads();
            bv = s_v[0];
            br = s_r[0];
            for (int w = 1; w < NT / 64; ++w)
                if (greedy_better(s_v[w], s_r[w], bv, br)) { bv = s_v[w]; br = s_r[w]; }
            __syncthreads();
        };
        block_best();
        if (threadIdx.x == 0) {
            st_ag(a.cand_v + cb, bv);
            st_ag(a.cand_r + cb, br);
        }
        if (!arrive_last(a.cnt, ncb)) return;
        bv = -3.402823466e+38f;
        br = 0u;
        for (int k0 = threadIdx.x; k0 < ncb; k0 += NT) {
            const float cv = ld_ag(a.cand_v + k0);
            const uint32_t cr = ld_ag(a.cand_r + k0);
            if (greedy_better(cv, cr, bv, br)) { bv = cv; br = cr; }
        }
        block_best();
        if (threadIdx.x == 0) *j.out_id = (uint16_t)greedy_index(br);
    }
}

// Single-query attention of one layer, one 1024-thread workgroup per head.
// A pass covers ATT_KPT * 1024 / (dh / 16) keys; every K and V row of the
// pass is requested before any arithmetic (a thread scores ATT_KPT keys with
// dh / 16 lanes per key and sums 2 * ATT_KPT value rows of 8 dims), so the
// head's cache arrives in one round trip per pass.  Scores, softmax and the
// value sum stay in the workgroup; caches longer than a pass loop with an
// online rescale.  Loads go through buffer descriptors over the valid rows
// [0, L) with the whole offset in the range-checked vector operand, so rows
// past the chain read as zeros.
constexpr int ATT_NT = 1024;
constexpr int ATT_KPT = 5;
constexpr int ATT_VR = 2 * ATT_KPT;

__global__ __launch_bounds__(ATT_NT) void dec_attn(DecArgs a, const f16* Kc, const f16* Vc, int L) {
    __shared__ float sc[ATT_KPT * ATT_NT];
    __shared__ float red[ATT_NT * 2];
    __shared__ float stat[2 * (ATT_NT / 64)];
    const int d = a.d, dh = a.dh, h = blockIdx.x;
    const float scale = 1.0f / sqrtf((float)dh);
    const int tpk = dh / 16, kstep = ATT_NT / tpk, kpp = ATT_KPT * kstep;
    const int ndg = dh / 8, G = ATT_NT / ndg;
    const int kl = threadIdx.x / tpk, part = threadIdx.x % tpk;
    const int dg = threadIdx.x % ndg, kg = threadIdx.x / ndg;
    const uint32_t row = (uint32_t)d * 2;  // bytes per cache row
    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(Kc, (uint32_t)L * row);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(Vc, (uint32_t)L * row);
    const uint32_t kvo = (uint32_t)kl * row + (uint32_t)(h * dh + part * 16) * 2;
    const uint32_t vvo = (uint32_t)kg * row + (uint32_t)(h * dh + dg * 8) * 2;
    const half8* qp = reinterpret_cast<const half8*>(a.q + h * dh + part * 16);
    const half8 q0 = qp[0], q1 = qp[1];
    float m_run = -INFINITY, l_run = 0.0f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < L; p0 += kpp) {
        const int np = min(kpp, L - p0);
        half8 kv[ATT_KPT][2], v[ATT_VR];
#pragma unroll
        for (int t = 0; t < ATT_KPT; ++t) {
            const uint32_t vo = kvo + (uint32_t)(p0 + t * kstep) * row;
            kv[t][0] = as_half8(buf_load16(kres, vo, 0));
            kv[t][1] = as_half8(buf_load16(kres, vo + 16, 0));
        }
#pragma unroll
        for (int u = 0; u < ATT_VR; ++u) v[u] = as_half8(buf_load16(vres, vvo + (uint32_t)(p0 + u * G) * row, 0));
        // scores
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < ATT_KPT; ++t) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                s = __builtin_amdgcn_fdot2(half2_t{q0[e], q0[e + 1]}, half2_t{kv[t][0][e], kv[t][0][e + 1]}, s, false);
                s = __builtin_amdgcn_fdot2(half2_t{q1[e], q1[e + 1]}, half2_t{kv[t][1][e], kv[t][1][e + 1]}, s, false);
            }
            for (int o2 = 1; o2 < tpk; o2 <<= 1) s += __shfl_xor(s, o2, 64);
            const int k = kl + t * kstep;
            s = (k < np) ? s * scale : -INFINITY;
            if (part == 0) sc[k] = s;
            mx = fmaxf(mx, s);
        }
        mx = wave_max(mx);
        if ((threadIdx.x & 63) == 0) stat[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = stat[0];
#pragma unroll
        for (int w = 1; w < ATT_NT / 64; ++w) mx = fmaxf(mx, stat[w]);
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_run == -INFINITY) ? 0.0f : expf(m_run - m_new);
        // probabilities, written back by the lanes that stored the scores
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < ATT_KPT; ++t) {
            const int k = kl + t * kstep;
            if (part == 0) {
                const float x = sc[k];
                const float pe = (x == -INFINITY) ? 0.0f : expf(x - m_new);
                sc[k] = pe;
                ps += pe;
            }
        }
        ps = wave_sum(ps);
        if ((threadIdx.x & 63) == 0) stat[ATT_NT / 64 + (threadIdx.x >> 6)] = ps;
        __syncthreads();
        ps = 0.0f;
#pragma unroll
        for (int w = 0; w < ATT_NT / 64; ++w) ps += stat[ATT_NT / 64 + w];
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
        for (int u = 0; u < ATT_VR; ++u) {
            const float pk = sc[kg + u * G];  // zero past np (rows read as zeros too)
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += pk * (float)v[u][e];
        }
        __syncthreads();  // sc and stat are rewritten by the next pass
    }
    // sum over the key groups: per dim group, G partial vectors of 8
    // values, reduced through LDS in 4 rounds of a quarter of the threads
    float tot = 0.0f;
    const int dg2 = threadIdx.x / 8, e2 = threadIdx.x % 8;
    for (int r = 0; r < 4; ++r) {
        if (threadIdx.x / (ATT_NT / 4) == r)
#pragma unroll
            for (int e = 0; e < 8; ++e) red[(threadIdx.x % (ATT_NT / 4)) * 8 + e] = o[e];
        __syncthreads();
        if (threadIdx.x < dh)
            for (int g = 0; g < G / 4; ++g) tot += red[(g * ndg + dg2) * 8 + e2];
        __syncthreads();
    }
    if (threadIdx.x < dh) a.att[h * dh + threadIdx.x] = (f16)(l_run > 0.0f ? tot / l_run : 0.0f);
}

}  // namespace

void model_free_workspace() {
    if (g_ws.buf) (void)hipFree(g_ws.buf);
    g_ws = ModelWs{};
    if (g_fws.buf) (void)hipFree(g_fws.buf);
    g_fws = ModelWs{};
    if (g_fcnt) (void)hipFree(g_fcnt);
    g_fcnt = nullptr;
    g_fcnt_n = 0;
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
// Rows in flight: 256 threads x 24 loads cover K <= 768 in one batch;
// longer rows take 1024 threads x 12 loads per batch (K = 3072: two batches).
template <int PRO, int EPI>
void launch_gemv(dim3 grid, int K, const DecArgs& a, const GemvJob& j, hipStream_t st) {
    const size_t lds = (size_t)K * sizeof(float);
    if (K <= 24 * (256 / (GCB / 8)))
        hipLaunchKernelGGL((dec_gemv<GCB, 256, 24, PRO, EPI>), grid, dim3(256), lds, st, a, j);
    else
        hipLaunchKernelGGL((dec_gemv<GCB, 1024, 12, PRO, EPI>), grid, dim3(1024), lds, st, a, j);
}

// Fused path: five kernels per layer and one LM-head kernel per token.
int run_tokens_fused(const evkhip_model_cfg& c, const f16* E, const f16* Wout, uint64_t per_layer, f16* cache_h,
                     const uint16_t* feed, uint16_t* ids, uint32_t n, uint32_t pos0, f16* logits, hipStream_t st) {
    const int d = (int)c.d, hid = (int)c.hidden, V = (int)c.vocab, H = (int)c.heads, dh = (int)c.dh;
    auto cdiv = [](int x, int y) { return (x + y - 1) / y; };
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t cnt_n = 1;  // the LM head's arrival counter
    const size_t off_q = al((size_t)d * 2), off_att = off_q + al((size_t)d * 2);
    const size_t off_hg = off_att + al((size_t)d * 2);
    const size_t off_cv = off_hg + al((size_t)hid * 2);
    const size_t off_cr = off_cv + al((size_t)cdiv(V, GCB) * 4);
    const size_t need = off_cr + al((size_t)cdiv(V, GCB) * 4);
    if (need > g_fws.elems) {
        if (g_fws.buf) EVK_HIP(hipFree(g_fws.buf));
        g_fws.buf = nullptr;
        g_fws.elems = 0;
        EVK_HIP(hipMalloc(&g_fws.buf, need));
        g_fws.elems = need;
    }
    if (cnt_n > g_fcnt_n) {
        if (g_fcnt) EVK_HIP(hipFree(g_fcnt));
        g_fcnt = nullptr;
        g_fcnt_n = 0;
        EVK_HIP(hipMalloc(&g_fcnt, cnt_n * sizeof(unsigned)));
        EVK_HIP(hipMemsetAsync(g_fcnt, 0, cnt_n * sizeof(unsigned), st));
        g_fcnt_n = cnt_n;
    }
    char* base = reinterpret_cast<char*>(g_fws.buf);
    DecArgs a{};
    a.d = d; a.heads = H; a.dh = dh; a.hidden = hid; a.vocab = V; a.max_seq = (int)c.max_seq;
    a.eps = c.eps; a.rope_base = c.rope_base;
    a.x = reinterpret_cast<f16*>(base);
    a.q = reinterpret_cast<f16*>(base + off_q);
    a.att = reinterpret_cast<f16*>(base + off_att);
    a.hg = reinterpret_cast<f16*>(base + off_hg);
    a.cand_v = reinterpret_cast<float*>(base + off_cv);
    a.cand_r = reinterpret_cast<uint32_t*>(base + off_cr);
    a.cnt = g_fcnt;
    auto grid = [&](int N) { return dim3((unsigned)cdiv(N, GCB)); };
    for (uint32_t s = 0; s < n; ++s) {
        const int pos = (int)(pos0 + s);
        const uint16_t* tok = feed ? feed + s : ids + s;
        for (uint32_t l = 0; l < c.layers; ++l) {
            const f16* Wqkv = E + (uint64_t)c.vocab * d + l * per_layer;
            const f16* Wo = Wqkv + (uint64_t)d * 3 * d;
            const f16* W1 = Wo + (uint64_t)d * d;
            const f16* W2 = W1 + (uint64_t)d * hid;
            f16* Kc = cache_h + (uint64_t)l * 2 * c.max_seq * d;
            f16* Vc = Kc + (uint64_t)c.max_seq * d;
            GemvJob j{};
            j.in = a.x; j.W = Wqkv; j.K = d; j.N = 3 * d; j.Kc = Kc; j.Vc = Vc; j.pos = pos; j.E = E; j.tok = tok;
            if (l == 0)
                launch_gemv<PRO_EMBED_RMS, EPI_QKV>(grid(3 * d), d, a, j, st);
            else
                launch_gemv<PRO_RMS, EPI_QKV>(grid(3 * d), d, a, j, st);
            hipLaunchKernelGGL(dec_attn, dim3((unsigned)H), dim3(ATT_NT), 0, st, a, (const f16*)Kc, (const f16*)Vc,
                               pos + 1);
            GemvJob jo{};
            jo.in = a.att; jo.W = Wo; jo.K = d; jo.N = d;
            launch_gemv<PRO_PLAIN, EPI_RESID>(grid(d), d, a, jo, st);
            GemvJob j1{};
            j1.in = a.x; j1.W = W1; j1.K = d; j1.N = hid;
            launch_gemv<PRO_RMS, EPI_GELU>(grid(hid), d, a, j1, st);
            GemvJob j2{};
            j2.in = a.hg; j2.W = W2; j2.K = hid; j2.N = d;
            launch_gemv<PRO_PLAIN, EPI_RESID>(grid(d), hid, a, j2, st);
        }
        if (!feed || s + 1 == n) {
            GemvJob jh{};
            jh.in = a.x; jh.W = Wout; jh.K = d; jh.N = V; jh.logits = logits;
            jh.out_id = feed ? ids : ids + s + 1;
            launch_gemv<PRO_RMS, EPI_HEAD>(grid(V), d, a, jh, st);
        }
    }
    EVK_HIP(hipGetLastError());
    return EVKHIP_OK;
}

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
    // the fused attention gives each key dh/16 lanes of one wave (a power of two)
    // (the fused GEMVs keep their input vector in LDS: K floats next to 33 KB
    // of reduction space, within 64 KB per workgroup)
    if ((c.dh == 16 || c.dh == 32 || c.dh == 64 || c.dh == 128) && c.d <= 7680 && c.hidden <= 7680 &&
        (int64_t)c.max_seq * c.d * 2 < INT32_MAX)
        return run_tokens_fused(c, W.E, W.Wout, W.per_layer, cache_h, feed, ids, n, pos0, (f16*)logits, st);

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
