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

// Batched prefill: rows i of qkv (n, 3d) are positions pos0 + i.  q and k
// are rotated with rope_k's formula (pairs within a head, fp32, one fp16
// rounding), q, k, v are regrouped per head as (heads, n, dh) for the flash
// kernels, and the k, v rows go to the cache at their positions.  One thread
// per pair of columns.
__global__ __launch_bounds__(256) void prefill_split_k(const f16* qkv, int n, int d, int dh, float base, int pos0,
                                                       f16* Qh, f16* Kh, f16* Vh, f16* Kc, f16* Vc) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int pairs = d / 2;
    if (gid >= (int64_t)n * pairs) return;
    const int c = 2 * (int)(gid % pairs), i = (int)(gid / pairs);
    const int h = c / dh, j = c % dh, pp = j / 2;
    const f16* row = qkv + (int64_t)i * 3 * d;
    const float inv_freq = powf(base, -2.0f * (float)pp / (float)dh);
    float sn, cs;
    sincosf((float)(pos0 + i) * inv_freq, &sn, &cs);
    const int64_t o = ((int64_t)h * n + i) * dh + j, oc = (int64_t)(pos0 + i) * d + c;
    float x0 = (float)row[c], x1 = (float)row[c + 1];
    Qh[o] = (f16)(x0 * cs - x1 * sn);
    Qh[o + 1] = (f16)(x0 * sn + x1 * cs);
    x0 = (float)row[d + c];
    x1 = (float)row[d + c + 1];
    const f16 k0 = (f16)(x0 * cs - x1 * sn), k1 = (f16)(x0 * sn + x1 * cs);
    Kh[o] = k0;
    Kh[o + 1] = k1;
    Kc[oc] = k0;
    Kc[oc + 1] = k1;
    const f16 v0 = row[2 * d + c], v1 = row[2 * d + c + 1];
    Vh[o] = v0;
    Vh[o + 1] = v1;
    Vc[oc] = v0;
    Vc[oc + 1] = v1;
}

// (heads, n, dh) -> (n, heads * dh), 16 bytes per thread
__global__ __launch_bounds__(256) void prefill_merge_k(const f16* Oh, f16* A, int n, int d, int dh) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int c8 = d / 8;
    if (gid >= (int64_t)n * c8) return;
    const int c = 8 * (int)(gid % c8), i = (int)(gid / c8);
    const int h = c / dh, j = c % dh;
    *reinterpret_cast<u32x4*>(A + (int64_t)i * d + c) =
        *reinterpret_cast<const u32x4*>(Oh + ((int64_t)h * n + i) * dh + j);
}

struct ModelWs {
    f16* buf = nullptr;
    size_t elems = 0;
};
ModelWs g_ws;   // unfused path (fp16 elements)
ModelWs g_fws;  // fused path (bytes in `elems`)
ModelWs g_pws;  // batched prefill (fp16 elements)
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
// row) over a K range and runs its prologue and epilogue itself:
//   qkv  : x += pending W2 residual, rms_norm(x) . Wqkv -> rope(q), rope(k),
//          cache append (layer 0 takes x from the embedding row instead)
//   attn : single-query attention, each head split over key ranges
//   wo   : merge of the attention splits, att . Wo over K ranges -> partials
//   w1   : x += fp16(sum of the Wo partials), rms_norm(x) . W1 -> gelu
//   w2   : gelu . W2 over K ranges -> partials (added by the next qkv/head)
//   head : x += pending W2 residual, rms_norm(x) . Wout -> logits, greedy
//          argmax (shader tie order)
// Values cross workgroups only at kernel boundaries, except the LM head's
// greedy winner.  Rounding points are those of the unfused op sequence
// (every op output is fp16); partial sums are combined in a fixed order, so
// results do not depend on which workgroup finishes last.
// The LM head's block winners are written and read with agent-scope atomics
// (straight to the device coherence point, no L2 flush or invalidate), and a
// workgroup counts itself in only after those stores have completed; the
// counter is left at zero by the workgroup that consumes it.
// ---------------------------------------------------------------------------
constexpr int GCB = 64;   // GEMV output columns per workgroup (128 bytes of a weight row)

struct DecArgs {
    int d, heads, dh, hidden, vocab, max_seq;
    float eps, rope_base;
    float* apart;      // attention splits [split][head][dh + 4]: o / l, m, l
    float* cand_v;     // LM-head block winners
    uint32_t* cand_r;
    unsigned* cnt;     // counters (zero between launches)
};

enum { PRO_PLAIN = 0, PRO_RMS = 1, PRO_EMBED_RMS = 2, PRO_ATTN = 3, PRO_GELU = 4 };
enum { EPI_PART = 0, EPI_HEAD = 1 };
constexpr int ATT_SMAX = 16;  // attention splits per head, at most
constexpr int RES_SMAX = 8;   // K splits of a residual GEMV, at most

struct GemvJob {
    const f16* in;    // input vector (PRO_PLAIN), or x (rms prologues)
    const float* rpart;  // rms / gelu prologues: the producer's partials [rsplit][K]
    int rsplit;
    f16* xout;        // rms prologues: where workgroup (0, 0) stores the new x
    const f16* W;     // (K, N) row-major
    int K, N;
    const f16* E;     // PRO_EMBED_RMS: embedding table and the step's token
    const uint16_t* tok;
    f16* logits;      // EPI_HEAD
    uint16_t* out_id;
    int nsplit;       // PRO_ATTN: attention splits per head
    float* part;      // EPI_PART: K-split partials [ksplit][N]
};

// GEMV over a K range of a block of NCB output columns (one 128-byte line of
// each weight row when NCB = 64), with a prologue on the input vector and an
// epilogue on the block's outputs in the same workgroup.  Grid: (ceil(N /
// NCB), ksplit); workgroup (cb, ks) takes rows [ks * kc, (ks + 1) * kc),
// kc = ceil(K / ksplit).  NT threads = NCB/8 column groups x row groups; a
// thread issues LD 16-byte weight loads before it waits, so that the range's
// rows are in flight at once (256 threads x 24 loads cover 768 rows).  The
// first batch is issued before the prologue: the weights do not depend on
// the input vector, so both latencies overlap.  The input vector (K floats,
// plus the staged attention splits for PRO_ATTN) lives in dynamic LDS.
template <int NCB, int NT, int LD, int PRO, int EPI>
__global__ __launch_bounds__(NT) void dec_gemv(DecArgs a, GemvJob j) {
    constexpr int CG = NCB / 8, RG = NT / CG;
    extern __shared__ float hv[];  // K input values
    __shared__ float red[RG * NCB];
    __shared__ float y[NCB];
    __shared__ float s_v[NT / 64];
    __shared__ uint32_t s_r[NT / 64];
    const int N = j.N, K = j.K;
    const int cb = blockIdx.x, c0 = cb * NCB, nc = min(NCB, N - c0);
    const int kc = (K + (int)gridDim.y - 1) / (int)gridDim.y;
    const int r_lo = (int)blockIdx.y * kc, r_hi = min(K, r_lo + kc);

    const int cg = threadIdx.x % CG, rg = threadIdx.x / CG;
    const int col = c0 + cg * 8;
    const bool col_ok = col < N;
    // loads are branch-free: offsets outside a descriptor read zeros
    const __amdgpu_buffer_rsrc_t wres = buf_rsrc(j.W, (uint32_t)K * (uint32_t)N * 2u);
    half8 w[LD];
    auto load_batch = [&](int i0) {
#pragma unroll
        for (int u = 0; u < LD; ++u) {
            const int i = i0 + u * RG;
            w[u] = as_half8(buf_load16(wres, oob_or(col_ok && i < r_hi, ((uint32_t)i * (uint32_t)N + col) * 2u), 0));
        }
    };

    // ---- prologue: the input vector as fp16 values ----
    // For the sizes one pass of the workgroup covers (the "one" forms), the
    // prologue's loads are issued first and the first batch of weight loads
    // right after them (the weights do not depend on the input vector):
    // loads complete in issue order, so the prologue then waits for its own
    // data only, while the weights stream in.  The compiler barriers keep
    // that issue order.
    const int H = a.heads, dh = a.dh, W = dh + 4, S = j.nsplit;
    const int h_lo = r_lo / dh, nh = (r_hi - 1) / dh - h_lo + 1;  // PRO_ATTN: heads of the range
    const int per4 = nh * W / 4, tot4 = S * per4;                // PRO_ATTN: staged float4s
    const f16* x = j.in;
    if (PRO == PRO_EMBED_RMS) x = j.E + (int64_t)min((int)j.tok[0], a.vocab - 1) * K;
    const int rs = (PRO == PRO_RMS || PRO == PRO_GELU) ? j.rsplit : 0;
    const __amdgpu_buffer_rsrc_t xres = buf_rsrc(x, (uint32_t)K * 2u);
    const __amdgpu_buffer_rsrc_t pres = buf_rsrc(j.rpart, (uint32_t)(rs * K) * 4u);  // splits >= rs read zeros
    const __amdgpu_buffer_rsrc_t ares = buf_rsrc(a.apart, (uint32_t)(S * H * W) * 4u);
    const bool one = (PRO == PRO_PLAIN || PRO == PRO_GELU) ? (r_hi - r_lo <= 4 * NT)
                     : (PRO == PRO_ATTN) ? (S > 1 && tot4 <= 8 * NT)
                                         : (K <= 4 * NT);
    uint32_t xv[4];  // raw fp16 bits
    float pv[4][RES_SMAX];
    u32x4 sv[8];
    auto ld_h = [&](uint32_t off) { return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(xres, off, 0, 0); };
    auto hval = [](uint32_t bits) { return (float)__builtin_bit_cast(f16, (uint16_t)bits); };
    auto fetch_plain = [&](int i0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[u] = ld_h(oob_or(i0 + u * NT < r_hi, (uint32_t)(i0 + u * NT) * 2u));
    };
    auto fetch_stage = [&](int b0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int idx = b0 + u * NT, q = idx / per4;
            const uint32_t off = (uint32_t)((q * H + h_lo) * (W / 4) + (idx - q * per4)) * 16u;
            sv[u] = buf_load16(ares, oob_or(idx < tot4, off), 0);
        }
    };
    auto fetch_gelu = [&](int i0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * NT;
#pragma unroll
            for (int q = 0; q < RES_SMAX; ++q)
                pv[u][q] = buf_load_f32(pres, oob_or(i < r_hi, (uint32_t)(q * K + i) * 4u));
        }
    };
    auto fetch_x = [&](int i0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * NT;
            xv[u] = ld_h(oob_or(i < K, (uint32_t)i * 2u));
#pragma unroll
            for (int q = 0; q < RES_SMAX; ++q) pv[u][q] = buf_load_f32(pres, oob_or(i < K, (uint32_t)(q * K + i) * 4u));
        }
    };
    if (one) {
        if (PRO == PRO_PLAIN) fetch_plain(r_lo + (int)threadIdx.x);
        else if (PRO == PRO_GELU) fetch_gelu(r_lo + (int)threadIdx.x);
        else if (PRO == PRO_ATTN) fetch_stage(threadIdx.x);
        else fetch_x(threadIdx.x);
    }
    asm volatile("" ::: "memory");
    load_batch(r_lo + rg);
    asm volatile("" ::: "memory");
    if (one) {  // the prologue's values are taken from here on
        if (PRO == PRO_ATTN) {
#pragma unroll
            for (int u = 0; u < 8; ++u) asm volatile("" : "+v"(sv[u]));
        } else {
            if (PRO != PRO_GELU) {
#pragma unroll
                for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(xv[u]));
            }
            if (PRO == PRO_RMS || PRO == PRO_GELU) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int q = 0; q < RES_SMAX; ++q) asm volatile("" : "+v"(pv[u][q]));
            }
        }
    }

    if (PRO == PRO_PLAIN) {
        auto put = [&](int i0) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i0 + u * NT < r_hi) hv[i0 + u * NT] = hval(xv[u]);
        };
        if (one) {
            put(r_lo + (int)threadIdx.x);
        } else {
            for (int i0 = r_lo + (int)threadIdx.x; i0 < r_hi; i0 += 4 * NT) {
                fetch_plain(i0);
                put(i0);
            }
        }
    } else if (PRO == PRO_GELU) {
        // gelu(fp16(sum of the W1 partials)) of the rows [r_lo, r_hi)
        auto put = [&](int i0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * NT;
                if (i >= r_hi) continue;
                float yv = 0.0f;
#pragma unroll
                for (int q = 0; q < RES_SMAX; ++q) yv += pv[u][q];
                hv[i] = (float)(f16)gelu_f((float)(f16)yv);
            }
        };
        if (one) {
            put(r_lo + (int)threadIdx.x);
        } else {
            for (int i0 = r_lo + (int)threadIdx.x; i0 < r_hi; i0 += 4 * NT) {
                fetch_gelu(i0);
                put(i0);
            }
        }
    } else if (PRO == PRO_ATTN) {
        // attention output of the heads in [r_lo, r_hi): each head's splits
        // (o_s / l_s, m_s, l_s) merged as sum_s w_s o_s / l_s / sum_s w_s with
        // w_s = l_s exp(m_s - max m); the splits of those heads are staged in
        // LDS after hv as [split][head][W]
        if (S == 1) {
            for (int i = r_lo + (int)threadIdx.x; i < r_hi; i += NT)
                hv[i] = (float)(f16)a.apart[(i / dh) * W + i % dh];
        } else {
            float* stg = hv + K;
            u32x4* dst = reinterpret_cast<u32x4*>(stg);
            auto put = [&](int b0) {
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (b0 + u * NT < tot4) dst[b0 + u * NT] = sv[u];
            };
            if (one) {
                put(threadIdx.x);
            } else {
                for (int b0 = threadIdx.x; b0 < tot4; b0 += 8 * NT) {
                    fetch_stage(b0);
                    put(b0);
                }
            }
            __syncthreads();
            auto merge = [&](int i) {
                const int hh = i / dh - h_lo, c = i % dh;
                float mq[ATT_SMAX], lq[ATT_SMAX], oq[ATT_SMAX];
#pragma unroll
                for (int q = 0; q < ATT_SMAX; ++q) {
                    const float* e = stg + (q * nh + hh) * W;
                    lq[q] = (q < S) ? e[dh + 1] : 0.0f;
                    mq[q] = (q < S) ? e[dh] : -INFINITY;
                    oq[q] = (q < S) ? e[c] : 0.0f;
                }
                float M = -INFINITY;
#pragma unroll
                for (int q = 0; q < ATT_SMAX; ++q)
                    if (lq[q] > 0.0f) M = fmaxf(M, mq[q]);
                float num = 0.0f, den = 0.0f;
#pragma unroll
                for (int q = 0; q < ATT_SMAX; ++q) {
                    const float wq = (lq[q] > 0.0f) ? lq[q] * expf(mq[q] - M) : 0.0f;
                    num += wq * oq[q];
                    den += wq;
                }
                hv[i] = (float)(f16)(den > 0.0f ? num / den : 0.0f);
            };
            if (r_hi - r_lo <= NT) {
                if (r_lo + (int)threadIdx.x < r_hi) merge(r_lo + threadIdx.x);
            } else {
                for (int i = r_lo + (int)threadIdx.x; i < r_hi; i += NT) merge(i);
            }
        }
    } else {
        // x (or the embedding row of the step's token), plus the pending
        // residual y = fp16(sum of the producer's K-split partials):
        // x <- fp16(x + y).  Workgroup (0, 0) stores the new x to j.xout.
        // Then rms_norm: fp16(clamp(x) / sqrt(mean(clamp(x)^2) + eps)).
        const bool wr = j.xout != nullptr && blockIdx.x == 0 && blockIdx.y == 0;
        float ss = 0.0f;
        auto put = [&](int i0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * NT;
                if (i >= K) continue;
                float v = hval(xv[u]);
                if (rs > 0) {
                    float yv = 0.0f;
#pragma unroll
                    for (int q = 0; q < RES_SMAX; ++q) yv += pv[u][q];
                    v = (float)(f16)(v + (float)(f16)yv);
                }
                if (wr) j.xout[i] = (f16)v;
                v = fminf(fmaxf(v, -65504.0f), 65504.0f);
                hv[i] = v;
                ss += v * v;
            }
        };
        if (one) {
            put(threadIdx.x);
        } else {
            for (int i0 = threadIdx.x; i0 < K; i0 += 4 * NT) {
                fetch_x(i0);
                put(i0);
            }
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NT / 64; ++w2) ss += red[w2];
        const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
        if (one) {  // own elements
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = threadIdx.x + u * NT;
                if (i < K) hv[i] = (float)(f16)(hv[i] * inv);
            }
        } else {
            for (int i = threadIdx.x; i < K; i += NT) hv[i] = (float)(f16)(hv[i] * inv);
        }
    }
    __syncthreads();

    // ---- the block's dot products over rows [r_lo, r_hi) ----
    {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int i0 = r_lo + rg; i0 < r_hi; i0 += RG * LD) {
            if (i0 != r_lo + rg) load_batch(i0);
#pragma unroll
            for (int u = 0; u < LD; ++u) {
                const int i = i0 + u * RG;
                const float h = (i < r_hi) ? hv[i] : 0.0f;
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
            y[c] = (EPI == EPI_PART) ? s : (float)(f16)s;  // fp16 output of the product, or a raw partial
        }
        __syncthreads();
    }

    // ---- epilogue ----
    if (EPI == EPI_PART) {
        float* out = j.part + (int64_t)blockIdx.y * N + c0;
        for (int c = threadIdx.x; c < nc; c += NT) out[c] = y[c];
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

// Single-query attention of one layer, with the QKV GEMV's K-split
// partials merged in its prologue: workgroup (h, s) forms q of head h
// (fp16(sum of partials), rope, fp16) and covers the cached keys
// [s * ppw * kpp, +ppw * kpp) below pos, kpp = ATT_KPT * 256 / (dh / 16)
// keys per pass.  The last split also forms k, v of position pos (rope on
// k), appends them to the caches and folds that key in after its range.
// Every K and V row of a pass is requested before any arithmetic (a thread
// scores ATT_KPT keys with dh / 16 lanes per key and sums 2 * ATT_KPT value
// rows of 8 dims), so a pass costs one round trip; the first pass is
// requested together with the partials.  The split's result (o / l, m, l)
// goes to a.apart; the Wo GEMV merges the splits in its prologue.  Loads go
// through buffer descriptors over the cached rows [0, pos) with the whole
// offset in the range-checked vector operand: rows past them read as
// zeros, and keys past the split's range are masked.
constexpr int ATT_NT = 256;
constexpr int ATT_KPT = 2;
constexpr int ATT_VR = 2 * ATT_KPT;

__global__ __launch_bounds__(ATT_NT) void dec_attn(DecArgs a, f16* Kc, f16* Vc, const float* qkv_part, int qsplit,
                                                   int pos, int ppw) {
    __shared__ float sc[ATT_KPT * ATT_NT];
    __shared__ float red[ATT_NT * 8];
    __shared__ float stat[2 * (ATT_NT / 64)];
    __shared__ float pre[3 * 128];            // fp16-rounded sums of q, k, v of the head
    __shared__ __attribute__((aligned(16))) f16 qh[128];
    __shared__ float kvn[2 * 128];            // k (rope'd), v of position pos
    const int d = a.d, dh = a.dh, h = blockIdx.x, sp = blockIdx.y;
    const bool last = sp + 1 == (int)gridDim.y;
    const int L = pos;  // cached keys
    const float scale = 1.0f / sqrtf((float)dh);
    const int tpk = dh / 16, kstep = ATT_NT / tpk, kpp = ATT_KPT * kstep;
    const int ndg = dh / 8, G = ATT_NT / ndg;
    const int kl = threadIdx.x / tpk, part = threadIdx.x % tpk;
    const int dg = threadIdx.x % ndg, kg = threadIdx.x / ndg;
    const int k_lo = sp * ppw * kpp, k_hi = min(L, k_lo + ppw * kpp);
    const uint32_t row = (uint32_t)d * 2;  // bytes per cache row
    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(Kc, (uint32_t)L * row);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(Vc, (uint32_t)L * row);
    const uint32_t kvo = (uint32_t)kl * row + (uint32_t)(h * dh + part * 16) * 2;
    const uint32_t vvo = (uint32_t)kg * row + (uint32_t)(h * dh + dg * 8) * 2;

    // partials of q (and k, v for the last split): entry t < dh (or < 3 dh),
    // t = threadIdx.x + u * ATT_NT, sums column (t / dh) * d + h * dh + t % dh
    // over the splits
    const int nsum = last ? 3 * dh : dh;
    const __amdgpu_buffer_rsrc_t pres = buf_rsrc(qkv_part, (uint32_t)(qsplit * 3 * d) * 4u);  // splits >= qsplit: zeros
    float pv[2][RES_SMAX];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = threadIdx.x + u * ATT_NT;
        const int pc = (t / dh) * d + h * dh + t % dh;
#pragma unroll
        for (int q = 0; q < RES_SMAX; ++q) pv[u][q] = buf_load_f32(pres, oob_or(t < nsum, (uint32_t)(q * 3 * d + pc) * 4u));
    }
    asm volatile("" ::: "memory");

    half8 kv[ATT_KPT][2], v[ATT_VR];
    auto load_pass = [&](int p0) {
#pragma unroll
        for (int t = 0; t < ATT_KPT; ++t) {
            const uint32_t vo = kvo + (uint32_t)(p0 + t * kstep) * row;
            kv[t][0] = as_half8(buf_load16(kres, vo, 0));
            kv[t][1] = as_half8(buf_load16(kres, vo + 16, 0));
        }
#pragma unroll
        for (int u = 0; u < ATT_VR; ++u) v[u] = as_half8(buf_load16(vres, vvo + (uint32_t)(p0 + u * G) * row, 0));
    };
    if (k_lo < k_hi) load_pass(k_lo);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int q = 0; q < RES_SMAX; ++q) asm volatile("" : "+v"(pv[u][q]));

    // q, k, v of the head: fp16 sums, then rope on q and k (pairs 2i, 2i+1)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = threadIdx.x + u * ATT_NT;
        float y = 0.0f;
#pragma unroll
        for (int q = 0; q < RES_SMAX; ++q) y += pv[u][q];
        if (t < nsum) pre[t] = (float)(f16)y;
    }
    __syncthreads();
    for (int t = threadIdx.x; t < nsum; t += ATT_NT) {
        const int which = t / dh, c = t % dh;
        if (which == 2) {
            const float vn = pre[t];
            kvn[dh + c] = vn;
            Vc[(int64_t)pos * d + h * dh + c] = (f16)vn;
        } else {
            const float x0 = pre[which * dh + (c & ~1)], x1 = pre[which * dh + (c | 1)];
            const float inv_freq = powf(a.rope_base, -2.0f * (float)(c / 2) / (float)dh);
            float sn, cs;
            sincosf((float)pos * inv_freq, &sn, &cs);
            const f16 r = (f16)((c & 1) ? (x0 * sn + x1 * cs) : (x0 * cs - x1 * sn));
            if (which == 0) {
                qh[c] = r;
            } else {
                kvn[c] = (float)r;
                Kc[(int64_t)pos * d + h * dh + c] = r;
            }
        }
    }
    __syncthreads();
    const half8 q0 = *reinterpret_cast<const half8*>(qh + part * 16);
    const half8 q1 = *reinterpret_cast<const half8*>(qh + part * 16 + 8);

    float m_run = -INFINITY, l_run = 0.0f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p0 = k_lo; p0 < k_hi; p0 += kpp) {
        const int np = min(kpp, k_hi - p0);
        if (p0 != k_lo) load_pass(p0);
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
            const float pk = sc[kg + u * G];  // zero past np
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += pk * (float)v[u][e];
        }
        __syncthreads();  // sc and stat are rewritten by the next pass
    }
    // sum over the G key groups of each dim group
#pragma unroll
    for (int e = 0; e < 8; ++e) red[threadIdx.x * 8 + e] = o[e];
    // the last split's new key: score q . k, summed by wave 0
    if (last && threadIdx.x < 64) {
        float sn = 0.0f;
        for (int c = threadIdx.x; c < dh; c += 64) sn += (float)qh[c] * kvn[c];
        sn = wave_sum(sn);
        if (threadIdx.x == 0) stat[0] = sn * scale;
    }
    __syncthreads();
    const float s_new = stat[0];
    if (threadIdx.x < dh) {
        const int dg2 = threadIdx.x / 8, e2 = threadIdx.x % 8;
        float tot = 0.0f;
        for (int g = 0; g < G; ++g) tot += red[(g * ndg + dg2) * 8 + e2];
        if (last) {
            const float m_new = fmaxf(m_run, s_new);
            const float alpha = (m_run == -INFINITY) ? 0.0f : expf(m_run - m_new);
            const float pn = expf(s_new - m_new);
            tot = tot * alpha + pn * kvn[dh + threadIdx.x];
            l_run = l_run * alpha + pn;
            m_run = m_new;
        }
        float* out = a.apart + ((int64_t)sp * a.heads + h) * (dh + 4);
        out[threadIdx.x] = l_run > 0.0f ? tot / l_run : 0.0f;
        if (threadIdx.x == 0) {
            out[dh] = m_run;
            out[dh + 1] = l_run;
        }
    }
}

}  // namespace

void model_free_workspace() {
    if (g_ws.buf) (void)hipFree(g_ws.buf);
    g_ws = ModelWs{};
    if (g_fws.buf) (void)hipFree(g_fws.buf);
    g_fws = ModelWs{};
    if (g_pws.buf) (void)hipFree(g_pws.buf);
    g_pws = ModelWs{};
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

// Rows in flight per workgroup: 256 threads hold 6, 12 or 24 loads of 32 row
// groups (192, 384 or 768 rows per K range in one batch); longer ranges take
// 1024 threads x 12 loads per batch.
int gemv_rows_cap(int R) { return R <= 192 ? 192 : R <= 384 ? 384 : R <= 768 ? 768 : 0; }
int gemv_static_lds(int R) { return gemv_rows_cap(R) ? 8448 : 33024; }

template <int PRO, int EPI>
void launch_gemv(int N, int K, int ksplit, size_t extra_lds, const DecArgs& a, const GemvJob& j, hipStream_t st) {
    const dim3 grid((unsigned)((N + GCB - 1) / GCB), (unsigned)ksplit);
    const size_t lds = (size_t)K * sizeof(float) + extra_lds;
    const int cap = gemv_rows_cap((K + ksplit - 1) / ksplit);
    if (cap == 192)
        hipLaunchKernelGGL((dec_gemv<GCB, 256, 6, PRO, EPI>), grid, dim3(256), lds, st, a, j);
    else if (cap == 384)
        hipLaunchKernelGGL((dec_gemv<GCB, 256, 12, PRO, EPI>), grid, dim3(256), lds, st, a, j);
    else if (cap == 768)
        hipLaunchKernelGGL((dec_gemv<GCB, 256, 24, PRO, EPI>), grid, dim3(256), lds, st, a, j);
    else
        hipLaunchKernelGGL((dec_gemv<GCB, 1024, 12, PRO, EPI>), grid, dim3(1024), lds, st, a, j);
}

// K splits of the two residual GEMVs (Wo, W2): ranges of about 192 rows.
int residual_ksplit(int K) { return std::min(RES_SMAX, (K + 191) / 192); }

// Fused path: five kernels per layer and one LM-head kernel per token.  The
// residual stream ping-pongs between two buffers: a kernel whose prologue
// adds the pending residual reads x from one and workgroup (0, 0) stores the
// sum to the other, which the following kernels read.
int run_tokens_fused(const evkhip_model_cfg& c, const f16* E, const f16* Wout, uint64_t per_layer, f16* cache_h,
                     const uint16_t* feed, uint16_t* ids, uint32_t n, uint32_t pos0, f16* logits, hipStream_t st) {
    const int d = (int)c.d, hid = (int)c.hidden, V = (int)c.vocab, H = (int)c.heads, dh = (int)c.dh;
    auto cdiv = [](int x, int y) { return (x + y - 1) / y; };
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int ks_o = residual_ksplit(d), ks_2 = residual_ksplit(hid);
    // attention splits: as many as the Wo GEMV can stage in LDS next to its
    // input vector, for the heads one K range of it covers
    const int att_w = dh + 4;
    const int ro = cdiv(d, ks_o);
    const int nh_max = std::min(H, cdiv(ro, dh) + 1);
    const int smax =
        std::max(1, std::min(ATT_SMAX, (65536 - gemv_static_lds(ro) - d * 4) / (nh_max * att_w * 4)));
    const int kpp = ATT_KPT * ATT_NT / (dh / 16);
    const size_t cnt_n = 1;  // the LM head's arrival counter
    const int ks_q = residual_ksplit(d), ks_1 = residual_ksplit(d);
    const size_t part_n = (size_t)RES_SMAX * std::max(3 * d, hid);
    const size_t off_xb = al((size_t)d * 2);
    const size_t off_pa = off_xb + al((size_t)d * 2), off_pb = off_pa + al(part_n * 4);
    const size_t off_apart = off_pb + al(part_n * 4);
    const size_t off_cv = off_apart + al((size_t)smax * H * att_w * 4);
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
    a.apart = reinterpret_cast<float*>(base + off_apart);
    a.cand_v = reinterpret_cast<float*>(base + off_cv);
    a.cand_r = reinterpret_cast<uint32_t*>(base + off_cr);
    a.cnt = g_fcnt;
    // partials: QKV and W1 write A, Wo and W2 write B; every kernel reads
    // the other buffer than the one it writes
    float* pa = reinterpret_cast<float*>(base + off_pa);
    float* pb = reinterpret_cast<float*>(base + off_pb);
    f16* xbuf[2] = {reinterpret_cast<f16*>(base), reinterpret_cast<f16*>(base + off_xb)};
    int xc = 0;  // buffer holding x, up to the pending residual
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
            j.W = Wqkv; j.K = d; j.N = 3 * d; j.E = E; j.tok = tok; j.part = pa;
            j.xout = xbuf[xc ^ 1];
            if (l == 0) {
                launch_gemv<PRO_EMBED_RMS, EPI_PART>(3 * d, d, ks_q, 0, a, j, st);
            } else {
                j.in = xbuf[xc]; j.rpart = pb; j.rsplit = ks_2;
                launch_gemv<PRO_RMS, EPI_PART>(3 * d, d, ks_q, 0, a, j, st);
            }
            xc ^= 1;
            const int npass = std::max(1, cdiv(pos, kpp));
            const int ppw = cdiv(npass, std::min(npass, smax));
            const int nsplit = cdiv(npass, ppw);  // the last split also takes key pos
            hipLaunchKernelGGL(dec_attn, dim3((unsigned)H, (unsigned)nsplit), dim3(ATT_NT), 0, st, a, Kc, Vc,
                               (const float*)pa, ks_q, pos, ppw);
            GemvJob jo{};
            jo.W = Wo; jo.K = d; jo.N = d; jo.nsplit = nsplit; jo.part = pb;
            const size_t stage = nsplit > 1 ? (size_t)nsplit * nh_max * att_w * 4 : 0;
            launch_gemv<PRO_ATTN, EPI_PART>(d, d, ks_o, stage, a, jo, st);
            GemvJob j1{};
            j1.in = xbuf[xc]; j1.rpart = pb; j1.rsplit = ks_o; j1.xout = xbuf[xc ^ 1];
            j1.W = W1; j1.K = d; j1.N = hid; j1.part = pa;
            launch_gemv<PRO_RMS, EPI_PART>(hid, d, ks_1, 0, a, j1, st);
            xc ^= 1;
            GemvJob j2{};
            j2.rpart = pa; j2.rsplit = ks_1; j2.W = W2; j2.K = hid; j2.N = d; j2.part = pb;
            launch_gemv<PRO_GELU, EPI_PART>(d, hid, ks_2, 0, a, j2, st);
        }
        // x of the next step's layer 0 comes from the embedding; the last
        // layer's W2 partials are still pending here
        if (!feed || s + 1 == n) {
            GemvJob jh{};
            jh.in = xbuf[xc]; jh.rpart = pb; jh.rsplit = ks_2;
            jh.W = Wout; jh.K = d; jh.N = V; jh.logits = logits;
            jh.out_id = feed ? ids : ids + s + 1;
            launch_gemv<PRO_RMS, EPI_HEAD>(V, d, 1, 0, a, jh, st);
        }
    }
    EVK_HIP(hipGetLastError());
    return EVKHIP_OK;
}

// Validates cfg/buffers and runs n tokens.  feed != null: token s is feed[s],
// only the last step runs the LM head (into ids[0]); otherwise token s is
// ids[s] and every step writes ids[s+1].
// Prefill of a prompt at positions 0..n-1 as whole-sequence ops (the
// reference evaluates the sequence this way, evk_ai.h:670-712): per layer
// rms_norm over the n rows, X.Wqkv on the MFMA GEMM, rope and the cache rows,
// causal flash attention per head (heads as the batch), X.Wo, residual,
// rms_norm, gelu(X.W1).W2, residual; then the last row's logits and greedy id.
// Same op sequence and fp16 rounding points as the token loop; the GEMMs sum
// in another order.  Returns 1 when the shape is not taken (the token loop
// serves it), an evkhip error code otherwise.
int run_prefill_batched(const evkhip_model_cfg& c, const f16* E, const f16* Wout, uint64_t per_layer, f16* cache_h,
                        const uint16_t* feed, uint16_t* ids, uint32_t n, f16* logits, hipStream_t st) {
    const int d = (int)c.d, hid = (int)c.hidden, H = (int)c.heads, dh = (int)c.dh;
    if (n < 16 || !flash_mfma_head(c.dh) || dh % 8 || (int64_t)n * 3 * d * 2 >= INT32_MAX ||
        (int64_t)n * hid * 2 >= INT32_MAX)
        return 1;
    const size_t nd = (size_t)n * d, nh = (size_t)n * hid;
    // X, Hn, QKV (3), Qh, Kh, Vh, Oh, A, T: 11 n d; HH, HG: 2 n hidden
    const size_t need = 11 * nd + 2 * nh;
    if (need * sizeof(f16) > ((size_t)1 << 31)) return 1;
    if (need > g_pws.elems) {
        if (g_pws.buf) EVK_HIP(hipFree(g_pws.buf));
        g_pws.buf = nullptr;
        g_pws.elems = 0;
        EVK_HIP(hipMalloc(&g_pws.buf, need * sizeof(f16)));
        g_pws.elems = need;
    }
    f16* X = g_pws.buf;
    f16* Hn = X + nd;
    f16* QKV = Hn + nd;  // 3 nd
    f16* Qh = QKV + 3 * nd;
    f16* Kh = Qh + nd;
    f16* Vh = Kh + nd;
    f16* Oh = Vh + nd;
    f16* A = Oh + nd;
    f16* T = A + nd;
    f16* HH = T + nd;
    f16* HG = HH + nh;
    auto gemm = [&](const f16* a, const f16* b, f16* out, int M, int N, int K) {
        GemmArgs g{};
        g.A = a;
        g.B = b;
        g.C = out;
        g.M = M;
        g.N = N;
        g.K = K;
        return gemm_dispatch(g, 1, false, false, true, st);
    };
    const unsigned g_split = (unsigned)(((int64_t)n * (d / 2) + 255) / 256);
    const unsigned g_merge = (unsigned)(((int64_t)n * (d / 8) + 255) / 256);
    CHECK(embed_launch(E, feed, X, n, d, (int)c.vocab, st));
    for (uint32_t l = 0; l < c.layers; ++l) {
        const f16* Wqkv = E + (uint64_t)c.vocab * d + l * per_layer;
        const f16* Wo = Wqkv + (uint64_t)d * 3 * d;
        const f16* W1 = Wo + (uint64_t)d * d;
        const f16* W2 = W1 + (uint64_t)d * hid;
        f16* Kc = cache_h + (uint64_t)l * 2 * c.max_seq * d;
        f16* Vc = Kc + (uint64_t)c.max_seq * d;
        CHECK(rms_norm_launch(X, Hn, n, d, c.eps, st));
        CHECK(gemm(Hn, Wqkv, QKV, (int)n, 3 * d, d));
        hipLaunchKernelGGL(prefill_split_k, dim3(g_split), dim3(256), 0, st, QKV, (int)n, d, dh, c.rope_base, 0, Qh,
                           Kh, Vh, Kc, Vc);
        FlashArgs fa{};
        fa.q = Qh;
        fa.k = Kh;
        fa.v = Vh;
        fa.out = Oh;
        fa.B = H;
        fa.H = 1;
        fa.N = (int)n;
        CHECK(flash_forward(fa, dh, true, true, st));
        hipLaunchKernelGGL(prefill_merge_k, dim3(g_merge), dim3(256), 0, st, Oh, A, (int)n, d, dh);
        CHECK(gemm(A, Wo, T, (int)n, d, d));
        CHECK(add_launch(X, T, X, (int64_t)nd, st));
        CHECK(rms_norm_launch(X, Hn, n, d, c.eps, st));
        CHECK(gemm(Hn, W1, HH, (int)n, hid, d));
        CHECK(gelu_launch(HH, HG, (int64_t)nh, st));
        CHECK(gemm(HG, W2, T, (int)n, d, hid));
        CHECK(add_launch(X, T, X, (int64_t)nd, st));
    }
    // the last position's logits and greedy id (rms_norm of its row into Hn's first row)
    CHECK(rms_norm_launch(X + (size_t)(n - 1) * d, Hn, 1, d, c.eps, st));
    CHECK(gemm(Hn, Wout, logits, 1, (int)c.vocab, d));
    CHECK(greedy_launch(logits, ids, 1, 1, (int)c.vocab, 0, 0, (int)c.vocab, st));
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
    if (feed && pos0 == 0) {  // a prompt from position 0: whole-sequence ops
        const int r = run_prefill_batched(c, W.E, W.Wout, W.per_layer, cache_h, feed, ids, n, (f16*)logits, st);
        if (r != 1) return r;
    }
    // the fused attention gives each key dh/16 lanes of one wave (a power of two)
    // (the fused GEMVs keep their input vector in LDS: K floats next to 33 KB
    // of reduction space, within 64 KB per workgroup)
    if ((c.dh == 16 || c.dh == 32 || c.dh == 64 || c.dh == 128) && c.d <= 7680 && c.hidden <= 7680 &&
        (int64_t)c.max_seq * c.d * 2 < INT32_MAX && (int64_t)c.vocab * c.d * 2 < INT32_MAX &&
        (int64_t)c.hidden * c.d * 2 < INT32_MAX)
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
