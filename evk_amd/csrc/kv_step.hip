// Fused KV-cached decode step of the reference caller's model: the blocks
// example/main_llm.cpp:528-546 builds (rms_norm, x.Wq / x.Wk / x.Wv, rope on
// q and k, causal attention, x + attn.Wo, rms_norm, gelu(x.W1).W2 residual),
// then rms_norm and x.Wout, for one new position of B sequences.  The
// reference samples by recomputing the whole sequence per position
// (main_llm.cpp:622-654); evk::ai::KVCacheDecoder keeps the keys and values
// and runs one position per step, op by op (16 launches a layer).  Here one
// workgroup per sequence runs every layer of the step and the logits in a
// single launch: at this size (d = 256, 1 MB of weights a layer) a step is
// bound by launch and memory latency, not by bytes, and a sequence's step
// needs no exchange with the other sequences.
//
// Rounding follows the op-by-op path (every op output is fp16, sums in
// fp32), so the step computes what KVCacheDecoder's per-op step computes up
// to summation order:
//   x = E[id]; per layer: h = rms_norm(x); q, k, v = fp16(h W); q, k = rope
//   at pos; cache rows pos <- k, v; o = fp16(softmax(q K^T / sqrt(d)) V)
//   over rows [0, pos]; x = fp16(x + fp16(o Wo)); h = rms_norm(x);
//   g = fp16(gelu(fp16(h W1))); x = fp16(x + fp16(g W2));
//   logits = fp16(rms_norm(x) Wout).
//
// Matrix-vector products (W stored (in, out) row-major, as the Graph keeps
// them): a thread owns 8 consecutive output columns (16-byte loads along a
// row) and a range of consecutive input rows; all of its rows' loads are
// requested before any is used.  The row ranges meet in LDS and are added
// in range order (deterministic).  Attention: 16 key slots x 32 groups of 8
// dimensions; a key's score is a shuffle sum over its 32 lanes, the value
// sums meet in LDS in slot order.
#include "kernels.h"

#include <math.h>

namespace evkhip {
namespace {

constexpr int KT = 512;         // threads per workgroup
constexpr int KWV = KT / 64;    // waves
constexpr int RED = 4096;       // floats of the reduction scratch
constexpr int MAX_ROWS = 32;    // input rows a thread loads at once in a product
constexpr int KB = 8;           // keys a lane loads at once in the attention

struct KvArgs {
    evkhip_kv_model m;
    const uint16_t* ids;
    int pos;
    f16* logits;
};

DEV float rnd16(float v) { return (float)(f16)v; }

// block-wide sum and max (every thread gets the result; fixed order)
DEV float block_sum(float v, float* sm) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < KWV; ++w) s += sm[w];
    return s;
}
DEV float block_max(float v, float* sm) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = -INFINITY;
#pragma unroll
    for (int w = 0; w < KWV; ++w) s = fmaxf(s, sm[w]);
    return s;
}

// y[n] = sum_k in[k] W[k][n] (fp32) for n < N, handed to store(n, y) once
// per column.  in: K floats in LDS.  K, N multiples of 8.
template <class Store>
DEV void product(const float* in, const f16* W, int K, int N, float* red, Store store) {
    const int tid = threadIdx.x;
    for (int n0 = 0; n0 < N; n0 += RED) {
        const int Nc = min(RED, N - n0), CG = Nc / 8;
        const int KG = max(1, min(KT / CG, (K + 7) / 8));  // row ranges
        const int RPG = (K + KG - 1) / KG;                   // rows per range
        const int cg = tid % CG, kg = tid / CG;
        float acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
        if (kg < KG) {
            const f16* wp = W + n0 + cg * 8;
            const int r_lo = kg * RPG, r_hi = min(K, r_lo + RPG);
            for (int r0 = r_lo; r0 < r_hi; r0 += MAX_ROWS) {
                u32x4 w[MAX_ROWS];
#pragma unroll
                for (int i = 0; i < MAX_ROWS; ++i)
                    if (r0 + i < r_hi) w[i] = *reinterpret_cast<const u32x4*>(wp + (int64_t)(r0 + i) * N);
#pragma unroll
                for (int i = 0; i < MAX_ROWS; ++i)
                    if (r0 + i < r_hi) {
                        const float a = in[r0 + i];
                        const half8 h = as_half8(w[i]);
#pragma unroll
                        for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(a, (float)h[c], acc[c]);
                    }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) red[kg * Nc + cg * 8 + c] = acc[c];
        }
        __syncthreads();
        for (int n = tid; n < Nc; n += KT) {
            float s = 0.0f;
            for (int g = 0; g < KG; ++g) s += red[g * Nc + n];
            store(n0 + n, s);
        }
        __syncthreads();
    }
}

// h = fp16(clamp(x) / sqrt(mean(clamp(x)^2) + eps)), as rms_norm_k
DEV void rms_norm_lds(const float* x, float* h, int d, float eps, float* sm) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < d; i += KT) {
        const float v = fminf(fmaxf(x[i], -65504.0f), 65504.0f);
        ss += v * v;
    }
    ss = block_sum(ss, sm);
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (int i = threadIdx.x; i < d; i += KT) {
        const float v = fminf(fmaxf(x[i], -65504.0f), 65504.0f);
        h[i] = rnd16(v * inv);
    }
    __syncthreads();
}

__global__ __launch_bounds__(KT, 1) void kv_step(KvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float kv_smem[];
    const evkhip_kv_model& m = a.m;
    const int d = (int)m.d, hid = (int)m.hidden, V = (int)m.vocab, S = (int)m.max_seq;
    const int b = blockIdx.x, pos = a.pos, tid = threadIdx.x;
    const int wide = d > hid ? d : hid;
    float* x = kv_smem;            // d: the residual stream
    float* h = x + d;              // wide: a product's input
    float* q = h + wide;           // d
    float* kk = q + d;             // d
    float* vv = kk + d;            // d
    float* o = vv + d;             // d
    float* sc = o + d;             // S: scores
    float* red = sc + S;           // max(RED, 16 d): products, the attention's slot sums
    float* sm = red + (16 * d > RED ? 16 * d : RED);  // KWV

    {
        const int tok = min((int)a.ids[b], V - 1);
        const f16* e = static_cast<const f16*>(m.emb) + (int64_t)tok * d;
        for (int i = tid; i < d; i += KT) x[i] = (float)e[i];
    }
    __syncthreads();
    const int L = pos + 1;
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)d);
    const int lane = tid & 63, slot = tid >> 5, dg = tid & 31;  // attention: 16 key slots x 32 groups

    for (int l = 0; l < (int)m.layers; ++l) {
        const f16* Wq = static_cast<const f16*>(m.w[l][0]);
        const f16* Wk = static_cast<const f16*>(m.w[l][1]);
        const f16* Wv = static_cast<const f16*>(m.w[l][2]);
        const f16* Wo = static_cast<const f16*>(m.w[l][3]);
        const f16* W1 = static_cast<const f16*>(m.w[l][4]);
        const f16* W2 = static_cast<const f16*>(m.w[l][5]);
        f16* Kc = static_cast<f16*>(m.k_cache[l]) + (int64_t)b * S * d;
        f16* Vc = static_cast<f16*>(m.v_cache[l]) + (int64_t)b * S * d;

        rms_norm_lds(x, h, d, m.eps, sm);
        product(h, Wq, d, d, red, [&](int n, float s) { q[n] = rnd16(s); });
        product(h, Wk, d, d, red, [&](int n, float s) { kk[n] = rnd16(s); });
        product(h, Wv, d, d, red, [&](int n, float s) { vv[n] = rnd16(s); });
        // rope on q and k (interleaved pairs, head size d) as rope_k; the
        // cache rows of this position
        for (int pr = tid; pr < d / 2; pr += KT) {
            const float inv_freq = powf(m.rope_base, -2.0f * (float)pr / (float)d);
            const float ang = (float)pos * inv_freq;
            float s, c;
            sincosf(ang, &s, &c);
            const float q0 = q[2 * pr], q1 = q[2 * pr + 1], k0 = kk[2 * pr], k1 = kk[2 * pr + 1];
            q[2 * pr] = rnd16(q0 * c - q1 * s);
            q[2 * pr + 1] = rnd16(q0 * s + q1 * c);
            const f16 kr0 = (f16)(k0 * c - k1 * s), kr1 = (f16)(k0 * s + k1 * c);
            Kc[(int64_t)pos * d + 2 * pr] = kr0;
            Kc[(int64_t)pos * d + 2 * pr + 1] = kr1;
            Vc[(int64_t)pos * d + 2 * pr] = (f16)vv[2 * pr];
            Vc[(int64_t)pos * d + 2 * pr + 1] = (f16)vv[2 * pr + 1];
            kk[2 * pr] = (float)kr0;
            kk[2 * pr + 1] = (float)kr1;
        }
        __syncthreads();
        // scores of keys [0, pos): this workgroup's cache rows (the row at
        // pos is this step's k, taken from LDS).  Lane group `slot` takes
        // keys slot, slot + 16, ...; its 32 lanes split the dimensions.
        // Eight keys' loads go out before any is used.
        for (int j0 = 0; j0 < L; j0 += 16 * KB) {
            float part[KB];
#pragma unroll
            for (int t = 0; t < KB; ++t) part[t] = 0.0f;
            for (int e0 = dg * 8; e0 < d; e0 += 256) {
                half8 kv8[KB];
#pragma unroll
                for (int t = 0; t < KB; ++t) {
                    const int j = j0 + slot + 16 * t;
                    if (j < pos) kv8[t] = *reinterpret_cast<const half8*>(Kc + (int64_t)j * d + e0);
                }
                float qv[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) qv[c] = q[e0 + c];
#pragma unroll
                for (int t = 0; t < KB; ++t) {
                    const int j = j0 + slot + 16 * t;
                    if (j == pos) {
#pragma unroll
                        for (int c = 0; c < 8; ++c) kv8[t][c] = (f16)kk[e0 + c];
                    }
                    if (j <= pos) {
#pragma unroll
                        for (int c = 0; c < 8; ++c) part[t] = __builtin_fmaf(qv[c], (float)kv8[t][c], part[t]);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < KB; ++t) {
                float v = part[t];
#pragma unroll
                for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
                const int j = j0 + slot + 16 * t;
                if (j < L && dg == 0) sc[j] = v * scale_log2;
            }
        }
        __syncthreads();
        float mx = -INFINITY;
        for (int j = tid; j < L; j += KT) mx = fmaxf(mx, sc[j]);
        mx = block_max(mx, sm);
        float sum = 0.0f;
        for (int j = tid; j < L; j += KT) {
            const float p = exp2f(sc[j] - mx);
            sc[j] = p;
            sum += p;
        }
        sum = block_sum(sum, sm);  // its barriers publish sc
        const float inv = 1.0f / sum;
        // o = P V / sum: slot s sums keys s, s+16, ... for its 8 dimensions
        for (int e0 = dg * 8; e0 < d; e0 += 256) {
            float acc[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
            for (int j0 = slot; j0 < L; j0 += 16 * KB) {
                half8 v8[KB];
#pragma unroll
                for (int t = 0; t < KB; ++t) {
                    const int j = j0 + 16 * t;
                    if (j < pos) v8[t] = *reinterpret_cast<const half8*>(Vc + (int64_t)j * d + e0);
                }
#pragma unroll
                for (int t = 0; t < KB; ++t) {
                    const int j = j0 + 16 * t;
                    if (j == pos) {
#pragma unroll
                        for (int c = 0; c < 8; ++c) v8[t][c] = (f16)vv[e0 + c];
                    }
                    if (j <= pos) {
                        const float pj = sc[j];
#pragma unroll
                        for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(pj, (float)v8[t][c], acc[c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) red[slot * d + e0 + c] = acc[c];
        }
        __syncthreads();
        for (int i = tid; i < d; i += KT) {
            float s = 0.0f;
            for (int t = 0; t < 16; ++t) s += red[t * d + i];
            o[i] = rnd16(s * inv);
        }
        __syncthreads();
        // x = x + o Wo; h = rms_norm(x); u = gelu(h W1); x = x + u W2
        product(o, Wo, d, d, red, [&](int n, float s) { x[n] = rnd16(x[n] + rnd16(s)); });
        rms_norm_lds(x, h, d, m.eps, sm);
        float* u = q;  // hidden values: q, k, v, o are free (4 d floats, or h's tail)
        float* uu = (hid <= 4 * d) ? u : h + d;
        product(h, W1, d, hid, red, [&](int n, float s) { uu[n] = rnd16(gelu_f(rnd16(s))); });
        product(uu, W2, hid, d, red, [&](int n, float s) { x[n] = rnd16(x[n] + rnd16(s)); });
    }
    rms_norm_lds(x, h, d, m.eps, sm);
    f16* lg = a.logits + (int64_t)b * V;
    product(h, static_cast<const f16*>(m.w_out), d, V, red, [&](int n, float s) { lg[n] = (f16)s; });
}

}  // namespace

int kv_step_lds_bytes(const evkhip_kv_model& m) {
    const int d = (int)m.d, hid = (int)m.hidden;
    const int wide = d > hid ? d : hid;
    return (int)((d + wide + 4 * d + (int)m.max_seq + (16 * d > RED ? 16 * d : RED) + KWV) * sizeof(float));
}

}  // namespace evkhip

using namespace evkhip;

extern "C" int evkhip_kv_decode_step(const evkhip_kv_model* m, const uint16_t* ids, uint32_t pos, void* logits,
                                     void* stream) {
    EVK_RETURN_IF(!m || !ids || !logits || !m->emb || !m->w_out, EVKHIP_ERR_INVALID_ARG,
                  "kv_decode_step: null argument");
    EVK_RETURN_IF(m->batch == 0 || m->d == 0 || m->hidden == 0 || m->vocab == 0 || m->layers == 0 ||
                      m->max_seq == 0,
                  EVKHIP_ERR_INVALID_ARG, "kv_decode_step: empty model dimension");
    EVK_RETURN_IF(pos >= m->max_seq, EVKHIP_ERR_SHAPE, "kv_decode_step: position %u past max_seq %u", pos,
                  m->max_seq);
    EVK_RETURN_IF(m->layers > EVKHIP_KV_MAX_LAYERS || m->d % 8 || m->hidden % 8 || m->vocab % 8 || m->d > 2048 ||
                      m->hidden > 8192 || m->max_seq > 8192 || m->batch > 65535,
                  EVKHIP_ERR_UNSUPPORTED,
                  "kv_decode_step: needs d, hidden, vocab multiples of 8 (d <= 2048, hidden <= 8192), max_seq <= "
                  "8192 and at most %d layers",
                  EVKHIP_KV_MAX_LAYERS);
    bool al = aligned16(m->emb) && aligned16(m->w_out);
    for (uint32_t l = 0; l < m->layers; ++l) {
        for (int i = 0; i < 6; ++i) {
            EVK_RETURN_IF(!m->w[l][i], EVKHIP_ERR_INVALID_ARG, "kv_decode_step: null weight %d of layer %u", i, l);
            al = al && aligned16(m->w[l][i]);
        }
        EVK_RETURN_IF(!m->k_cache[l] || !m->v_cache[l], EVKHIP_ERR_INVALID_ARG, "kv_decode_step: null cache of layer %u",
                      l);
        al = al && aligned16(m->k_cache[l]) && aligned16(m->v_cache[l]);
    }
    EVK_RETURN_IF(!al, EVKHIP_ERR_UNSUPPORTED, "kv_decode_step: needs 16-byte aligned weights and caches");
    const int lds = kv_step_lds_bytes(*m);
    int dev = 0, lds_max = 0;
    EVK_HIP(hipGetDevice(&dev));
    EVK_HIP(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    EVK_RETURN_IF(lds > lds_max, EVKHIP_ERR_UNSUPPORTED, "kv_decode_step: needs %d bytes of LDS, the GPU has %d", lds,
                  lds_max);
    KvArgs a{};
    a.m = *m;
    a.ids = ids;
    a.pos = (int)pos;
    a.logits = static_cast<f16*>(logits);
    hipLaunchKernelGGL(kv_step, dim3(m->batch), dim3(KT), (unsigned)lds, reinterpret_cast<hipStream_t>(stream), a);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "kv_decode_step launch");
}
