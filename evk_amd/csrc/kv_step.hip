// Fused KV-cached decode step of the reference caller's model: the blocks
// example/main_llm.cpp:528-546 builds (rms_norm, x.Wq / x.Wk / x.Wv, rope on
// q and k, causal attention, x + attn.Wo, rms_norm, gelu(x.W1).W2 residual),
// then rms_norm and x.Wout, for one new position of B sequences.  The
// reference samples by recomputing the whole sequence per position
// (main_llm.cpp:622-654); evk::ai::KVCacheDecoder keeps the keys and values
// and runs one position per step, op by op (16 launches a layer).  Here one
// workgroup per sequence (two, at d = 256, where they all fit on the GPU at
// once) runs every layer of the step and the logits in a single launch: at
// this size (d = 256, 1 MB of weights a layer) a step is bound by launch and
// memory latency, not by bytes, and a sequence's step needs no exchange with
// the other sequences.
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

// ---------------------------------------------------------------------------
// The step at d = 256 with hidden a multiple of 256 up to 1024 (the reference
// caller's shape has hidden 512): the same arithmetic and roundings as
// kv_step, reorganised so that the weight stream never stops.
//
// The weights are cut into units of 256 input rows x 256 output columns
// (128 KB of fp16): Wq, Wk, Wv, Wo, the hidden/256 column blocks of W1 and
// row blocks of W2 of each layer, then the column blocks of the LM head.  A
// thread owns 8 columns (cg = tid % 32) and 16 consecutive rows
// (kg = tid / 32) of a unit: 16 loads of 16 bytes, one 512-byte row per half
// wave and load.  Two register slots alternate: the next unit's loads are
// requested before the current unit is multiplied, so one unit is always in
// flight, also across the attention, the norms and the barriers (one
// workgroup streams about 110 GB/s from L2 with 64 KB or more in flight).
// A unit's row partial sums cross the two half-waves by a permlane swap and
// the eight waves in LDS, summed in wave order.  The q, k and v units share
// one barrier, and so do the W1 blocks.  rms_norm: the threads that write x
// also form its sum of squares (per wave, DPP), and each thread normalises
// only the 16 rows it multiplies, in registers.
//
// Attention: slot = tid / 32 takes keys slot, slot + 16, ...; its 32 lanes
// hold 8 dimensions each.  A score is a DPP sum within 16-lane rows plus a
// permlane swap across the slot's two rows, so every lane of the slot holds
// it.  Each slot runs an online softmax over its keys, four keys a pass with
// their K and V rows requested together (the first pass's before the v unit
// is multiplied, ahead of Wo, so they do not queue behind it); the two slots
// of a wave merge by a permlane swap and the eight waves in one LDS pass.
// ---------------------------------------------------------------------------
constexpr int U = 256;        // unit rows and columns; the model width
constexpr int UPART = 8 * U;  // floats of one unit's wave partials
constexpr int KB4 = 4;        // keys of a slot per attention pass

DEV float dpp_sum_row16(float x) {
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
    return x;
}
// rows 0 + 1 and rows 2 + 3 (16-lane rows), the same sum in every lane of the pair
DEV float add_row_pairs(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// lanes i and i + 32, the same sum in both
DEV float add_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

int kv_step256_lds_floats(const evkhip_kv_model& m) { return 5 * U + 32 + (int)m.hidden + 4 * UPART; }

__global__ __launch_bounds__(KT, 1) void kv_step256(KvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float kv_smem[];
    const evkhip_kv_model& m = a.m;
    const int hid = (int)m.hidden, V = (int)m.vocab, NL = (int)m.layers;
    const int nh = hid / U;  // W1 column blocks = W2 row blocks
    const int b = blockIdx.x, pos = a.pos, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cg = tid & 31, kg = tid >> 5;  // units: 8 columns, 16 rows; attention: 8 dimensions, key slot
    float* x = kv_smem;          // U: the residual stream
    float* q = x + U;            // U
    float* kk = q + U;           // U
    float* vv = kk + U;          // U
    float* o = vv + U;           // U
    float* ssq = o + U;          // 8: sums of squares of x per wave (waves 0-3)
    float* smax = ssq + 8;       // 16: the attention's running maximum per wave (8 used)
    float* lsum = smax + 16;     // 8: the attention's probability sum per wave
    float* u = lsum + 8;         // hid: gelu outputs
    float* part = u + hid;       // 4 x UPART: wave partials of up to four units

    const auto Wl = [&](int l, int i) { return static_cast<const f16*>(m.w[l][i]); };
    const f16* Wout = static_cast<const f16*>(m.w_out);
    const int nvb = (V + U - 1) / U;  // LM head column blocks
    // a unit's 16 loads through a descriptor over [base, base + bytes), rows
    // stride_b bytes apart (the row step in the scalar offset, so one VGPR
    // addresses all 16); lanes with !ok (the LM head's columns past the
    // vocabulary) get an offset past any descriptor and read zeros.  No
    // branch: the loads always go out, so the waits of the unit consumed next
    // count them exactly.
    const auto issue = [&](u32x4(&w)[16], const f16* base, uint32_t stride_b, uint32_t bytes, bool ok) {
        const auto r = buf_rsrc(base, bytes);
        const uint32_t v0 = oob_or(ok, (uint32_t)(kg * 16) * stride_b + (uint32_t)cg * 16);
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = buf_load16(r, v0, (uint32_t)i * stride_b);
        __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the work that follows
    };
    constexpr uint32_t UB = U * U * 2;  // bytes of a U x U matrix
    const auto issue_lm = [&](u32x4(&w)[16], int vb) {  // LM head column block vb (zeros past the last)
        const int c0 = min(vb, nvb) * U;
        issue(w, Wout + c0, (uint32_t)V * 2, (uint32_t)(U * V - c0) * 2, c0 + cg * 8 < V);
    };
    const auto fma_unit = [&](const u32x4(&w)[16], const float(&in)[16], float(&acc)[8]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const half8 hw = as_half8(w[i]);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(in[i], (float)hw[c], acc[c]);
        }
    };
    // the wave's sums of a unit's columns (its two row ranges) into part[buf]
    const auto put_part = [&](float(&acc)[8], int buf) {
        float r[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = add_halves(acc[c]);
        const float4 st = lane < 32 ? float4{r[0], r[1], r[2], r[3]} : float4{r[4], r[5], r[6], r[7]};
        *reinterpret_cast<float4*>(part + buf * UPART + wave * U + cg * 8 + (lane >> 5) * 4) = st;
    };
    const auto col_sum = [&](int buf, int n) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) s += part[buf * UPART + w * U + n];
        return s;
    };
    const auto lds_rows = [&](const float* src, float(&in)[16]) {
        const float4* p = reinterpret_cast<const float4*>(src + kg * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 v = p[j];
            in[4 * j] = v.x;
            in[4 * j + 1] = v.y;
            in[4 * j + 2] = v.z;
            in[4 * j + 3] = v.w;
        }
    };
    // threads 0..U-1 (waves 0-3), v = x[tid]: ssq[wave] = sum of clamp(x)^2 over the wave
    const auto sumsq_store = [&](float v) {
        const float c = fminf(fmaxf(v, -65504.0f), 65504.0f);
        const float s = add_halves(add_row_pairs(dpp_sum_row16(c * c)));
        if (lane == 0) ssq[wave] = s;
    };
    // h = fp16(clamp(x) / sqrt(mean(clamp(x)^2) + eps)) of this thread's 16 rows, as rms_norm_k
    float hr[16];
    const auto norm_rows = [&]() {
        const float inv = 1.0f / sqrtf((ssq[0] + ssq[1] + ssq[2] + ssq[3]) / (float)U + m.eps);
        float xr[16];
        lds_rows(x, xr);
#pragma unroll
        for (int i = 0; i < 16; ++i) hr[i] = rnd16(fminf(fmaxf(xr[i], -65504.0f), 65504.0f) * inv);
    };

    u32x4 wa[16], wb[16];
    issue(wa, Wl(0, 0), 2 * U, UB, true);
    // rope angles of this position: threads 0..U-1 take pair tid % (U / 2)
    float rc = 1.0f, rs = 0.0f;
    if (tid < U) {
        const int pr = tid & (U / 2 - 1);
        const float inv_freq = powf(m.rope_base, -2.0f * (float)pr / (float)U);
        sincosf((float)pos * inv_freq, &rs, &rc);
        const int tok = min((int)a.ids[b], V - 1);
        const float v = (float)static_cast<const f16*>(m.emb)[(int64_t)tok * U + tid];
        x[tid] = v;
        sumsq_store(v);
    }
    __syncthreads();
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)U);

    for (int l = 0; l < NL; ++l) {
        // this sequence's cache rows; the offset is formed in scalar registers
        // so that the descriptors below need no per-lane loop
        const uint64_t seq_off = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(b * (int)m.max_seq) * U;
        f16* Kc = static_cast<f16*>(m.k_cache[l]) + seq_off;
        f16* Vc = static_cast<f16*>(m.v_cache[l]) + seq_off;
        norm_rows();
        float acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
        issue(wb, Wl(l, 1), 2 * U, UB, true);
        fma_unit(wa, hr, acc);
        put_part(acc, 0);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
        issue(wa, Wl(l, 2), 2 * U, UB, true);
        fma_unit(wb, hr, acc);
        put_part(acc, 1);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
        // the attention's first keys and values (cache rows, independent of
        // this step) go out before the v unit is multiplied, Wo after it, so
        // that they do not queue behind Wo.  Descriptors over the rows
        // [0, pos): rows at and past pos read zeros.
        const auto rK = buf_rsrc(Kc, (uint32_t)pos * U * 2), rV = buf_rsrc(Vc, (uint32_t)pos * U * 2);
        half8 kp[KB4], vp[KB4];
#pragma unroll
        for (int t = 0; t < KB4; ++t) {
            kp[t] = as_half8(buf_load16(rK, (uint32_t)((kg + 16 * t) * U + cg * 8) * 2, 0));
            vp[t] = as_half8(buf_load16(rV, (uint32_t)((kg + 16 * t) * U + cg * 8) * 2, 0));
        }
        fma_unit(wa, hr, acc);
        issue(wb, Wl(l, 3), 2 * U, UB, true);
        put_part(acc, 2);
        __syncthreads();
        // q, k = rope(fp16(h Wq)), rope(fp16(h Wk)) (threads 0..127 q pairs,
        // 128..255 k pairs), v = fp16(h Wv); the cache rows of this position
        if (tid < U) {
            const int pr = tid & (U / 2 - 1);
            const float* pp = part + (tid < U / 2 ? 0 : UPART) + 2 * pr;
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const float2 t = *reinterpret_cast<const float2*>(pp + w * U);
                s0 += t.x;
                s1 += t.y;
            }
            const float a0 = rnd16(s0), a1 = rnd16(s1);
            const float r0 = a0 * rc - a1 * rs, r1 = a0 * rs + a1 * rc;
            if (tid < U / 2) {
                q[2 * pr] = rnd16(r0);
                q[2 * pr + 1] = rnd16(r1);
            } else {
                const f16 k0 = (f16)r0, k1 = (f16)r1;
                *reinterpret_cast<uint32_t*>(Kc + (int64_t)pos * U + 2 * pr) =
                    (uint32_t)__builtin_bit_cast(uint16_t, k0) | ((uint32_t)__builtin_bit_cast(uint16_t, k1) << 16);
                kk[2 * pr] = (float)k0;
                kk[2 * pr + 1] = (float)k1;
            }
        } else {
            const int n = tid - U;
            const float v = rnd16(col_sum(2, n));
            vv[n] = v;
            Vc[(int64_t)pos * U + n] = (f16)v;
        }
        __syncthreads();

        // attention: each key slot runs an online softmax over its keys
        // kg, kg + 16, ... (KB4 keys a pass, K and V rows requested together),
        // the slots of a wave merge by a permlane swap and the waves in LDS.
        // Key pos (this step's k and v, from LDS) is the last key of slot
        // pos % 16.
        float qv[8];
        {
            const float4 q0 = *reinterpret_cast<const float4*>(q + cg * 8);
            const float4 q1 = *reinterpret_cast<const float4*>(q + cg * 8 + 4);
            qv[0] = q0.x, qv[1] = q0.y, qv[2] = q0.z, qv[3] = q0.w;
            qv[4] = q1.x, qv[5] = q1.y, qv[6] = q1.z, qv[7] = q1.w;
        }
        float m_run = -INFINITY, l_run = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
        // keys j0 + kg + 16 t (t < KB4) that are below pos
        const auto absorb = [&](const half8(&kx)[KB4], const half8(&vx)[KB4], int j0) {
            float sv[KB4];
            float mn = m_run;
#pragma unroll
            for (int t = 0; t < KB4; ++t) {
                float d = 0.0f;
#pragma unroll
                for (int c = 0; c < 8; ++c) d = __builtin_fmaf(qv[c], (float)kx[t][c], d);
                sv[t] = add_row_pairs(dpp_sum_row16(d)) * scale_log2;
                mn = j0 + kg + 16 * t < pos ? fmaxf(mn, sv[t]) : mn;
            }
            const float f = m_run == -INFINITY ? 0.0f : exp2f(m_run - mn);
            l_run *= f;
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] *= f;
#pragma unroll
            for (int t = 0; t < KB4; ++t)
                if (j0 + kg + 16 * t < pos) {
                    const float pr = exp2f(sv[t] - mn);
                    l_run += pr;
#pragma unroll
                    for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(pr, (float)vx[t][c], acc[c]);
                }
            m_run = mn;
        };
        absorb(kp, vp, 0);
        for (int j0 = 16 * KB4; j0 < pos; j0 += 16 * KB4) {
#pragma unroll
            for (int t = 0; t < KB4; ++t) {
                kp[t] = as_half8(buf_load16(rK, (uint32_t)((j0 + kg + 16 * t) * U + cg * 8) * 2, 0));
                vp[t] = as_half8(buf_load16(rV, (uint32_t)((j0 + kg + 16 * t) * U + cg * 8) * 2, 0));
            }
            absorb(kp, vp, j0);
        }
        {
            const float4 k0 = *reinterpret_cast<const float4*>(kk + cg * 8);
            const float4 k1 = *reinterpret_cast<const float4*>(kk + cg * 8 + 4);
            const float kr[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            float d = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) d = __builtin_fmaf(qv[c], kr[c], d);
            const float s2 = add_row_pairs(dpp_sum_row16(d)) * scale_log2;  // the same in every slot
            if (kg == (pos & 15)) {
                const float mn = fmaxf(m_run, s2);
                const float f = m_run == -INFINITY ? 0.0f : exp2f(m_run - mn), pr = exp2f(s2 - mn);
                const float4 v0 = *reinterpret_cast<const float4*>(vv + cg * 8);
                const float4 v1 = *reinterpret_cast<const float4*>(vv + cg * 8 + 4);
                const float vr[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                l_run = l_run * f + pr;
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(pr, vr[c], acc[c] * f);
                m_run = mn;
            }
        }
        // the wave's two slots (lanes 0-31 and 32-63)
        {
            const auto rm = __builtin_amdgcn_permlane32_swap(__float_as_uint(m_run), __float_as_uint(m_run), false, false);
            const float m_lo = __uint_as_float(rm[0]), m_hi = __uint_as_float(rm[1]), mw = fmaxf(m_lo, m_hi);
            const float f_lo = m_lo == -INFINITY ? 0.0f : exp2f(m_lo - mw);
            const float f_hi = m_hi == -INFINITY ? 0.0f : exp2f(m_hi - mw);
            float r[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[c]), __float_as_uint(acc[c]), false, false);
                r[c] = __uint_as_float(t[0]) * f_lo + __uint_as_float(t[1]) * f_hi;
            }
            const auto rl = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
            const float lw = __uint_as_float(rl[0]) * f_lo + __uint_as_float(rl[1]) * f_hi;
            const float4 st = lane < 32 ? float4{r[0], r[1], r[2], r[3]} : float4{r[4], r[5], r[6], r[7]};
            *reinterpret_cast<float4*>(part + wave * U + cg * 8 + (lane >> 5) * 4) = st;
            if (lane == 0) {
                smax[wave] = mw;
                lsum[wave] = lw;
            }
        }
        __syncthreads();
        if (tid < U) {
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 8; ++w) M = fmaxf(M, smax[w]);
            float num = 0.0f, den = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const float f = smax[w] == -INFINITY ? 0.0f : exp2f(smax[w] - M);
                num = __builtin_fmaf(part[w * U + tid], f, num);
                den = __builtin_fmaf(lsum[w], f, den);
            }
            o[tid] = rnd16(num * (1.0f / den));
        }
        __syncthreads();

        // x = x + fp16(o Wo); the first W1 block goes out
        {
            float in[16];
            lds_rows(o, in);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
            issue(wa, Wl(l, 4), (uint32_t)hid * 2, (uint32_t)(U * hid) * 2, true);
            fma_unit(wb, in, acc);
            put_part(acc, 1);
        }
        __syncthreads();
        if (tid < U) {
            const float v = rnd16(x[tid] + rnd16(col_sum(1, tid)));
            x[tid] = v;
            sumsq_store(v);
        }
        __syncthreads();
        norm_rows();

        // MLP units t = 0 .. 2 nh - 1: W1 column block t (t < nh), then W2
        // row block t - nh; unit t sits in slot wa for even t.  After them
        // comes the next layer's Wq or the LM head's first block.
        float acc2[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc2[c] = 0.0f;
        const auto next_unit = [&](u32x4(&w)[16], int t) {  // selects only: one issue site
            const bool w1 = t < nh, w2 = !w1 && t < 2 * nh, lm = t >= 2 * nh && l + 1 == NL;
            const f16* base = w1   ? Wl(l, 4) + t * U
                              : w2 ? Wl(l, 5) + (int64_t)(t - nh) * U * U
                              : lm ? Wout
                                   : Wl(l + 1, 0);
            const uint32_t stride_b = w1 ? (uint32_t)hid * 2 : lm ? (uint32_t)V * 2 : 2 * U;
            const uint32_t bytes = w1 ? (uint32_t)(U * hid - t * U) * 2 : lm ? (uint32_t)(U * V) * 2 : UB;
            issue(w, base, stride_b, bytes, !lm || cg * 8 < V);
        };
        const auto consume_mlp = [&](const u32x4(&w)[16], int t) {
            if (t < nh) {
                float a1[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) a1[c] = 0.0f;
                fma_unit(w, hr, a1);
                put_part(a1, t);
                if (t == nh - 1) {
                    __syncthreads();
                    for (int n = tid; n < hid; n += KT) u[n] = rnd16(gelu_f(rnd16(col_sum(n / U, n % U))));
                    __syncthreads();
                }
            } else {
                float in[16];
                lds_rows(u + (t - nh) * U, in);
                fma_unit(w, in, acc2);
                if (t == 2 * nh - 1) {
                    put_part(acc2, 0);
                    __syncthreads();
                    if (tid < U) {
                        const float v = rnd16(x[tid] + rnd16(col_sum(0, tid)));
                        x[tid] = v;
                        sumsq_store(v);
                    }
                    __syncthreads();
                }
            }
        };
        for (int t = 0; t < 2 * nh; t += 2) {
            next_unit(wb, t + 1);
            consume_mlp(wa, t);
            next_unit(wa, t + 2);
            consume_mlp(wb, t + 1);
        }
    }

    // logits = fp16(rms_norm(x) Wout), column blocks of U; block vb sits in
    // slot wa for even vb
    norm_rows();
    f16* lg = a.logits + (int64_t)b * V;
    const auto lm_block = [&](const u32x4(&w)[16], int vb) {
        float a1[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) a1[c] = 0.0f;
        fma_unit(w, hr, a1);
        put_part(a1, vb & 1);
        __syncthreads();
        if (tid < U && vb * U + tid < V) lg[vb * U + tid] = (f16)col_sum(vb & 1, tid);
    };
    for (int vb = 0; vb < nvb; vb += 2) {  // an odd count ends with a block of zeros, not stored
        issue_lm(wb, vb + 1);
        lm_block(wa, vb);
        issue_lm(wa, vb + 2);
        lm_block(wb, vb + 1);
    }
}


// ---------------------------------------------------------------------------
// The d = 256 step on two workgroups per sequence (hidden a multiple of 256
// up to 1024).  Workgroup j of sequence b takes output columns
// [128 j, 128 j + 128) of q, k and v, the attention's v columns of the same
// range over every cached key, the rows of Wo that those columns multiply,
// hidden columns [j hidden / 2, (j + 1) hidden / 2) of W1 and the rows of W2
// that they multiply, and the LM-head blocks of 128 columns j, j + 2, ...;
// so each streams half of the weights.  A layer needs three swaps between
// the two: q and k; the fp32 partial products of Wo (every column); those of
// W2.  Both add the two partials in the same way, so they hold identical
// copies of x and round the same values the same way.  The swaps go through
// 64-bit words in device memory: the payload in the low half, the launch's
// tag in the high half, written and read at agent scope, so that a word's
// payload and tag always arrive together.  A mailbox copy is reused two
// layers later (layer parity), by which time the partner has read it (it
// cannot start that layer's phase before it has answered the one in
// between).  Waits are bounded; one that gives up raises a status bit and
// the step's outputs are then unreliable.
// A unit here is 256 rows x 128 columns: a thread owns 8 columns (cg = tid %
// 16) and 8 rows (kg = tid / 16).
// ---------------------------------------------------------------------------
constexpr int UC = 128;         // unit columns
constexpr int PPART = 8 * UC;   // floats of one unit's wave partials
constexpr int MBW = 640;        // mailbox words per (sequence, workgroup, layer parity)
constexpr int MB_QK = 0, MB_X1 = 128, MB_X2 = 384;
static_assert(EVKHIP_KV_MAX_LAYERS * 3 <= 256, "a layer's three tags sit in the tag's low byte");
constexpr int KBP = 8;          // keys of a slot per attention pass

// four halves at byte offset voff (zeros past the descriptor's end)
DEV half4 buf_load_h4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0));
}

struct KvPairArgs {
    KvArgs a;
    uint64_t* mb;      // (batch, 2, 2, MBW) words
    uint32_t launch;   // this launch's tag base, >= 1
    int spin;          // polls before a wait gives up
};

__device__ unsigned g_kv_pair_status;

DEV void kv_put(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// the payload of *p once it carries `tag` (bounded)
DEV uint32_t kv_take(const uint64_t* p, uint32_t tag, int spin) {
    uint64_t v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int s = 0; (uint32_t)(v >> 32) != tag && s < spin; ++s) {
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if ((uint32_t)(v >> 32) != tag)
        __hip_atomic_fetch_or(&g_kv_pair_status, (unsigned)EVKHIP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    return (uint32_t)v;
}

int kv_pair_lds_floats(const evkhip_kv_model& m) { return 5 * U + 32 + (int)m.hidden + 4 * PPART + 8; }

__global__ __launch_bounds__(KT, 1) void kv_step256x2(KvPairArgs pa) {
    extern __shared__ __attribute__((aligned(16))) float kv_smem[];
    const KvArgs& a = pa.a;
    const evkhip_kv_model& m = a.m;
    const int hid = (int)m.hidden, V = (int)m.vocab, NL = (int)m.layers, B = (int)m.batch;
    const int nh2 = hid / U;             // this workgroup's W1 column units = W2 row units
    const int b = blockIdx.x % B, j = blockIdx.x / B, pos = a.pos, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cg = tid & 15, kg = tid >> 4;  // units: 8 of 128 columns, 8 of 256 rows
    const int c0 = j * UC, pc0 = (j ^ 1) * UC;  // this and the partner's d-wide columns
    const int h0 = j * (hid / 2);  // and hidden columns
    float* x = kv_smem;          // U: the residual stream
    float* q = x + U;            // U
    float* kk = q + U;           // U
    float* vv = kk + U;          // U
    float* o = vv + U;           // U
    float* ssq = o + U;          // 8: sums of squares of x per wave (waves 0-3)
    float* smax = ssq + 8;       // 16: the attention's running maximum per wave
    float* lsum = smax + 16;     // 8: the attention's probability sum per wave
    float* u = lsum + 8;         // hid: gelu outputs (this workgroup's half)
    float* part = u + hid;       // 4 x PPART: wave partials
    uint64_t* mine = pa.mb + (size_t)(b * 2 + j) * 2 * MBW;
    const uint64_t* theirs = pa.mb + (size_t)(b * 2 + (j ^ 1)) * 2 * MBW;
    const uint32_t tbase = pa.launch << 8;
    const int spin = pa.spin;

    const auto Wl = [&](int l, int i) { return static_cast<const f16*>(m.w[l][i]); };
    const f16* Wout = static_cast<const f16*>(m.w_out);
    // a unit of 256 rows x 128 columns (rows kg * 8 + i, columns cg * 8 ..)
    // or, rows128, of 128 rows x 256 columns (rows (kg % 16) * 8 + i,
    // columns (kg / 16) * 128 + cg * 8 ..: waves 0-3 the first 128 columns)
    const auto issue = [&](u32x4(&w)[8], const f16* base, uint32_t stride_b, uint32_t bytes, bool ok, bool rows128) {
        // the operands are uniform; formed in scalar registers so that the
        // loads need no per-lane descriptor loop
        const uint64_t bp = reinterpret_cast<uint64_t>(base);
        base = reinterpret_cast<const f16*>(
            ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(bp >> 32)) << 32) |
            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)bp));
        stride_b = (uint32_t)__builtin_amdgcn_readfirstlane((int)stride_b);
        bytes = (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes);
        const auto r = buf_rsrc(base, bytes);
        const uint32_t v0 = oob_or(ok, rows128 ? (uint32_t)((kg & 15) * 8) * stride_b + (uint32_t)((kg >> 4) * UC + cg * 8) * 2
                                               : (uint32_t)(kg * 8) * stride_b + (uint32_t)cg * 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = buf_load16(r, v0, (uint32_t)i * stride_b);
        __builtin_amdgcn_sched_barrier(0);
    };
    constexpr uint32_t UB = U * U * 2;
    const auto fma8 = [&](const u32x4(&w)[8], const float(&in)[8], float(&acc)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const half8 hw = as_half8(w[i]);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(in[i], (float)hw[c], acc[c]);
        }
    };
    const auto zero8 = [](float(&v)[8]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = 0.0f;
    };
    // the wave's sums of a unit's columns (its four row groups) into part[buf]:
    // row q of the wave's 16-lane rows stores columns cg * 8 + 2 q, + 1
    const auto put_part = [&](float(&acc)[8], int buf) {
        float r[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = add_halves(add_row_pairs(acc[c]));
        const int qr = lane >> 4;
        const float2 st = qr == 0 ? float2{r[0], r[1]} : qr == 1 ? float2{r[2], r[3]} : qr == 2 ? float2{r[4], r[5]}
                                                                                      : float2{r[6], r[7]};
        *reinterpret_cast<float2*>(part + buf * PPART + wave * UC + cg * 8 + 2 * qr) = st;
    };
    const auto col_sum = [&](int buf, int n) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) s += part[buf * PPART + w * UC + n];
        return s;
    };
    // column n (of 256) of a rows128 unit: the partials of waves 4 (n / 128) .. + 3
    const auto col_sum128 = [&](int buf, int n) {
        const float* p = part + buf * PPART + (n >> 7) * 4 * UC + (n & 127);
        return ((p[0] + p[UC]) + p[2 * UC]) + p[3 * UC];
    };
    const auto read8 = [](const float* p, float(&in)[8]) {
        const float4 v0 = *reinterpret_cast<const float4*>(p);
        const float4 v1 = *reinterpret_cast<const float4*>(p + 4);
        in[0] = v0.x, in[1] = v0.y, in[2] = v0.z, in[3] = v0.w;
        in[4] = v1.x, in[5] = v1.y, in[6] = v1.z, in[7] = v1.w;
    };
    // threads 0..U-1 (waves 0-3): ssq[wave] = sum of clamp(x)^2 over the wave
    const auto sumsq_all = [&]() {
        if (tid < U) {
            const float c = fminf(fmaxf(x[tid], -65504.0f), 65504.0f);
            const float s = add_halves(add_row_pairs(dpp_sum_row16(c * c)));
            if (lane == 0) ssq[wave] = s;
        }
    };
    float hr[8];  // rms_norm(x) of this thread's rows kg * 8 + i
    const auto norm_rows = [&]() {
        const float inv = 1.0f / sqrtf((ssq[0] + ssq[1] + ssq[2] + ssq[3]) / (float)U + m.eps);
        float xr[8];
        read8(x + kg * 8, xr);
#pragma unroll
        for (int i = 0; i < 8; ++i) hr[i] = rnd16(fminf(fmaxf(xr[i], -65504.0f), 65504.0f) * inv);
    };

    u32x4 wa[8], wb[8];
    issue(wa, Wl(0, 0) + c0, 2 * U, UB - c0 * 2, true, false);
    // rope angles: threads 0..127 take pair c0 / 2 + tid % 64 (q for tid < 64, k after)
    float rc = 1.0f, rs = 0.0f;
    if (tid < 128) {
        const int pr = c0 / 2 + (tid & 63);
        const float inv_freq = powf(m.rope_base, -2.0f * (float)pr / (float)U);
        sincosf((float)pos * inv_freq, &rs, &rc);
    }
    if (tid < U) {
        const int tok = min((int)a.ids[b], V - 1);
        x[tid] = (float)static_cast<const f16*>(m.emb)[(int64_t)tok * U + tid];
    }
    __syncthreads();
    sumsq_all();
    __syncthreads();
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)U);

    for (int l = 0; l < NL; ++l) {
        const uint64_t seq_off = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(b * (int)m.max_seq) * U;
        f16* Kc = static_cast<f16*>(m.k_cache[l]) + seq_off;
        f16* Vc = static_cast<f16*>(m.v_cache[l]) + seq_off;
        uint64_t* mbo = mine + (l & 1) * MBW;
        const uint64_t* mbi = theirs + (l & 1) * MBW;
        const uint32_t tg = tbase | (uint32_t)(l * 3);
        norm_rows();
        float acc[8];
        zero8(acc);
        issue(wb, Wl(l, 1) + c0, 2 * U, UB - c0 * 2, true, false);
        fma8(wa, hr, acc);
        put_part(acc, 0);
        zero8(acc);
        issue(wa, Wl(l, 2) + c0, 2 * U, UB - c0 * 2, true, false);
        fma8(wb, hr, acc);
        put_part(acc, 1);
        zero8(acc);
        // the attention's first cached keys (slot sl: keys 16 t + sl; a lane
        // scores 8 dimensions and sums 4 of this workgroup's v columns) go
        // out before the v unit is multiplied; rows past pos read zeros
        const int sl = tid >> 5, dg = tid & 31;
        const auto rK = buf_rsrc(Kc, (uint32_t)pos * U * 2), rV = buf_rsrc(Vc, (uint32_t)pos * U * 2);
        half8 kp[KBP];
        half4 vp[KBP];
#pragma unroll
        for (int t = 0; t < KBP; ++t) {
            const int key = 16 * t + sl;
            kp[t] = as_half8(buf_load16(rK, (uint32_t)(key * U + dg * 8) * 2, 0));
            vp[t] = buf_load_h4(rV, (uint32_t)(key * U + c0 + dg * 4) * 2);
        }
        fma8(wa, hr, acc);
        // Wo rows of this workgroup's o columns, all output columns
        issue(wb, Wl(l, 3) + (int64_t)c0 * U, 2 * U, (uint32_t)(U - c0) * U * 2, true, true);
        put_part(acc, 2);
        __syncthreads();
        // this workgroup's q, k (rope) and v columns; the cache row's columns;
        // q and k swapped with the partner (v stays: each sums its own columns)
        if (tid < 192) {
            const int i = tid & 63, kind = tid >> 6;  // 0 q, 1 k, 2 v: local pair i
            const float s0 = col_sum(kind, 2 * i), s1 = col_sum(kind, 2 * i + 1);
            const float a0 = rnd16(s0), a1 = rnd16(s1);
            if (kind == 0) {
                const float v0 = rnd16(a0 * rc - a1 * rs), v1 = rnd16(a0 * rs + a1 * rc);
                q[c0 + 2 * i] = v0;
                q[c0 + 2 * i + 1] = v1;
                kv_put(mbo + MB_QK + tid, tg, pack_h2(v0, v1));
            } else if (kind == 1) {
                const float v0 = (float)(f16)(a0 * rc - a1 * rs), v1 = (float)(f16)(a0 * rs + a1 * rc);
                kk[c0 + 2 * i] = v0;
                kk[c0 + 2 * i + 1] = v1;
                *reinterpret_cast<uint32_t*>(Kc + (int64_t)pos * U + c0 + 2 * i) = pack_h2(v0, v1);
                kv_put(mbo + MB_QK + tid, tg, pack_h2(v0, v1));
            } else {
                vv[c0 + 2 * i] = a0;
                vv[c0 + 2 * i + 1] = a1;
                *reinterpret_cast<uint32_t*>(Vc + (int64_t)pos * U + c0 + 2 * i) = pack_h2(a0, a1);
            }
            if (kind < 2) {
                const uint32_t w = kv_take(mbi + MB_QK + tid, tg, spin);
                float* dst = kind == 0 ? q : kk;
                dst[pc0 + 2 * i] = (float)__builtin_bit_cast(f16, (uint16_t)(w & 0xFFFFu));
                dst[pc0 + 2 * i + 1] = (float)__builtin_bit_cast(f16, (uint16_t)(w >> 16));
            }
        }
        __syncthreads();

        // attention over every cached key for this workgroup's v columns: an
        // online softmax per slot
        float qv[8];
        read8(q + dg * 8, qv);
        float m_run = -INFINITY, l_run = 0.0f;
        float av[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const auto absorb = [&](const half8(&kx)[KBP], const half4(&vx)[KBP], int p0) {
            float sv[KBP];
            float mn = m_run;
#pragma unroll
            for (int t = 0; t < KBP; ++t) {
                sv[t] = 0.0f;
                // keys 16 t + p0 .. + 15 all at or past pos: no slot scores
                // (a uniform branch; their loads read zeros and stay)
                if (p0 + 16 * t < pos) {
                    float d = 0.0f;
#pragma unroll
                    for (int c = 0; c < 8; ++c) d = __builtin_fmaf(qv[c], (float)kx[t][c], d);
                    sv[t] = add_row_pairs(dpp_sum_row16(d)) * scale_log2;
                    mn = p0 + 16 * t + sl < pos ? fmaxf(mn, sv[t]) : mn;
                }
            }
            const float f = m_run == -INFINITY ? 0.0f : exp2f(m_run - mn);
            l_run *= f;
#pragma unroll
            for (int c = 0; c < 4; ++c) av[c] *= f;
#pragma unroll
            for (int t = 0; t < KBP; ++t)
                if (p0 + 16 * t + sl < pos) {
                    const float pr = exp2f(sv[t] - mn);
                    l_run += pr;
#pragma unroll
                    for (int c = 0; c < 4; ++c) av[c] = __builtin_fmaf(pr, (float)vx[t][c], av[c]);
                }
            m_run = mn;
        };
        absorb(kp, vp, 0);
        for (int p0 = 16 * KBP; p0 < pos; p0 += 16 * KBP) {
#pragma unroll
            for (int t = 0; t < KBP; ++t) {
                const int key = p0 + 16 * t + sl;
                kp[t] = as_half8(buf_load16(rK, (uint32_t)(key * U + dg * 8) * 2, 0));
                vp[t] = buf_load_h4(rV, (uint32_t)(key * U + c0 + dg * 4) * 2);
            }
            absorb(kp, vp, p0);
        }
        {
            float kr[8];
            read8(kk + dg * 8, kr);
            float d = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) d = __builtin_fmaf(qv[c], kr[c], d);
            const float s2 = add_row_pairs(dpp_sum_row16(d)) * scale_log2;
            if (sl == (pos & 15)) {
                const float mn = fmaxf(m_run, s2);
                const float f = m_run == -INFINITY ? 0.0f : exp2f(m_run - mn), pr = exp2f(s2 - mn);
                const float4 vr = *reinterpret_cast<const float4*>(vv + c0 + dg * 4);
                l_run = l_run * f + pr;
                av[0] = __builtin_fmaf(pr, vr.x, av[0] * f);
                av[1] = __builtin_fmaf(pr, vr.y, av[1] * f);
                av[2] = __builtin_fmaf(pr, vr.z, av[2] * f);
                av[3] = __builtin_fmaf(pr, vr.w, av[3] * f);
                m_run = mn;
            }
        }
        {
            const auto rm = __builtin_amdgcn_permlane32_swap(__float_as_uint(m_run), __float_as_uint(m_run), false, false);
            const float m_lo = __uint_as_float(rm[0]), m_hi = __uint_as_float(rm[1]), mw = fmaxf(m_lo, m_hi);
            const float f_lo = m_lo == -INFINITY ? 0.0f : exp2f(m_lo - mw);
            const float f_hi = m_hi == -INFINITY ? 0.0f : exp2f(m_hi - mw);
            float r[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(av[c]), __float_as_uint(av[c]), false, false);
                r[c] = __uint_as_float(t[0]) * f_lo + __uint_as_float(t[1]) * f_hi;
            }
            const auto rl = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
            const float lw = __uint_as_float(rl[0]) * f_lo + __uint_as_float(rl[1]) * f_hi;
            const float2 st = lane < 32 ? float2{r[0], r[1]} : float2{r[2], r[3]};
            *reinterpret_cast<float2*>(part + wave * UC + dg * 4 + (lane >> 5) * 2) = st;
            if (lane == 0) {
                smax[wave] = mw;
                lsum[wave] = lw;
            }
        }
        __syncthreads();
        // the waves' partials merged: o over this workgroup's columns
        if (tid < UC) {
            float Mw = -INFINITY, num = 0.0f, den = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; ++w) Mw = fmaxf(Mw, smax[w]);
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const float f = smax[w] == -INFINITY ? 0.0f : exp2f(smax[w] - Mw);
                num = __builtin_fmaf(part[w * UC + tid], f, num);
                den = __builtin_fmaf(lsum[w], f, den);
            }
            o[c0 + tid] = rnd16(num * (1.0f / den));
        }
        __syncthreads();

        // x = x + fp16(o Wo): this workgroup's rows of Wo give a partial of
        // every column; the partner's partial added (a + b == b + a exactly)
        {
            float in[8];
            read8(o + c0 + (kg & 15) * 8, in);
            zero8(acc);
            issue(wa, Wl(l, 4) + h0, (uint32_t)hid * 2, (uint32_t)(U * hid - h0) * 2, true, false);
            fma8(wb, in, acc);
            put_part(acc, 1);
        }
        __syncthreads();
        if (tid < U) {
            const float p = col_sum128(1, tid);
            kv_put(mbo + MB_X1 + tid, tg + 1, __float_as_uint(p));
            const float pp = __uint_as_float(kv_take(mbi + MB_X1 + tid, tg + 1, spin));
            x[tid] = rnd16(x[tid] + rnd16(p + pp));
        }
        sumsq_all();
        __syncthreads();
        norm_rows();

        // MLP units t = 0 .. 2 nh2 - 1: W1 column unit t of this workgroup's
        // hidden half (t < nh2), then W2 rows t - nh2 of that half (128 each)
        float acc2[8];
        zero8(acc2);
        const auto next_unit = [&](u32x4(&w)[8], int t) {
            const bool w1 = t < nh2, w2 = !w1 && t < 2 * nh2, lm = t >= 2 * nh2 && l + 1 == NL;
            const int vb0 = j * UC;  // the LM head's first block of this workgroup
            const int r2 = h0 + (t - nh2) * UC;  // first W2 row of unit t
            const f16* base = w1   ? Wl(l, 4) + h0 + t * UC
                              : w2 ? Wl(l, 5) + (int64_t)r2 * U
                              : lm ? Wout + vb0
                                   : Wl(l + 1 < NL ? l + 1 : l, 0) + c0;
            const uint32_t stride_b = w1 ? (uint32_t)hid * 2 : lm ? (uint32_t)V * 2 : 2 * U;
            const uint32_t bytes = w1   ? (uint32_t)(U * hid - h0 - t * UC) * 2
                                   : w2 ? (uint32_t)(hid - r2) * U * 2
                                   : lm ? (uint32_t)(U * V - (vb0 < V ? vb0 : 0)) * 2
                                        : UB - c0 * 2;
            issue(w, base, stride_b, bytes, !lm || vb0 + cg * 8 < V, w2);
        };
        const auto consume_mlp = [&](const u32x4(&w)[8], int t) {
            if (t < nh2) {
                float a1[8];
                zero8(a1);
                fma8(w, hr, a1);
                put_part(a1, t);
                if (t == nh2 - 1) {
                    __syncthreads();
                    for (int i = tid; i < hid / 2; i += KT) u[h0 + i] = rnd16(gelu_f(rnd16(col_sum(i / UC, i % UC))));
                    __syncthreads();
                }
            } else {
                float in[8];
                read8(u + h0 + (t - nh2) * UC + (kg & 15) * 8, in);
                fma8(w, in, acc2);
                if (t == 2 * nh2 - 1) {
                    put_part(acc2, 0);
                    __syncthreads();
                    if (tid < U) {
                        const float p = col_sum128(0, tid);
                        kv_put(mbo + MB_X2 + tid, tg + 2, __float_as_uint(p));
                        const float pp = __uint_as_float(kv_take(mbi + MB_X2 + tid, tg + 2, spin));
                        x[tid] = rnd16(x[tid] + rnd16(p + pp));
                    }
                    sumsq_all();
                    __syncthreads();
                }
            }
        };
        for (int t = 0; t < 2 * nh2; t += 2) {
            next_unit(wb, t + 1);
            consume_mlp(wa, t);
            next_unit(wa, t + 2);
            consume_mlp(wb, t + 1);
        }
    }

    // logits: this workgroup's LM-head blocks of 128 columns, j, j + 2, ...
    norm_rows();
    f16* lg = a.logits + (int64_t)b * V;
    const int nvb = (V + UC - 1) / UC;
    const auto issue_lm = [&](u32x4(&w)[8], int vb) {  // zeros past the last block
        const int cb = (vb < nvb ? vb : nvb) * UC;
        issue(w, Wout + cb, (uint32_t)V * 2, (uint32_t)(U * V - cb) * 2, cb + cg * 8 < V, false);
    };
    const auto lm_block = [&](u32x4(&w)[8], int vb, int buf) {
        float a1[8];
        zero8(a1);
        fma8(w, hr, a1);
        issue_lm(w, vb + 4);
        put_part(a1, buf);
        __syncthreads();
        if (tid < UC && vb * UC + tid < V) lg[vb * UC + tid] = (f16)col_sum(buf, tid);
    };
    issue_lm(wb, j + 2);
    for (int vb = j; vb < nvb; vb += 4) {
        lm_block(wa, vb, 0);
        lm_block(wb, vb + 2, 1);
    }
}

}  // namespace

int kv_step_lds_bytes(const evkhip_kv_model& m) {
    const int d = (int)m.d, hid = (int)m.hidden;
    const int wide = d > hid ? d : hid;
    return (int)((d + wide + 4 * d + (int)m.max_seq + (16 * d > RED ? 16 * d : RED) + KWV) * sizeof(float));
}

}  // namespace evkhip

using namespace evkhip;

// ---- the pair step's mailboxes (grow-only; zeroed when allocated) ----
namespace evkhip {
namespace {
struct KvPairWs {
    uint64_t* mb = nullptr;
    size_t words = 0;
    int dev = -1;
    uint32_t launch = 0;  // tag base of the last launch
};
KvPairWs g_kvp;
}  // namespace

void kv_step_free_workspace() {
    if (g_kvp.mb) (void)hipFree(g_kvp.mb);
    g_kvp = KvPairWs{};
}

int kv_step_status(uint32_t* flags, bool clear) {
    unsigned v = 0;
    EVK_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_kv_pair_status), sizeof(v), 0, hipMemcpyDeviceToHost));
    if (clear && v) {
        const unsigned zero = 0;
        EVK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_kv_pair_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice));
    }
    *flags = v;
    return EVKHIP_OK;
}
}  // namespace evkhip

extern "C" int evkhip_debug_kv_set_launch(uint32_t distance) {
    EVK_RETURN_IF(distance == 0 || distance >= (1u << 24), EVKHIP_ERR_INVALID_ARG,
                  "debug_kv_set_launch: distance %u outside [1, 2^24)", distance);
    EVK_RETURN_IF(!g_kvp.mb, EVKHIP_ERR_UNSUPPORTED,
                  "debug_kv_set_launch: no multi-workgroup kv decode step has run in this process");
    EVK_HIP(hipDeviceSynchronize());
    g_kvp.launch = (1u << 24) - distance;
    return EVKHIP_OK;
}

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
    // d = 256 with hidden a multiple of 256 up to 1024: the streamed step
    const bool units = m->d == U && m->hidden % U == 0 && m->hidden <= 4 * U;
    const int lds = units ? kv_step256_lds_floats(*m) * (int)sizeof(float) : kv_step_lds_bytes(*m);
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
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // two workgroups a sequence where all of them fit on the GPU at once and
    // the launch is not captured (its tags come from a host counter)
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    EVK_HIP(hipStreamIsCapturing(st, &cap));
    const bool pair = units && cap == hipStreamCaptureStatusNone && 2 * (int64_t)m->batch <= device_cu_count();
    if (pair) {
        const size_t words = (size_t)m->batch * 2 * 2 * MBW;
        if (words > g_kvp.words || g_kvp.dev != dev) {
            if (g_kvp.mb) EVK_HIP(hipFree(g_kvp.mb));
            g_kvp = KvPairWs{};
            EVK_HIP(hipMalloc(&g_kvp.mb, words * sizeof(uint64_t)));
            EVK_HIP(hipMemsetAsync(g_kvp.mb, 0, words * sizeof(uint64_t), st));
            g_kvp.words = words;
            g_kvp.dev = dev;
        }
        if (++g_kvp.launch >= (1u << 24)) {  // tags would wrap: start over from clean mailboxes
            EVK_HIP(hipMemsetAsync(g_kvp.mb, 0, g_kvp.words * sizeof(uint64_t), st));
            g_kvp.launch = 1;
        }
        KvPairArgs pa{};
        pa.a = a;
        pa.mb = g_kvp.mb;
        pa.launch = g_kvp.launch;
        // a hand-over takes a few polls; a wait that gives up marks the status
        pa.spin = (int)std::min(flash_spin_limit(), 1u << 15);
        const int plds = kv_pair_lds_floats(*m) * (int)sizeof(float);
        hipLaunchKernelGGL(kv_step256x2, dim3(2 * m->batch), dim3(KT), (unsigned)plds, st, pa);
    } else {
        hipLaunchKernelGGL(units ? kv_step256 : kv_step, dim3(m->batch), dim3(KT), (unsigned)lds, st, a);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "kv_decode_step launch");
}
