// Training-path ops of evk::ai on gfx950: the reference's non-inference
// compute shaders (scale, relu(_bwd), gelu_bwd, sgd, adam, softmax(_bwd),
// rms_norm_bwd, mse_loss, cross_entropy(+count, +scale), sum_batch,
// causal_mask, position_add(_bwd), rope_bwd, embed_bwd).
//
// Design:
//   - Elementwise ops: a thread owns 8 consecutive elements and moves them
//     with 16-byte accesses when the 8 are whole and the caller's pointers
//     are 16-byte aligned (checked on the host), per element otherwise.
//   - Row ops (softmax, softmax backward, rms_norm backward): one wave per
//     row, 4 rows per 256-thread workgroup; a lane strides the row.
//   - Reductions run in a fixed order (per-lane partials, then a tree), so
//     results do not depend on scheduling; the reference's float atomics in
//     cross_entropy.comp are replaced by per-row losses summed in row order.
//   - Each op rounds to fp16 where its shader does (every stored value).
#include "common.h"
#include "kernels.h"

#include <math.h>

namespace evkhip {

// e^x as 2^(x log2 e) on v_exp_f32: the row maximum is subtracted inside one
// FMA, exp(a - m) = 2^(a log2e - m log2e)
constexpr float kLog2eT = 1.4426950408889634f;
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

namespace {

constexpr int EW_NT = 256;  // threads of an elementwise workgroup

DEV float hf(f16 x) { return (float)x; }

// 8 consecutive fp16 values at p[i0..i0+8) (fewer at the tail) as floats
// Streaming accesses: nontemporal loads and stores for data that a kernel
// reads or writes once (elementwise ops, Adam: 65 -> 77 % of HBM; the
// cross-entropy rows: 66 -> 71 %; the register softmax measured slower)
DEV half8 ld_stream(const half8* p) {
    return __builtin_bit_cast(half8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}
DEV void st_stream(half8* p, const half8& v) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}
DEV void ld8(const f16* p, int64_t i0, int64_t n, bool vec, float (&v)[8]) {
    if (vec && i0 + 8 <= n) {
        const half8 h = ld_stream(reinterpret_cast<const half8*>(p + i0));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = i0 + e < n ? hf(p[i0 + e]) : 0.0f;
    }
}
DEV void st8(f16* p, int64_t i0, int64_t n, bool vec, const float (&v)[8]) {
    if (vec && i0 + 8 <= n) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (f16)v[e];
        st_stream(reinterpret_cast<half8*>(p + i0), h);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (i0 + e < n) p[i0 + e] = (f16)v[e];
    }
}
DEV int64_t first8() { return ((int64_t)blockIdx.x * EW_NT + threadIdx.x) * 8; }

// Fill of `n` 16-bit words with a repeated 32-bit pattern: word i takes the
// pattern's low half for even i and its high half for odd i.  A kernel, not
// hipMemsetAsync, so that a captured HIP graph holds no memset node.
__global__ __launch_bounds__(EW_NT) void fill_k(uint16_t* p, uint32_t pattern, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    if (vec && i0 + 8 <= n) {
        *reinterpret_cast<u32x4*>(p + i0) = u32x4{pattern, pattern, pattern, pattern};
    } else {
        for (int64_t i = i0; i < n && i < i0 + 8; ++i) p[i] = (uint16_t)((i & 1) ? pattern >> 16 : pattern);
    }
}

// scale.comp: x = fp16(x * s)
__global__ __launch_bounds__(EW_NT) void scale_k(f16* x, float s, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float v[8];
    ld8(x, i0, n, vec, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= s;
    st8(x, i0, n, vec, v);
}

// relu.comp: out = fp16(max(0, in))
__global__ __launch_bounds__(EW_NT) void relu_k(const f16* in, f16* out, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float v[8];
    ld8(in, i0, n, vec, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = fmaxf(v[e], 0.0f);
    st8(out, i0, n, vec, v);
}

// relu_bwd.comp: grad_in = fp16(grad_in + (in > 0 ? grad_out : 0))
__global__ __launch_bounds__(EW_NT) void relu_bwd_k(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float g[8], x[8], a[8];
    ld8(gout, i0, n, vec, g);
    ld8(in, i0, n, vec, x);
    ld8(gin, i0, n, vec, a);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] += x[e] > 0.0f ? g[e] : 0.0f;
    st8(gin, i0, n, vec, a);
}

// d/dx of the tanh GELU (gelu_bwd.comp): 0.5 (1 + t) + 0.5 x (1 - t^2) du/dx
DEV float gelu_grad(float x) {
    const float ka = 0.7978845608028654f, kb = 0.044715f;
    const float x2 = x * x;
    const float t = tanhf(ka * (x + kb * x2 * x));
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * (ka * (1.0f + 3.0f * kb * x2));
}

// gelu_bwd.comp: grad_in = fp16(grad_in + grad_out * gelu'(in))
__global__ __launch_bounds__(EW_NT) void gelu_bwd_k(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float g[8], x[8], a[8];
    ld8(gout, i0, n, vec, g);
    ld8(in, i0, n, vec, x);
    ld8(gin, i0, n, vec, a);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] += g[e] * gelu_grad(x[e]);
    st8(gin, i0, n, vec, a);
}

// sgd.comp: param = fp16(param - lr * grad)
__global__ __launch_bounds__(EW_NT) void sgd_k(f16* param, const f16* grad, float lr, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float p[8], g[8];
    ld8(param, i0, n, vec, p);
    ld8(grad, i0, n, vec, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] -= lr * g[e];
    st8(param, i0, n, vec, p);
}

// adam.comp, per element: the state is fp16 m / rms (m_norm) and
// log2(rms) + 41 (0 means rms = 0); moments in fp32; a non-finite gradient
// leaves everything unchanged; non-finite results are not stored.
struct AdamArgs {
    f16* param;
    const f16* grad;
    f16* m;
    f16* v;
    float lr, beta1, beta2, c1inv, c2inv, eps;
};
// one element; returns false when the gradient is not finite (nothing changes)
DEV void adam_one(const AdamArgs& a, float g, float& p, float& mq, float& vq) {
    const float kOffset = 41.0f, kMinRms = 1.0e-12f;
    if (!isfinite(g)) return;
    // hardware exp2 / log2 / sqrt / reciprocal (about 1 ulp in fp32): the
    // state and the parameter are stored in fp16, far coarser than that
    float rms = vq > 0.0f ? __builtin_amdgcn_exp2f(vq - kOffset) : 0.0f;
    float m = mq * rms;
    float v = rms * rms;
    m = a.beta1 * m + (1.0f - a.beta1) * g;
    v = a.beta2 * v + (1.0f - a.beta2) * g * g;
    rms = __builtin_amdgcn_sqrtf(fmaxf(v, 0.0f));
    const float m_norm = m * __builtin_amdgcn_rcpf(fmaxf(rms, 1.0e-8f));
    if (isfinite(m_norm)) mq = m_norm;
    const float log_rms = __builtin_amdgcn_logf(fmaxf(rms, kMinRms)) + kOffset;
    if (isfinite(log_rms)) vq = log_rms;
    const float upd = a.lr * (m * a.c1inv) * __builtin_amdgcn_rcpf(rms * __builtin_amdgcn_sqrtf(a.c2inv) + a.eps);
    if (isfinite(upd)) p = fminf(fmaxf(p - upd, -65504.0f), 65504.0f);
}
// 8 elements per thread; a value that is not updated is stored back as it
// was read (its fp16 bits round-trip exactly)
__global__ __launch_bounds__(EW_NT) void adam_k(AdamArgs a, int64_t n, bool vec) {
    const int64_t i0 = first8();
    if (i0 >= n) return;
    float p[8], g[8], m[8], v[8];
    ld8(a.param, i0, n, vec, p);
    ld8(a.grad, i0, n, vec, g);
    ld8(a.m, i0, n, vec, m);
    ld8(a.v, i0, n, vec, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) adam_one(a, g[e], p[e], m[e], v[e]);
    st8(a.param, i0, n, vec, p);
    st8(a.m, i0, n, vec, m);
    st8(a.v, i0, n, vec, v);
}

// position_add.comp: out[b, t, d] = fp16(in[b, t, d] + pos[t, d])
__global__ __launch_bounds__(EW_NT) void position_add_k(const f16* in, const f16* pos, f16* out, int64_t n,
                                                        int64_t per_batch) {
    const int64_t i = (int64_t)blockIdx.x * EW_NT + threadIdx.x;
    if (i >= n) return;
    out[i] = (f16)(hf(in[i]) + hf(pos[i % per_batch]));
}

// position_add_bwd.comp mode 1: grad_pos[j] = fp16(grad_pos[j] + sum_b grad_out[b, j]),
// the batches added in order after the existing value
__global__ __launch_bounds__(EW_NT) void position_pos_bwd_k(const f16* gout, f16* gpos, int64_t per_batch,
                                                            int batch) {
    const int64_t j = (int64_t)blockIdx.x * EW_NT + threadIdx.x;
    if (j >= per_batch) return;
    float s = hf(gpos[j]);
    for (int b = 0; b < batch; ++b) s += hf(gout[(int64_t)b * per_batch + j]);
    gpos[j] = (f16)s;
}

// sum_batch.comp: out[i] = fp16(out[i] + sum_b in[b, i]), same order
__global__ __launch_bounds__(EW_NT) void sum_batch_k(const f16* in, f16* out, int64_t per_batch, int batch) {
    const int64_t i = (int64_t)blockIdx.x * EW_NT + threadIdx.x;
    if (i >= per_batch) return;
    float s = hf(out[i]);
    for (int b = 0; b < batch; ++b) s += hf(in[(int64_t)b * per_batch + i]);
    out[i] = (f16)s;
}

// rope_bwd.comp: the transposed rotation of rope.comp added to grad_in,
// pair p of position t at angle t * base^(-2p / E)
__global__ __launch_bounds__(EW_NT) void rope_bwd_k(const f16* gout, f16* gin, int64_t pairs, int S, int E,
                                                    float base) {
    const int64_t gid = (int64_t)blockIdx.x * EW_NT + threadIdx.x;
    if (gid >= pairs) return;
    const int P = E / 2;
    const int p = (int)(gid % P);
    const int64_t bt = gid / P;
    const int t = (int)(bt % S);
    const int64_t i = bt * E + 2 * p;
    const float g0 = hf(gout[i]), g1 = hf(gout[i + 1]);
    const float inv_freq = powf(base, -2.0f * (float)p / (float)E);
    float sn, cs;
    sincosf((float)t * inv_freq, &sn, &cs);
    gin[i] = (f16)(hf(gin[i]) + (g0 * cs + g1 * sn));
    gin[i + 1] = (f16)(hf(gin[i + 1]) + (-g0 * sn + g1 * cs));
}

// causal_mask.comp: scores[b, i, j] = -65504 where j > i
__global__ __launch_bounds__(EW_NT) void causal_mask_k(f16* scores, int64_t n, int N) {
    const int64_t gid = (int64_t)blockIdx.x * EW_NT + threadIdx.x;
    if (gid >= n) return;
    const int j = (int)(gid % N), i = (int)((gid / N) % N);
    if (j > i) scores[gid] = (f16)(-65504.0f);
}

// embed_bwd.comp: grad_emb[tok] += grad_out[idx] for idx in order.  A thread
// owns one embedding dimension and walks the indices in order, so every
// (token, dim) accumulates in the reference's sequence of fp16 roundings;
// ids >= vocab are skipped (the shader would write past the table).
__global__ __launch_bounds__(EW_NT) void embed_bwd_k(const f16* gout, const uint16_t* idx, f16* gemb, int64_t n_idx,
                                                     int dim, int vocab) {
    const int d = blockIdx.x * EW_NT + threadIdx.x;
    if (d >= dim) return;
    for (int64_t r = 0; r < n_idx; ++r) {
        const int tok = idx[r];
        if (tok >= vocab) continue;
        f16* dst = gemb + (int64_t)tok * dim + d;
        *dst = (f16)(hf(*dst) + hf(gout[r * dim + d]));
    }
}

// ---- row ops: one wave per row, 4 rows per workgroup ----
constexpr int ROWS_PER_WG = EW_NT / 64;

// softmax.comp: entries <= -65504 are masked (probability 0); the others
// are exp(x * scale - max) / sum, normalised from the input so that each
// output is rounded once
__global__ __launch_bounds__(EW_NT) void softmax_k(const f16* in, f16* out, float scale, int D, int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const f16* x = in + row * D;
    f16* y = out + row * D;
    const float kMask = -65504.0f;
    float mx = -3.402823466e+38f;
    for (int j = lane; j < D; j += 64) {
        const float r = hf(x[j]);
        if (r > kMask) mx = fmaxf(mx, r * scale);
    }
    mx = wave_max(mx);
    const float sl2 = scale * kLog2eT, nm2 = -mx * kLog2eT;
    float sum = 0.0f;
    for (int j = lane; j < D; j += 64) {
        const float r = hf(x[j]);
        if (r > kMask) sum += exp2_fast(__builtin_fmaf(r, sl2, nm2));
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / fmaxf(sum, 1e-20f);
    for (int j = lane; j < D; j += 64) {
        const float r = hf(x[j]);
        y[j] = (f16)(r > kMask ? exp2_fast(__builtin_fmaf(r, sl2, nm2)) * inv : 0.0f);
    }
}

// softmax.comp with rows in registers: D % 8 == 0, 16-byte aligned rows,
// D <= 64 * 8 * NV.  A wave takes RPW rows and requests all of them before
// any arithmetic; each exponential is formed once.  One HBM read and one
// write per element.
template <int NV, int RPW>
__global__ __launch_bounds__(EW_NT) void softmax_reg_k(const f16* in, f16* out, float scale, int D, int64_t rows) {
    const int64_t row0 = ((int64_t)blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6)) * RPW;
    const int lane = threadIdx.x & 63;
    if (row0 >= rows) return;
    const int nc = D / 8;  // 16-byte chunks of a row
    const float kMask = -65504.0f;
    half8 r[RPW][NV];
#pragma unroll
    for (int k = 0; k < RPW; ++k)
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int c = lane + 64 * u;
            if (row0 + k < rows && c < nc) r[k][u] = reinterpret_cast<const half8*>(in + (row0 + k) * D)[c];
        }
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        if (row0 + k >= rows) break;
        float mx = -3.402823466e+38f;
#pragma unroll
        for (int u = 0; u < NV; ++u)
            if (lane + 64 * u < nc)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = (float)r[k][u][e];
                    if (v > kMask) mx = fmaxf(mx, v * scale);
                }
        mx = wave_max(mx);
        const float sl2 = scale * kLog2eT, nm2 = -mx * kLog2eT;
        float ex[NV][8];
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < NV; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = (float)r[k][u][e];
                ex[u][e] = (lane + 64 * u < nc && v > kMask) ? exp2_fast(__builtin_fmaf(v, sl2, nm2)) : 0.0f;
                sum += ex[u][e];
            }
        sum = wave_sum(sum);
        const float inv = 1.0f / fmaxf(sum, 1e-20f);
        half8* y = reinterpret_cast<half8*>(out + (row0 + k) * D);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int c = lane + 64 * u;
            if (c >= nc) continue;
            half8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (f16)(ex[u][e] * inv);
            y[c] = o;
        }
    }
}

// softmax_bwd.comp: grad_in = fp16(grad_in + p (g - sum_j g_j p_j) scale)
__global__ __launch_bounds__(EW_NT) void softmax_bwd_k(const f16* probs, const f16* gout, f16* gin, float scale, int D,
                                                       int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const f16* p = probs + row * D;
    const f16* g = gout + row * D;
    f16* o = gin + row * D;
    float dot = 0.0f;
    for (int j = lane; j < D; j += 64) dot += hf(p[j]) * hf(g[j]);
    dot = wave_sum(dot);
    for (int j = lane; j < D; j += 64) o[j] = (f16)(hf(o[j]) + hf(p[j]) * (hf(g[j]) - dot) * scale);
}

// rms_norm_bwd.comp: with y = x / rms, rms = sqrt(mean(x^2) + eps) over the
// row (x clamped to the fp16 range), grad_in += g / rms - x (g . y) / (D rms^2)
__global__ __launch_bounds__(EW_NT) void rms_norm_bwd_k(const f16* in, const f16* gout, f16* gin, float eps, int D,
                                                        int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const f16* x = in + row * D;
    const f16* g = gout + row * D;
    f16* o = gin + row * D;
    auto clampx = [](float v) { return fminf(fmaxf(v, -65504.0f), 65504.0f); };
    float ss = 0.0f;
    for (int j = lane; j < D; j += 64) {
        const float v = clampx(hf(x[j]));
        ss += v * v;
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float dot = 0.0f;
    for (int j = lane; j < D; j += 64) dot += hf(g[j]) * (clampx(hf(x[j])) * inv);
    dot = wave_sum(dot);
    const float sc = dot / (float)D;
    for (int j = lane; j < D; j += 64) {
        const float v = clampx(hf(x[j]));
        o[j] = (f16)(hf(o[j]) + (hf(g[j]) * inv - v * inv * inv * sc));
    }
}

// ---- reductions ----
constexpr int RED_NT = 1024;

// sum of one value per thread over a workgroup of RED_NT threads, in a fixed
// order; every thread gets the total
DEV float block_sum(float v, float* sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < RED_NT / 64; ++w) t += sh[w];
    __syncthreads();
    return t;
}

// mse_loss.comp: grad = fp16(2 (p - t) / n); result = fp16(sum (p - t)^2 / n).
// One workgroup; lane-strided partial sums, then a fixed tree.
__global__ __launch_bounds__(RED_NT) void mse_loss_k(const f16* pred, const f16* tgt, f16* grad, f16* result,
                                                     int64_t n) {
    __shared__ float sh[RED_NT / 64];
    const float gs = 2.0f / (float)n;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += RED_NT) {
        const float diff = hf(pred[i]) - hf(tgt[i]);
        s += diff * diff;
        grad[i] = (f16)(gs * diff);
    }
    s = block_sum(s, sh);
    if (threadIdx.x == 0) result[0] = (f16)(s / (float)n);
}

// cross_entropy_count.comp: number of valid targets (t != 0, t < V) into ws[0]
__global__ __launch_bounds__(RED_NT) void ce_count_k(const uint16_t* tgt, float* ws, int64_t rows, int V) {
    __shared__ float sh[RED_NT / 64];
    float c = 0.0f;
    for (int64_t r = threadIdx.x; r < rows; r += RED_NT) {
        const int t = tgt[r];
        c += (t != 0 && t < V) ? 1.0f : 0.0f;
    }
    c = block_sum(c, sh);
    if (threadIdx.x == 0) ws[0] = c;
}

// cross_entropy.comp, one workgroup per row: logits clamped to +-65000;
// grad = softmax / n_valid, minus 1 / n_valid at the target; the row's loss
// (lse - logit[target]) / n_valid goes to ws[1 + row].  Ignored rows (target
// 0 or >= V) get zero gradients and zero loss.
constexpr int CE_NT = 256;
__global__ __launch_bounds__(CE_NT) void ce_row_k(const f16* logits, const uint16_t* tgt, f16* grad, float* ws, int V) {
    __shared__ float sh[2 * (CE_NT / 64)];
    const int64_t row = blockIdx.x;
    const f16* x = logits + row * V;
    f16* g = grad + row * V;
    const int t = tgt[row];
    const float n_valid = ws[0];
    const bool valid = t != 0 && t < V && n_valid > 0.0f;
    if (!valid) {
        for (int j = threadIdx.x; j < V; j += CE_NT) g[j] = (f16)0.0f;
        if (threadIdx.x == 0) ws[1 + row] = 0.0f;
        return;
    }
    const float inv_valid = 1.0f / n_valid;
    auto lv = [&](int j) { return fminf(fmaxf(hf(x[j]), -65000.0f), 65000.0f); };
    float mx = -3.402823466e+38f;
    for (int j = threadIdx.x; j < V; j += CE_NT) mx = fmaxf(mx, lv(j));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = sh[0];
#pragma unroll
    for (int w = 1; w < CE_NT / 64; ++w) mx = fmaxf(mx, sh[w]);
    const float nm2 = -mx * kLog2eT;
    float sum = 0.0f;
    for (int j = threadIdx.x; j < V; j += CE_NT) sum += exp2_fast(__builtin_fmaf(lv(j), kLog2eT, nm2));
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) sh[CE_NT / 64 + (threadIdx.x >> 6)] = sum;
    __syncthreads();
    sum = 0.0f;
#pragma unroll
    for (int w = 0; w < CE_NT / 64; ++w) sum += sh[CE_NT / 64 + w];
    sum = fmaxf(sum, 1e-20f);
    const float inv_sum = 1.0f / sum, log_sum = logf(sum);
    const float scale_g = inv_sum * inv_valid;
    for (int j = threadIdx.x; j < V; j += CE_NT) {
        float gv = exp2_fast(__builtin_fmaf(lv(j), kLog2eT, nm2)) * scale_g;
        if (j == t) gv -= inv_valid;
        g[j] = (f16)gv;
    }
    if (threadIdx.x == 0) ws[1 + row] = ((mx + log_sum) - lv(t)) * inv_valid;
}

// ce_row_k with the row in registers: V % 8 == 0, 16-byte aligned rows,
// V <= NT * 8 * NV; one HBM read and one write per logit
template <int NV, int NT>
__global__ __launch_bounds__(NT) void ce_row_reg_k(const f16* logits, const uint16_t* tgt, f16* grad, float* ws,
                                                   int V) {
    constexpr int CE_NT = NT;
    __shared__ float sh[2 * (CE_NT / 64)];
    const int64_t row = blockIdx.x;
    const half8* x = reinterpret_cast<const half8*>(logits + row * V);
    half8* g = reinterpret_cast<half8*>(grad + row * V);
    const int nc = V / 8;
    const int t = tgt[row];
    const float n_valid = ws[0];
    const bool valid = t != 0 && t < V && n_valid > 0.0f;
    if (!valid) {
        const half8 z = {};
        for (int c = threadIdx.x; c < nc; c += CE_NT) g[c] = z;
        if (threadIdx.x == 0) ws[1 + row] = 0.0f;
        return;
    }
    half8 r[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int c = threadIdx.x + CE_NT * u;
        if (c < nc) r[u] = ld_stream(x + c);
    }
    auto cl = [](f16 h) { return fminf(fmaxf((float)h, -65000.0f), 65000.0f); };
    float mx = -3.402823466e+38f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
        if (threadIdx.x + CE_NT * u < nc)
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, cl(r[u][e]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = sh[0];
#pragma unroll
    for (int w = 1; w < CE_NT / 64; ++w) mx = fmaxf(mx, sh[w]);
    const float nm2 = -mx * kLog2eT;
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
        if (threadIdx.x + CE_NT * u < nc)
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += exp2_fast(__builtin_fmaf(cl(r[u][e]), kLog2eT, nm2));
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) sh[CE_NT / 64 + (threadIdx.x >> 6)] = sum;
    __syncthreads();
    sum = 0.0f;
#pragma unroll
    for (int w = 0; w < CE_NT / 64; ++w) sum += sh[CE_NT / 64 + w];
    sum = fmaxf(sum, 1e-20f);
    const float inv_valid = 1.0f / n_valid;
    const float inv_sum = 1.0f / sum, log_sum = logf(sum);
    const float scale_g = inv_sum * inv_valid;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int c = threadIdx.x + CE_NT * u;
        if (c >= nc) continue;
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (f16)(exp2_fast(__builtin_fmaf(cl(r[u][e]), kLog2eT, nm2)) * scale_g);
        if (c == (t >> 3)) {  // the target's chunk: its gradient and the row loss
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e == (t & 7)) {
                    const float xv = cl(r[u][e]);
                    o[e] = (f16)(exp2_fast(__builtin_fmaf(xv, kLog2eT, nm2)) * scale_g - inv_valid);
                    ws[1 + row] = ((mx + log_sum) - xv) * inv_valid;
                }
        }
        st_stream(g + c, o);
    }
}

// cross_entropy_scale.comp: the mean loss (0 when nothing is valid or the
// sum is not finite), summed over rows in a fixed order
__global__ __launch_bounds__(RED_NT) void ce_final_k(const float* ws, f16* result, int64_t rows) {
    __shared__ float sh[RED_NT / 64];
    float s = 0.0f;
    for (int64_t r = threadIdx.x; r < rows; r += RED_NT) s += ws[1 + r];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) {
        float loss = (ws != nullptr && ws[0] > 0.0f) ? s : 0.0f;
        if (!isfinite(loss)) loss = 0.0f;
        result[0] = (f16)loss;
    }
}

// cross-entropy workspace (grow-only): [n_valid | loss of each row]
float* g_ce_ws = nullptr;
size_t g_ce_ws_n = 0;

int launched(const char* what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, what);
}
unsigned ew_grid8(int64_t n) { return (unsigned)((n + 8LL * EW_NT - 1) / (8LL * EW_NT)); }
unsigned ew_grid(int64_t n) { return (unsigned)((n + EW_NT - 1) / EW_NT); }
unsigned row_grid(int64_t rows) { return (unsigned)((rows + ROWS_PER_WG - 1) / ROWS_PER_WG); }

}  // namespace

void train_ops_free_workspace() {
    if (g_ce_ws) (void)hipFree(g_ce_ws);
    g_ce_ws = nullptr;
    g_ce_ws_n = 0;
}

int fill_launch(void* p, uint32_t pattern, int64_t n16, bool vec, hipStream_t st) {
    if (n16 == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(fill_k, dim3(ew_grid8(n16)), dim3(EW_NT), 0, st, static_cast<uint16_t*>(p), pattern, n16,
                       vec);
    return launched("fill launch");
}

int scale_launch(f16* x, float s, int64_t n, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(scale_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, x, s, n, vec);
    return launched("scale launch");
}
int relu_launch(const f16* in, f16* out, int64_t n, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(relu_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, in, out, n, vec);
    return launched("relu launch");
}
int relu_bwd_launch(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(relu_bwd_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, gout, in, gin, n, vec);
    return launched("relu_backward launch");
}
int gelu_bwd_launch(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(gelu_bwd_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, gout, in, gin, n, vec);
    return launched("gelu_backward launch");
}
int sgd_launch(f16* param, const f16* grad, float lr, int64_t n, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(sgd_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, param, grad, lr, n, vec);
    return launched("sgd launch");
}
int adam_launch(f16* param, const f16* grad, f16* m, f16* v, int64_t n, float lr, float beta1, float beta2,
                float c1inv, float c2inv, float eps, bool vec, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    AdamArgs a{param, grad, m, v, lr, beta1, beta2, c1inv, c2inv, eps};
    hipLaunchKernelGGL(adam_k, dim3(ew_grid8(n)), dim3(EW_NT), 0, st, a, n, vec);
    return launched("adam launch");
}
int softmax_launch(const f16* in, f16* out, float scale, int D, int64_t rows, bool vec, hipStream_t st) {
    if (rows == 0 || D == 0) return EVKHIP_OK;
    if (vec && D % 8 == 0 && D <= 64 * 8 * 4) {
        const unsigned g2 = (unsigned)((rows + 2 * ROWS_PER_WG - 1) / (2 * ROWS_PER_WG));
        if (D <= 64 * 8)
            hipLaunchKernelGGL((softmax_reg_k<1, 2>), dim3(g2), dim3(EW_NT), 0, st, in, out, scale, D, rows);
        else if (D <= 64 * 8 * 2)
            hipLaunchKernelGGL((softmax_reg_k<2, 2>), dim3(g2), dim3(EW_NT), 0, st, in, out, scale, D, rows);
        else
            hipLaunchKernelGGL((softmax_reg_k<4, 1>), dim3(row_grid(rows)), dim3(EW_NT), 0, st, in, out, scale, D,
                               rows);
        return launched("softmax launch");
    }
    hipLaunchKernelGGL(softmax_k, dim3(row_grid(rows)), dim3(EW_NT), 0, st, in, out, scale, D, rows);
    return launched("softmax launch");
}
int softmax_bwd_launch(const f16* probs, const f16* gout, f16* gin, float scale, int D, int64_t rows,
                       hipStream_t st) {
    if (rows == 0 || D == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(softmax_bwd_k, dim3(row_grid(rows)), dim3(EW_NT), 0, st, probs, gout, gin, scale, D, rows);
    return launched("softmax_backward launch");
}
int rms_norm_bwd_launch(const f16* in, const f16* gout, f16* gin, float eps, int D, int64_t rows, hipStream_t st) {
    if (rows == 0 || D == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(rms_norm_bwd_k, dim3(row_grid(rows)), dim3(EW_NT), 0, st, in, gout, gin, eps, D, rows);
    return launched("rms_norm_backward launch");
}
int mse_loss_launch(const f16* pred, const f16* tgt, f16* grad, f16* result, int64_t n, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(mse_loss_k, dim3(1), dim3(RED_NT), 0, st, pred, tgt, grad, result, n);
    return launched("mse_loss launch");
}
int cross_entropy_launch(const f16* logits, const uint16_t* tgt, f16* grad, f16* result, int64_t rows, int V,
                         bool vec, hipStream_t st) {
    if (rows == 0) {  // nothing valid: loss 0
        hipLaunchKernelGGL(ce_final_k, dim3(1), dim3(RED_NT), 0, st, (const float*)nullptr, result, (int64_t)0);
        return launched("cross_entropy launch");
    }
    const size_t need = (size_t)rows + 1;
    if (need > g_ce_ws_n) {
        if (g_ce_ws) EVK_HIP(hipFree(g_ce_ws));
        g_ce_ws = nullptr;
        g_ce_ws_n = 0;
        EVK_HIP(hipMalloc(&g_ce_ws, need * sizeof(float)));
        g_ce_ws_n = need;
    }
    hipLaunchKernelGGL(ce_count_k, dim3(1), dim3(RED_NT), 0, st, tgt, g_ce_ws, rows, V);
    if (vec && V % 8 == 0 && V <= 512 * 8 * 8) {
        if (V <= CE_NT * 8 * 4)
            hipLaunchKernelGGL((ce_row_reg_k<4, CE_NT>), dim3((unsigned)rows), dim3(CE_NT), 0, st, logits, tgt, grad,
                               g_ce_ws, V);
        else
            hipLaunchKernelGGL((ce_row_reg_k<8, 512>), dim3((unsigned)rows), dim3(512), 0, st, logits, tgt, grad,
                               g_ce_ws, V);
    } else {
        hipLaunchKernelGGL(ce_row_k, dim3((unsigned)rows), dim3(CE_NT), 0, st, logits, tgt, grad, g_ce_ws, V);
    }
    hipLaunchKernelGGL(ce_final_k, dim3(1), dim3(RED_NT), 0, st, (const float*)g_ce_ws, result, rows);
    return launched("cross_entropy launch");
}
int sum_batch_launch(const f16* in, f16* out, int batch, int64_t per_batch, hipStream_t st) {
    if (per_batch == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(sum_batch_k, dim3(ew_grid(per_batch)), dim3(EW_NT), 0, st, in, out, per_batch, batch);
    return launched("sum_batch launch");
}
int causal_mask_launch(f16* scores, int64_t batch, int N, hipStream_t st) {
    const int64_t n = batch * N * N;
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(causal_mask_k, dim3(ew_grid(n)), dim3(EW_NT), 0, st, scores, n, N);
    return launched("causal_mask launch");
}
int position_add_launch(const f16* in, const f16* pos, f16* out, int B, int64_t per_batch, hipStream_t st) {
    const int64_t n = (int64_t)B * per_batch;
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(position_add_k, dim3(ew_grid(n)), dim3(EW_NT), 0, st, in, pos, out, n, per_batch);
    return launched("position_add launch");
}
int position_add_bwd_launch(const f16* gout, f16* gin, f16* gpos, int B, int64_t per_batch, hipStream_t st) {
    const int64_t n = (int64_t)B * per_batch;
    if (n == 0) return EVKHIP_OK;
    // grad_in += grad_out (the add of two tensors), then grad_pos
    int e = add_launch(gin, gout, gin, n, st);
    if (e != EVKHIP_OK) return e;
    hipLaunchKernelGGL(position_pos_bwd_k, dim3(ew_grid(per_batch)), dim3(EW_NT), 0, st, gout, gpos, per_batch, B);
    return launched("position_add_backward launch");
}
int rope_bwd_launch(const f16* gout, f16* gin, int B, int S, int E, float base, hipStream_t st) {
    const int64_t pairs = (int64_t)B * S * (E / 2);
    if (pairs == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(rope_bwd_k, dim3(ew_grid(pairs)), dim3(EW_NT), 0, st, gout, gin, pairs, S, E, base);
    return launched("rope_backward launch");
}
int embed_bwd_launch(const f16* gout, const uint16_t* idx, f16* gemb, int64_t n_idx, int dim, int vocab,
                     hipStream_t st) {
    if (n_idx == 0 || dim == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(embed_bwd_k, dim3(ew_grid(dim)), dim3(EW_NT), 0, st, gout, idx, gemb, n_idx, dim, vocab);
    return launched("embed_backward launch");
}

}  // namespace evkhip
