// Decode-step kernels: single-query attention (split over the cache with an
// in-kernel merge) and the bandwidth-trivial ops a KV-cached step needs.
// References: shaders/single_query_attention.comp:26-72, rms_norm.comp:21-49,
// rope.comp:18-41, gelu.comp:15-30, add.comp:18-26, embed.comp:18-28,
// greedy_sample.comp:24-64.
#include "kernels.h"

#include <math.h>

#include <algorithm>

namespace evkhip {

namespace {

// ---------------------------------------------------------------------------
// Single-query attention.  Grid (heads, nsplit); 256 threads.  A workgroup
// covers cache rows [split*chunk, +chunk) of one head: LPK = DH/8 lanes per
// key (16 bytes each), 256/LPK keys per pass (DH = 256: 32 lanes, 8 keys).  Partial (m, l, o) go to
// workspace; the last workgroup of a head merges the splits in split order.
// ---------------------------------------------------------------------------
struct SqArgs {
    const f16* q;
    const f16* kc;
    const f16* vc;
    f16* out;
    int64_t row_stride;  // elements between consecutive cache rows
    int64_t cache_bstride;  // elements between the caches of consecutive sequences
    int heads, L, chunk;    // heads per sequence; grid.x = sequences * heads
    float scale_log2;
    float* part;         // [heads][nsplit][2 + DH]
    unsigned* counters;  // [heads]
};

constexpr float kLog2e = 1.4426950408889634f;

template <int DH>
__global__ __launch_bounds__(256) void sq_attention(SqArgs a) {
    constexpr int LPK = DH / 8;             // lanes per key
    constexpr int KPP = 256 / LPK;          // keys per pass
    static_assert(KPP >= 4, "at least one key slot per wave");
    __shared__ float s_m[4], s_w[4];
    __shared__ float s_o[4][DH];
    __shared__ unsigned s_last;
    // h: (sequence, head) pair; q, out and the workspace are indexed by it,
    // the caches by the sequence's cache and the head's columns
    const int h = blockIdx.x, split = blockIdx.y, nsplit = gridDim.y;
    const int seq = h / a.heads, hc = h - seq * a.heads;
    const f16* kc = a.kc + (int64_t)seq * a.cache_bstride + (int64_t)hc * DH;
    const f16* vc = a.vc + (int64_t)seq * a.cache_bstride + (int64_t)hc * DH;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = tid % LPK, kslot = tid / LPK;
    const int j0 = split * a.chunk, j1 = min(a.L, j0 + a.chunk);

    float qv[8];
    {
        half8 qh = *reinterpret_cast<const half8*>(a.q + (int64_t)h * DH + sub * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = (float)qh[e];
    }
    float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;

    for (int jb = j0; jb < j1; jb += KPP) {
        const int j = jb + kslot;
        float s = -INFINITY;
        half8 vh;
        if (j < j1) {
            const f16* kr = kc + (int64_t)j * a.row_stride + sub * 8;
            half8 kh = *reinterpret_cast<const half8*>(kr);
            vh = *reinterpret_cast<const half8*>(vc + (int64_t)j * a.row_stride + sub * 8);
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d += qv[e] * (float)kh[e];
#pragma unroll
            for (int off = LPK / 2; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
            s = d * a.scale_log2;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) vh[e] = (f16)0.0f;
        }
        // online softmax per lane group (all LPK lanes of a key hold the same s)
        float mn = fmaxf(m, s);
        float base = mn == -INFINITY ? 0.0f : mn;
        float al = exp2f(m - base), pe = exp2f(s - base);
        l = l * al + pe;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = o[e] * al + pe * (float)vh[e];
        m = mn;
    }
    // Merge the key slots of the workgroup: within a wave (slots sharing sub)
    // then across waves through LDS.
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
        float mn = fmaxf(m, m2);
        float base = mn == -INFINITY ? 0.0f : mn;
        float a1 = exp2f(m - base), a2 = exp2f(m2 - base);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = o[e] * a1 + __shfl_xor(o[e], off, 64) * a2;
        l = l * a1 + l2 * a2;
        m = mn;
    }
    if (lane < LPK) {
        if (sub == 0) { s_m[wave] = m; s_w[wave] = l; }
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[wave][sub * 8 + e] = o[e];
    }
    __syncthreads();
    float* part = a.part + ((int64_t)h * nsplit + split) * (2 + DH);
    if (tid < DH) {
        float mm = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
        float base = mm == -INFINITY ? 0.0f : mm;
        float ll = 0.0f, oo = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float f = exp2f(s_m[w] - base);
            ll += s_w[w] * f;
            oo += s_o[w][tid] * f;
        }
        if (nsplit == 1) {
            a.out[(int64_t)h * DH + tid] = (f16)(ll > 0.0f ? oo / ll : 0.0f);
        } else {
            part[2 + tid] = oo;
            if (tid == 0) { part[0] = mm; part[1] = ll; }
        }
    }
    if (nsplit == 1) return;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(a.counters + h, 1u);
        s_last = prev == (unsigned)(nsplit - 1);
        if (s_last) a.counters[h] = 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (tid < DH) {
        const float* ph = a.part + (int64_t)h * nsplit * (2 + DH);
        float mm = -INFINITY;
        for (int sp = 0; sp < nsplit; ++sp)
            mm = fmaxf(mm, __hip_atomic_load(ph + sp * (2 + DH), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        float base = mm == -INFINITY ? 0.0f : mm;
        float ll = 0.0f, oo = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp) {
            const float* q = ph + sp * (2 + DH);
            float f = exp2f(__hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - base);
            ll += __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * f;
            oo += __hip_atomic_load(q + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * f;
        }
        a.out[(int64_t)h * DH + tid] = (f16)(ll > 0.0f ? oo / ll : 0.0f);
    }
}

// Any head size: one workgroup per head, the shader's algorithm with the
// softmax and the P.V product spread over the workgroup.
__global__ __launch_bounds__(256) void sq_attention_scalar(SqArgs a, int dh) {
    extern __shared__ float sh[];  // scores[L] then q[dh]
    float* sc = sh;
    float* qs = sh + a.L;
    __shared__ float s_red[256];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int seq = h / a.heads, hc = h - seq * a.heads;
    const f16* kc = a.kc + (int64_t)seq * a.cache_bstride + (int64_t)hc * dh;
    const f16* vc = a.vc + (int64_t)seq * a.cache_bstride + (int64_t)hc * dh;
    for (int d = tid; d < dh; d += 256) qs[d] = (float)a.q[(int64_t)h * dh + d];
    __syncthreads();
    const float inv = a.scale_log2;
    float mx = -INFINITY;
    for (int j = tid; j < a.L; j += 256) {
        const f16* kr = kc + (int64_t)j * a.row_stride;
        float s = 0.0f;
        for (int d = 0; d < dh; ++d) s += qs[d] * (float)kr[d];
        sc[j] = s * inv;
        mx = fmaxf(mx, sc[j]);
    }
    s_red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s_red[tid] = fmaxf(s_red[tid], s_red[tid + o]);
        __syncthreads();
    }
    mx = s_red[0];
    __syncthreads();
    float sum = 0.0f;
    for (int j = tid; j < a.L; j += 256) {
        sc[j] = exp2f(sc[j] - mx);
        sum += sc[j];
    }
    s_red[tid] = sum;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s_red[tid] += s_red[tid + o];
        __syncthreads();
    }
    const float is = s_red[0] > 0.0f ? 1.0f / s_red[0] : 0.0f;
    for (int d = tid; d < dh; d += 256) {
        float acc = 0.0f;
        for (int j = 0; j < a.L; ++j) acc += sc[j] * (float)vc[(int64_t)j * a.row_stride + d];
        a.out[(int64_t)h * dh + d] = (f16)(acc * is);
    }
}

// ---------------------------------------------------------------------------
// KV-cache append: rows [pos0, pos0 + n) of each sequence's cache (max_seq, D)
// take the rows of src (batch, n, D).  One thread per 8 values (16 bytes)
// when D % 8 == 0 and both buffers are 16-byte aligned, else per value.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kv_write_k(const f16* src, f16* cache, int64_t total, int n, int D,
                                                  int max_seq, int pos0, int vec) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int W = vec ? 8 : 1;
    const int64_t e0 = i * W;  // element index in src
    if (e0 >= total) return;
    const int64_t row = e0 / D, col = e0 % D;
    const int64_t b = row / n, r = row % n;
    f16* dst = cache + (b * max_seq + pos0 + r) * D + col;
    if (vec) *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src + e0);
    else *dst = src[e0];
}

// ---------------------------------------------------------------------------
// rms_norm: one wave per row, 4 rows per workgroup.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_k(const f16* in, f16* out, int64_t rows, int D, float eps) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const f16* x = in + row * D;
    float ss = 0.0f;
    for (int j = lane; j < D; j += 64) {
        float v = fminf(fmaxf((float)x[j], -65504.0f), 65504.0f);
        ss += v * v;
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    for (int j = lane; j < D; j += 64) {
        float v = fminf(fmaxf((float)x[j], -65504.0f), 65504.0f);
        out[row * D + j] = (f16)(v * inv);
    }
}

// rope: one thread per rotated pair.
__global__ __launch_bounds__(256) void rope_k(const f16* in, f16* out, int B, int S, int E, float base,
                                               int pos0, int hd) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int pairs = E / 2;
    if (gid >= (int64_t)B * S * pairs) return;
    const int pr = (int)(gid % pairs);
    const int64_t tmp = gid / pairs;
    const int t = (int)(tmp % S);
    const int64_t idx = tmp * E + 2 * pr;
    const int pp = pr % (hd / 2);
    const float x0 = (float)in[idx], x1 = (float)in[idx + 1];
    const float inv_freq = powf(base, -2.0f * (float)pp / (float)hd);
    const float ang = (float)(pos0 + t) * inv_freq;
    float s, c;
    sincosf(ang, &s, &c);
    out[idx] = (f16)(x0 * c - x1 * s);
    out[idx + 1] = (f16)(x0 * s + x1 * c);
}


__global__ __launch_bounds__(256) void gelu_k(const f16* in, f16* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = (f16)gelu_f((float)in[i]);
}

__global__ __launch_bounds__(256) void add_k(const f16* a, const f16* b, f16* c, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) c[i] = (f16)((float)a[i] + (float)b[i]);
}

__global__ __launch_bounds__(256) void embed_k(const f16* table, const uint16_t* idx, f16* out, int64_t n_idx,
                                                int dim, int vocab) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= n_idx * dim) return;
    const int64_t i = gid / dim;
    const int d = (int)(gid % dim);
    const int tok = min((int)idx[i], vocab - 1);
    out[gid] = table[(int64_t)tok * dim + d];
}

// ---------------------------------------------------------------------------
// greedy_sample.  The shader's winner is the maximum under the total order
// (value desc, bitrev8(j mod 256) asc, j asc) over valid candidates
// (value > -FLT_MAX), j = token - token_base; with no valid candidate it is
// token_base.  Any reduction tree over this order gives the same winner.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void greedy_k(const f16* logits, uint16_t* out, int S, int V, int position,
                                                 int token_base, int token_count) {
    __shared__ float s_v[4];
    __shared__ uint32_t s_r[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const f16* row = logits + ((int64_t)b * S + position) * V + token_base;
    float bv = -3.402823466e+38f;
    uint32_t br = 0u;  // rank of j = 0 (token_base)
    for (int j = tid; j < token_count; j += 256) {
        float v = (float)row[j];
        uint32_t r = greedy_rank((uint32_t)j);
        if (v > -3.402823466e+38f && greedy_better(v, r, bv, br)) { bv = v; br = r; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = __shfl_xor(bv, o, 64);
        uint32_t r2 = __shfl_xor(br, o, 64);
        if (greedy_better(v2, r2, bv, br)) { bv = v2; br = r2; }
    }
    if ((tid & 63) == 0) { s_v[tid >> 6] = bv; s_r[tid >> 6] = br; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (greedy_better(s_v[w], s_r[w], bv, br)) { bv = s_v[w]; br = s_r[w]; }
        // rank -> j: low 16 bits hold j >> 8, high bits bitrev8(j & 255)
        uint32_t lo = __builtin_bitreverse32(br >> 16) >> 24;
        uint32_t j = ((br & 0xFFFFu) << 8) | lo;
        out[b] = (uint16_t)(token_base + j);
    }
}

// Decode-attention workspace (grow-only).
float* g_sq_part = nullptr;
size_t g_sq_part_elems = 0;
unsigned* g_sq_cnt = nullptr;
size_t g_sq_cnt_n = 0;

}  // namespace

void decode_ops_free_workspace() {
    if (g_sq_part) (void)hipFree(g_sq_part);
    if (g_sq_cnt) (void)hipFree(g_sq_cnt);
    g_sq_part = nullptr;
    g_sq_cnt = nullptr;
    g_sq_part_elems = g_sq_cnt_n = 0;
}

int sq_attention_launch(const f16* q, const f16* kc, const f16* vc, f16* out, int64_t row_stride, int heads,
                        int dh, int L, bool vec_ok, hipStream_t st, int batch, int64_t cache_bstride) {
    SqArgs a{};
    a.q = q; a.kc = kc; a.vc = vc; a.out = out;
    a.row_stride = row_stride; a.heads = heads; a.L = L;
    a.cache_bstride = cache_bstride;
    // from here on `heads` counts (sequence, head) pairs: one grid row each
    heads *= batch;
    a.scale_log2 = (1.0f / sqrtf((float)dh)) * kLog2e;
    const bool vec = vec_ok && (dh == 16 || dh == 32 || dh == 64 || dh == 128 || dh == 256) && (row_stride % 8 == 0);
    if (!vec) {
        size_t shm = sizeof(float) * ((size_t)L + dh);
        if (shm > 64 * 1024)
            return set_error(EVKHIP_ERR_UNSUPPORTED, "single_query_attention: head size %d with %d cached rows "
                             "needs the vector path (dh in {16,32,64,128,256})", dh, L);
        hipLaunchKernelGGL(sq_attention_scalar, dim3(heads), dim3(256), shm, st, a, dh);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? EVKHIP_OK : check_hip(e, "sq_attention_scalar launch");
    }
    // split so that each workgroup streams at least 64 rows and the grid has
    // about two workgroups per CU
    const int cus = device_cu_count();
    int nsplit = 1, chunk = std::max(L, 1);
    if (L > 64) {
        nsplit = std::max(1, std::min((L + 63) / 64, (2 * cus + heads - 1) / heads));
        chunk = (L + nsplit - 1) / nsplit;
        nsplit = (L + chunk - 1) / chunk;
    }
    a.chunk = chunk;
    if (nsplit > 1) {
        size_t need = (size_t)heads * nsplit * (2 + dh);
        if (need > g_sq_part_elems) {
            if (g_sq_part) EVK_HIP(hipFree(g_sq_part));
            // a failed allocation below leaves an empty workspace, never a
            // stale size over a null pointer
            g_sq_part = nullptr;
            g_sq_part_elems = 0;
            EVK_HIP(hipMalloc(&g_sq_part, need * sizeof(float)));
            g_sq_part_elems = need;
        }
        if ((size_t)heads > g_sq_cnt_n) {
            if (g_sq_cnt) EVK_HIP(hipFree(g_sq_cnt));
            g_sq_cnt = nullptr;
            g_sq_cnt_n = 0;
            EVK_HIP(hipMalloc(&g_sq_cnt, heads * sizeof(unsigned)));
            // ordered on the launch stream before the first sq_attention
            EVK_HIP(hipMemsetAsync(g_sq_cnt, 0, heads * sizeof(unsigned), st));
            g_sq_cnt_n = heads;
        }
    }
    a.part = g_sq_part;
    a.counters = g_sq_cnt;
    dim3 grid(heads, nsplit);
    switch (dh) {
        case 16: hipLaunchKernelGGL(sq_attention<16>, grid, dim3(256), 0, st, a); break;
        case 32: hipLaunchKernelGGL(sq_attention<32>, grid, dim3(256), 0, st, a); break;
        case 64: hipLaunchKernelGGL(sq_attention<64>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(sq_attention<128>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(sq_attention<256>, grid, dim3(256), 0, st, a); break;
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "sq_attention launch");
}

int kv_cache_write_launch(const f16* src, f16* cache, int batch, int n, int D, int max_seq, int pos0,
                          hipStream_t st) {
    const int64_t total = (int64_t)batch * n * D;
    if (total == 0) return EVKHIP_OK;
    const int vec = (D % 8 == 0) && aligned16(src) && aligned16(cache);
    const int64_t threads = vec ? total / 8 : total;
    hipLaunchKernelGGL(kv_write_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src, cache, total, n,
                       D, max_seq, pos0, vec);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "kv_cache_write launch");
}

int rms_norm_launch(const f16* in, f16* out, int64_t rows, int D, float eps, hipStream_t st) {
    if (rows == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(rms_norm_k, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, in, out, rows, D, eps);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "rms_norm launch");
}

int rope_launch(const f16* in, f16* out, int B, int S, int E, float base, int pos0, int hd, hipStream_t st) {
    int64_t n = (int64_t)B * S * (E / 2);
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(rope_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, out, B, S, E, base, pos0,
                       hd);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "rope launch");
}

int gelu_launch(const f16* in, f16* out, int64_t n, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(gelu_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, out, n);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gelu launch");
}

int add_launch(const f16* a, const f16* b, f16* c, int64_t n, hipStream_t st) {
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(add_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, c, n);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "add launch");
}

int embed_launch(const f16* table, const uint16_t* idx, f16* out, int64_t n_idx, int dim, int vocab,
                 hipStream_t st) {
    int64_t n = n_idx * dim;
    if (n == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(embed_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, table, idx, out, n_idx, dim,
                       vocab);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "embed launch");
}

int greedy_launch(const f16* logits, uint16_t* out, int B, int S, int V, int position, int token_base,
                  int token_count, hipStream_t st) {
    if (B == 0) return EVKHIP_OK;
    hipLaunchKernelGGL(greedy_k, dim3(B), dim3(256), 0, st, logits, out, S, V, position, token_base, token_count);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "greedy_sample launch");
}

}  // namespace evkhip
