/*
 * CPU oracle for the evk AI hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels in
 * evk_amd/csrc are compared against; it is never linked into the product
 * library and only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Every function restates the reference
 * algorithm named in its comment (paths relative to carloshgsilva/evk).
 *
 * Conventions
 *   - fp16 tensors are passed as uint16_t bit patterns, row-major, contiguous.
 *   - Arithmetic is fp32 (fp64 where noted) with one fp16 rounding at every
 *     point where the reference stores an fp16 tensor.
 *   - The fp32->fp16 rounding is the reference's own float16_t conversion.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   f16 conversion   : oracle/_ref build of evk_ai.h float16_t, IEEE cases.
 *   matmul           : oracle/_ref cpu_matmul_nn/tn (tests.h:52-86), identity
 *                      and broadcast KATs (tests.h:163-219), fp64 brute force.
 *   attention fwd    : V==1 => O==1, K==0 => prefix mean of V, fp64 numpy
 *                      softmax, sum exp(s-lse)==1, head-permutation symmetry.
 *   attention bwd    : reference KATs tests.h:401-471 and :1499-1563, causal
 *                      uniform closed form, fp64 finite differences.
 *   sq attention     : L==1 => V0, K==0 => mean(V), row of causal fwd.
 *   rms/rope/gelu/.. : reference KATs tests.h:1169-1190,1224-1252,1318-1356,
 *                      1411-1444,1472-1497 plus their closed formulas.
 *   greedy           : tests.h:1472-1497 KAT, brute-force total order.
 *   decode model     : composition of the above; small-model step-by-step
 *                      equality with a numpy restatement.
 *   training ops     : reference KATs tests.h:221-399,619-730,1109-1470;
 *                      fp64 Adam, finite differences (gelu', rms_norm
 *                      backward), softmax Jacobian, rope adjoint identity,
 *                      closed forms (mask, sum_batch, embed backward order)
 *                      in tests/test_oracle_train.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32, restating float16_t (evk_ai.h:52-158).                     */
/* Normals round to nearest even; the subnormal branch rounds half-up on the  */
/* single guard bit and values below 2^-24 flush to signed zero, exactly as   */
/* the reference does (evk_ai.h:99-120).                                      */
/* ------------------------------------------------------------------------ */
EXPORT uint16_t orc_f32_to_f16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t sign = bits >> 31;
    uint32_t e8 = (bits >> 23) & 0xFFu;
    uint32_t mant = bits & 0x7FFFFFu;
    uint16_t hs = (uint16_t)(sign << 15);
    if (e8 == 0xFFu) {
        if (mant == 0) return hs | 0x7C00u;
        uint16_t payload = (uint16_t)((mant >> 13) & 0x3FFu);
        return hs | 0x7C00u | (payload ? payload : 1u);
    }
    int32_t e = (int32_t)e8 - 127;
    if (e > 15) return hs | 0x7C00u;
    if (e >= -14) {
        uint32_t he = (uint32_t)(e + 15);
        uint32_t m10 = mant >> 13;
        uint32_t rest = mant & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (m10 & 1u))) {
            m10++;
            if (m10 == 0x400u) {
                m10 = 0;
                he++;
                if (he == 0x1Fu) return hs | 0x7C00u;
            }
        }
        return hs | (uint16_t)(he << 10) | (uint16_t)(m10 & 0x3FFu);
    }
    if (e < -24) return hs;
    uint32_t full = mant | 0x800000u;
    int shift = -14 - e;
    uint32_t sub = full >> (13 + shift);
    if ((full >> (12 + shift)) & 1u) sub++;
    return hs | (uint16_t)(sub & 0x3FFu);
}

EXPORT float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    float out;
    if (e == 0) {
        if (m == 0) return sign ? -0.0f : 0.0f;
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 0x1Fu) {
        if (m == 0) return sign ? -INFINITY : INFINITY;
        bits = (sign << 31) | (0xFFu << 23) | (m << 13);
        memcpy(&out, &bits, 4);
        return out;
    }
    bits = (sign << 31) | ((e - 15 + 127) << 23) | (m << 13);
    memcpy(&out, &bits, 4);
    return out;
}

static float h2f(uint16_t h) { return orc_f16_to_f32(h); }
static uint16_t f2h(float f) { return orc_f32_to_f16(f); }

EXPORT void orc_f16_to_f32_n(const uint16_t* src, float* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = h2f(src[i]);
}
EXPORT void orc_f32_to_f16_n(const float* src, uint16_t* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = f2h(src[i]);
}

EXPORT int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
EXPORT void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* Portable seeded inputs (this build's own generator; the reference seeds    */
/* with platform rand(), evk_ai.h:306-344, which is not reproducible).        */
/* splitmix64 stream; uniform = top 24 bits; normal = Box-Muller.             */
/* ------------------------------------------------------------------------ */
static uint64_t sm64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double u24(uint64_t x) { return (double)(x >> 40) * (1.0 / 16777216.0); }

EXPORT void orc_fill_uniform_f16(uint16_t* out, uint64_t n, uint64_t seed, float lo, float hi) {
    uint64_t s = seed;
    for (uint64_t i = 0; i < n; ++i) {
        double u = u24(sm64(&s));
        out[i] = f2h((float)(lo + (hi - lo) * u));
    }
}

EXPORT void orc_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, float mean, float stddev) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(sm64(&s) >> 40) + 1.0) * (1.0 / 16777216.0);
        double u2 = u24(sm64(&s));
        double r = sqrt(-2.0 * log(u1));
        out[i] = f2h((float)(mean + stddev * r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = f2h((float)(mean + stddev * r * sin(two_pi * u2)));
    }
}

EXPORT void orc_fill_tokens_u16(uint16_t* out, uint64_t n, uint64_t seed, uint32_t vocab) {
    uint64_t s = seed;
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint16_t)(sm64(&s) % vocab);
}

/* ------------------------------------------------------------------------ */
/* matmul: C[b] (+)= op(A[b]) . op(B[b])                                     */
/* Semantics of evk::ai::matmul (evk_ai.cpp:254-330, matmul.comp:44-141):    */
/*   A stored (M,K) or (K,M) if ta; B stored (K,N) or (N,K) if tb;            */
/*   a per-batch stride of 0 broadcasts an operand; acc adds into C.          */
/* orc_matmul_naive is the r->n->k fp32 loop of tests.h:52-68 (the reference  */
/* CPU path); orc_matmul is the same sum with a cache-friendly loop order.    */
/* ------------------------------------------------------------------------ */
static float a_at(const uint16_t* a, int ta, uint32_t M, uint32_t K, uint32_t r, uint32_t k) {
    return h2f(ta ? a[(uint64_t)k * M + r] : a[(uint64_t)r * K + k]);
}
static float b_at(const uint16_t* b, int tb, uint32_t K, uint32_t N, uint32_t k, uint32_t n) {
    return h2f(tb ? b[(uint64_t)n * K + k] : b[(uint64_t)k * N + n]);
}

EXPORT void orc_matmul_naive(const uint16_t* a, const uint16_t* b, uint16_t* c,
                             uint32_t batch, uint32_t M, uint32_t N, uint32_t K,
                             int ta, int tb, int acc,
                             uint64_t strideA, uint64_t strideB, uint64_t strideC) {
    float* af = (float*)malloc(sizeof(float) * (uint64_t)M * K);
    float* bf = (float*)malloc(sizeof(float) * (uint64_t)K * N);
    for (uint32_t bi = 0; bi < batch; ++bi) {
        const uint16_t* ab = a + bi * strideA;
        const uint16_t* bb = b + bi * strideB;
        uint16_t* cb = c + bi * strideC;
        for (uint32_t r = 0; r < M; ++r)
            for (uint32_t k = 0; k < K; ++k) af[(uint64_t)r * K + k] = a_at(ab, ta, M, K, r, k);
        for (uint32_t k = 0; k < K; ++k)
            for (uint32_t n = 0; n < N; ++n) bf[(uint64_t)k * N + n] = b_at(bb, tb, K, N, k, n);
        for (uint32_t r = 0; r < M; ++r) {
            for (uint32_t n = 0; n < N; ++n) {
                float sum = 0.0f;
                for (uint32_t k = 0; k < K; ++k) sum += af[(uint64_t)r * K + k] * bf[(uint64_t)k * N + n];
                uint64_t ci = (uint64_t)r * N + n;
                cb[ci] = f2h(acc ? h2f(cb[ci]) + sum : sum);
            }
        }
    }
    free(af);
    free(bf);
}

/* Row-sliced naive loop (rows [r0,r1) of batch 0, NN, no acc): the bounded  */
/* sample the CPU baseline times for large shapes.                           */
EXPORT void orc_matmul_naive_rows(const float* af, const float* bf, float* cf,
                                  uint32_t r0, uint32_t r1, uint32_t N, uint32_t K) {
    for (uint32_t r = r0; r < r1; ++r)
        for (uint32_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < K; ++k) sum += af[(uint64_t)r * K + k] * bf[(uint64_t)k * N + n];
            cf[(uint64_t)r * N + n] = sum;
        }
}

EXPORT void orc_matmul(const uint16_t* a, const uint16_t* b, uint16_t* c,
                       uint32_t batch, uint32_t M, uint32_t N, uint32_t K,
                       int ta, int tb, int acc,
                       uint64_t strideA, uint64_t strideB, uint64_t strideC) {
    float* bf = (float*)malloc(sizeof(float) * (uint64_t)K * N);
    for (uint32_t bi = 0; bi < batch; ++bi) {
        const uint16_t* ab = a + bi * strideA;
        const uint16_t* bb = b + bi * strideB;
        uint16_t* cb = c + bi * strideC;
        #pragma omp parallel for schedule(static)
        for (uint32_t k = 0; k < K; ++k)
            for (uint32_t n = 0; n < N; ++n) bf[(uint64_t)k * N + n] = b_at(bb, tb, K, N, k, n);
        #pragma omp parallel
        {
            float* row = (float*)malloc(sizeof(float) * N);
            float* arow = (float*)malloc(sizeof(float) * K);
            #pragma omp for schedule(dynamic, 4)
            for (uint32_t r = 0; r < M; ++r) {
                for (uint32_t k = 0; k < K; ++k) arow[k] = a_at(ab, ta, M, K, r, k);
                for (uint32_t n = 0; n < N; ++n) row[n] = 0.0f;
                for (uint32_t k = 0; k < K; ++k) {
                    const float av = arow[k];
                    const float* brow = bf + (uint64_t)k * N;
                    for (uint32_t n = 0; n < N; ++n) row[n] += av * brow[n];
                }
                for (uint32_t n = 0; n < N; ++n) {
                    uint64_t ci = (uint64_t)r * N + n;
                    cb[ci] = f2h(acc ? h2f(cb[ci]) + row[n] : row[n]);
                }
            }
            free(row);
            free(arow);
        }
    }
    free(bf);
}

/* ------------------------------------------------------------------------ */
/* Attention.                                                                 */
/* Layout of evk::ai::flash_attention (evk_ai.h:497-501, evk_ai.cpp:332-369): */
/*   Q,O (B,N,H*Dh); K,V (B,N,Hkv*Dh).  The reference is MQA (Hkv==1); Hkv==H  */
/*   (MHA) is also accepted here for the decode model's cache.               */
/*   scale = 1/sqrt(Dh); optional causal mask j<=i; lse (B,H,N) fp32.          */
/* Softmax is evaluated exactly (two passes) in fp32/fp64.                    */
/* ------------------------------------------------------------------------ */
EXPORT void orc_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              uint16_t* o, float* lse,
                              uint32_t B, uint32_t H, uint32_t Hkv, uint32_t N, uint32_t Dh,
                              int causal, float scale) {
    const uint64_t D = (uint64_t)H * Dh, Dkv = (uint64_t)Hkv * Dh;
    const uint32_t group = H / Hkv;
    #pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * N);
        float* qf = (float*)malloc(sizeof(float) * Dh);
        double* acc = (double*)malloc(sizeof(double) * Dh);
        #pragma omp for collapse(2) schedule(dynamic, 8)
        for (uint32_t bh = 0; bh < B * H; ++bh) {
            for (uint32_t i = 0; i < N; ++i) {
                uint32_t b = bh / H, h = bh % H, hk = h / group;
                const uint16_t* qr = q + ((uint64_t)b * N + i) * D + (uint64_t)h * Dh;
                for (uint32_t d = 0; d < Dh; ++d) qf[d] = h2f(qr[d]);
                uint32_t L = causal ? i + 1 : N;
                float m = -INFINITY;
                for (uint32_t j = 0; j < L; ++j) {
                    const uint16_t* kr = k + ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh;
                    float dot = 0.0f;
                    for (uint32_t d = 0; d < Dh; ++d) dot += qf[d] * h2f(kr[d]);
                    s[j] = dot * scale;
                    if (s[j] > m) m = s[j];
                }
                double l = 0.0;
                for (uint32_t d = 0; d < Dh; ++d) acc[d] = 0.0;
                for (uint32_t j = 0; j < L; ++j) {
                    double p = exp((double)s[j] - (double)m);
                    l += p;
                    const uint16_t* vr = v + ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh;
                    for (uint32_t d = 0; d < Dh; ++d) acc[d] += p * (double)h2f(vr[d]);
                }
                uint16_t* orow = o + ((uint64_t)b * N + i) * D + (uint64_t)h * Dh;
                for (uint32_t d = 0; d < Dh; ++d) orow[d] = f2h((float)(acc[d] / l));
                if (lse) lse[((uint64_t)b * H + h) * N + i] = (float)((double)m + log(l));
            }
        }
        free(s);
        free(qf);
        free(acc);
    }
}

/* Textbook FlashAttention-2 backward (not the shader's algorithm, which uses */
/* an un-normalised D and races for N>16: flash_attention_bwd.comp:119-131,  */
/* 210-231).  Contract of evk::ai::flash_attention_bwd (evk_ai.cpp:371-473):  */
/*   dQ (B,N,H*Dh); dK,dV (B,N,Hkv*Dh) summed over the heads sharing them;    */
/*   O is not read: D_i = sum_j P_ij dP_ij, which equals rowsum(dO_i * O_i).  */
EXPORT void orc_attention_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* dO, uint16_t* dQ, uint16_t* dK, uint16_t* dV,
                              uint32_t B, uint32_t H, uint32_t Hkv, uint32_t N, uint32_t Dh,
                              int causal, float scale) {
    const uint64_t D = (uint64_t)H * Dh, Dkv = (uint64_t)Hkv * Dh;
    const uint32_t group = H / Hkv;
    double* gk = (double*)calloc((uint64_t)B * N * Dkv, sizeof(double));
    double* gv = (double*)calloc((uint64_t)B * N * Dkv, sizeof(double));
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t hk = 0; hk < Hkv; ++hk) {
            /* dK/dV for one kv head gather from `group` query heads: keep the  */
            /* accumulation serial per (b,hk) and parallel over query rows with  */
            /* per-thread partials to stay deterministic.                        */
            int nt = orc_max_threads();
            double* pk = (double*)calloc((uint64_t)nt * N * Dh, sizeof(double));
            double* pv = (double*)calloc((uint64_t)nt * N * Dh, sizeof(double));
            #pragma omp parallel
            {
                int tid = 0;
#ifdef _OPENMP
                tid = omp_get_thread_num();
#endif
                double* myk = pk + (uint64_t)tid * N * Dh;
                double* myv = pv + (uint64_t)tid * N * Dh;
                double* p = (double*)malloc(sizeof(double) * N);
                double* dp = (double*)malloc(sizeof(double) * N);
                double* dq = (double*)malloc(sizeof(double) * Dh);
                #pragma omp for collapse(2) schedule(static)
                for (uint32_t hh = 0; hh < group; ++hh) {
                    for (uint32_t i = 0; i < N; ++i) {
                        uint32_t h = hk * group + hh;
                        const uint16_t* qr = q + ((uint64_t)b * N + i) * D + (uint64_t)h * Dh;
                        const uint16_t* dor = dO + ((uint64_t)b * N + i) * D + (uint64_t)h * Dh;
                        uint32_t L = causal ? i + 1 : N;
                        double m = -INFINITY;
                        for (uint32_t j = 0; j < L; ++j) {
                            const uint16_t* kr = k + ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh;
                            const uint16_t* vr = v + ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh;
                            float dot = 0.0f, dpv = 0.0f;
                            for (uint32_t d = 0; d < Dh; ++d) {
                                dot += h2f(qr[d]) * h2f(kr[d]);
                                dpv += h2f(dor[d]) * h2f(vr[d]);
                            }
                            p[j] = (double)dot * scale;
                            dp[j] = dpv;
                            if (p[j] > m) m = p[j];
                        }
                        double l = 0.0;
                        for (uint32_t j = 0; j < L; ++j) { p[j] = exp(p[j] - m); l += p[j]; }
                        double Di = 0.0;
                        for (uint32_t j = 0; j < L; ++j) { p[j] /= l; Di += p[j] * dp[j]; }
                        for (uint32_t d = 0; d < Dh; ++d) dq[d] = 0.0;
                        for (uint32_t j = 0; j < L; ++j) {
                            const uint16_t* kr = k + ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh;
                            double ds = p[j] * (dp[j] - Di) * scale;
                            for (uint32_t d = 0; d < Dh; ++d) {
                                dq[d] += ds * h2f(kr[d]);
                                myk[(uint64_t)j * Dh + d] += ds * h2f(qr[d]);
                                myv[(uint64_t)j * Dh + d] += p[j] * h2f(dor[d]);
                            }
                        }
                        uint16_t* dqr = dQ + ((uint64_t)b * N + i) * D + (uint64_t)h * Dh;
                        for (uint32_t d = 0; d < Dh; ++d) dqr[d] = f2h((float)dq[d]);
                    }
                }
                free(p);
                free(dp);
                free(dq);
            }
            for (int t = 0; t < nt; ++t)
                for (uint32_t j = 0; j < N; ++j)
                    for (uint32_t d = 0; d < Dh; ++d) {
                        uint64_t gi = ((uint64_t)b * N + j) * Dkv + (uint64_t)hk * Dh + d;
                        gk[gi] += pk[((uint64_t)t * N + j) * Dh + d];
                        gv[gi] += pv[((uint64_t)t * N + j) * Dh + d];
                    }
            free(pk);
            free(pv);
        }
    }
    for (uint64_t i = 0; i < (uint64_t)B * N * Dkv; ++i) {
        dK[i] = f2h((float)gk[i]);
        dV[i] = f2h((float)gv[i]);
    }
    free(gk);
    free(gv);
}

/* Single-query attention (single_query_attention.comp:26-72), generalised  */
/* to `heads` heads of `dh` channels: head h of the query attends to columns */
/* [h*dh,(h+1)*dh) of cache rows 0..L-1 (row stride `row_stride` elements).  */
/* heads==1, dh<=64, L<=160 is exactly the shader's contract.                */
EXPORT void orc_sq_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                             uint16_t* out, uint32_t heads, uint32_t dh, uint32_t L,
                             uint64_t row_stride) {
    float* s = (float*)malloc(sizeof(float) * (L ? L : 1));
    float* w = (float*)malloc(sizeof(float) * (L ? L : 1));
    const float inv = 1.0f / sqrtf((float)dh);
    for (uint32_t h = 0; h < heads; ++h) {
        const uint16_t* qh = q + (uint64_t)h * dh;
        float mx = -3.402823466e+38f;
        for (uint32_t j = 0; j < L; ++j) {
            const uint16_t* kr = kc + (uint64_t)j * row_stride + (uint64_t)h * dh;
            float acc = 0.0f;
            for (uint32_t d = 0; d < dh; ++d) acc += h2f(qh[d]) * h2f(kr[d]);
            s[j] = acc * inv;
            if (s[j] > mx) mx = s[j];
        }
        float sum = 0.0f;
        for (uint32_t j = 0; j < L; ++j) { w[j] = expf(s[j] - mx); sum += w[j]; }
        float is = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (uint32_t d = 0; d < dh; ++d) {
            float acc = 0.0f;
            for (uint32_t j = 0; j < L; ++j)
                acc += (w[j] * is) * h2f(vc[(uint64_t)j * row_stride + (uint64_t)h * dh + d]);
            out[(uint64_t)h * dh + d] = f2h(acc);
        }
    }
    free(s);
    free(w);
}

/* ------------------------------------------------------------------------ */
/* Decode-step support ops.                                                   */
/* ------------------------------------------------------------------------ */

/* rms_norm.comp:21-49: clamp to +-65504, x * rsqrt(mean(x^2) + eps), no gain */
EXPORT void orc_rms_norm(const uint16_t* in, uint16_t* out, uint64_t rows, uint32_t D, float eps) {
    for (uint64_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * D;
        float ss = 0.0f;
        for (uint32_t j = 0; j < D; ++j) {
            float t = fminf(fmaxf(h2f(x[j]), -65504.0f), 65504.0f);
            ss += t * t;
        }
        float inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (uint32_t j = 0; j < D; ++j) {
            float t = fminf(fmaxf(h2f(x[j]), -65504.0f), 65504.0f);
            out[r * D + j] = f2h(t * inv);
        }
    }
}

/* rope.comp:18-41 over (B,S,E): pairs (2p,2p+1) rotate by                     */
/* theta = t * base^(-2p/hd).  Extensions (defaults give the reference):      */
/*   t = pos0 + sequence index; hd = head_dim (0 => E) splits E into E/hd      */
/*   independently rotated heads.                                             */
EXPORT void orc_rope(const uint16_t* in, uint16_t* out, uint32_t B, uint32_t S, uint32_t E,
                     float base, uint32_t pos0, uint32_t head_dim) {
    uint32_t hd = head_dim ? head_dim : E;
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t t = 0; t < S; ++t)
            for (uint32_t pr = 0; pr < E / 2; ++pr) {
                uint64_t idx = ((uint64_t)b * S + t) * E + 2u * pr;
                uint32_t p = pr % (hd / 2);
                float x0 = h2f(in[idx]), x1 = h2f(in[idx + 1]);
                float inv_freq = powf(base, -2.0f * (float)p / (float)hd);
                float ang = (float)(pos0 + t) * inv_freq;
                float c = cosf(ang), s = sinf(ang);
                out[idx] = f2h(x0 * c - x1 * s);
                out[idx + 1] = f2h(x0 * s + x1 * c);
            }
}

/* gelu.comp:15-30 (tanh approximation) */
EXPORT float orc_gelu_f32(float x) {
    const float a = 0.7978845608028654f, bcoef = 0.044715f;
    float x3 = x * x * x;
    return 0.5f * x * (1.0f + tanhf(a * (x + bcoef * x3)));
}
EXPORT void orc_gelu(const uint16_t* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = f2h(orc_gelu_f32(h2f(in[i])));
}

/* add.comp:18-26 */
EXPORT void orc_add(const uint16_t* a, const uint16_t* b, uint16_t* c, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) c[i] = f2h(h2f(a[i]) + h2f(b[i]));
}

/* embed.comp:18-28: out[i,:] = E[idx[i],:] (ids are raw u16) */
EXPORT void orc_embed(const uint16_t* table, const uint16_t* idx, uint16_t* out,
                      uint64_t n_idx, uint32_t dim) {
    for (uint64_t i = 0; i < n_idx; ++i)
        memcpy(out + i * dim, table + (uint64_t)idx[i] * dim, sizeof(uint16_t) * dim);
}

/* greedy_sample.comp:24-64, simulated lane by lane: 256 invocations scan      */
/* tokens lid, lid+256, ... keeping the first strict maximum (initial value    */
/* -FLT_MAX, initial token token_base), then the strided tree reduction keeps  */
/* the lower slot unless the upper one is strictly greater.                    */
EXPORT uint16_t orc_greedy_row(const uint16_t* row, uint32_t token_base, uint32_t token_count) {
    float bv[256];
    uint32_t bt[256];
    for (uint32_t lid = 0; lid < 256; ++lid) {
        float best = -3.402823466e+38f;
        uint32_t tok = token_base;
        for (uint32_t j = lid; j < token_count; j += 256) {
            float val = h2f(row[token_base + j]);
            if (val > best) { best = val; tok = token_base + j; }
        }
        bv[lid] = best;
        bt[lid] = tok;
    }
    for (uint32_t stride = 128; stride > 0; stride >>= 1)
        for (uint32_t lid = 0; lid < stride; ++lid)
            if (bv[lid + stride] > bv[lid]) { bv[lid] = bv[lid + stride]; bt[lid] = bt[lid + stride]; }
    return (uint16_t)bt[0];
}

EXPORT void orc_greedy_sample(const uint16_t* logits, uint16_t* out_tokens,
                              uint32_t B, uint32_t S, uint32_t V, uint32_t position,
                              uint32_t token_base, uint32_t token_count) {
    for (uint32_t b = 0; b < B; ++b)
        out_tokens[b] = orc_greedy_row(logits + ((uint64_t)b * S + position) * V, token_base, token_count);
}

/* ------------------------------------------------------------------------ */
/* KV-cached greedy decode model (the caller of the hot path).                */
/* Block structure follows CausalAttentionBlock::forward                      */
/* (example/main_llm.cpp:528-546) and MeshTokenModel (:598-606): pre-norm     */
/* rms_norm (no gain), x.W projections with W stored (in,out), rope on q and   */
/* k, causal attention, x.Wo residual, rms_norm, gelu(x.W1).W2 residual, final  */
/* rms_norm, x.Wout, greedy argmax.  Multi-head with per-head rope and a       */
/* KV cache is this build's decode form of that block.                        */
/*                                                                            */
/* Weight blob layout (fp16, contiguous):                                     */
/*   E (vocab,d); per layer: Wqkv (d,3d) [q|k|v columns], Wo (d,d),           */
/*   W1 (d,hidden), W2 (hidden,d); then Wout (d,vocab).                       */
/* Cache layout: per layer K (max_seq,d) then V (max_seq,d).                   */
/* ------------------------------------------------------------------------ */
typedef struct {
    uint32_t vocab, d, heads, dh, layers, hidden, max_seq;
    float eps, rope_base;
} orc_model_cfg;

EXPORT uint64_t orc_model_weight_elems(const orc_model_cfg* c) {
    uint64_t d = c->d;
    uint64_t per = d * 3 * d + d * d + d * c->hidden + (uint64_t)c->hidden * d;
    return (uint64_t)c->vocab * d + c->layers * per + d * c->vocab;
}
EXPORT uint64_t orc_model_cache_elems(const orc_model_cfg* c) {
    return (uint64_t)c->layers * 2 * c->max_seq * c->d;
}

/* y(1,N) = fp16(x(1,K) . W(K,N)), fp32 accumulation */
static void gemv16(const uint16_t* x, const uint16_t* W, uint16_t* y, uint32_t K, uint32_t N,
                   uint64_t ldw, float* scratch) {
    #pragma omp parallel for schedule(static)
    for (uint32_t n = 0; n < N; ++n) scratch[n] = 0.0f;
    #pragma omp parallel
    {
        #pragma omp for schedule(static)
        for (uint32_t nb = 0; nb < (N + 255) / 256; ++nb) {
            uint32_t n0 = nb * 256, n1 = n0 + 256 < N ? n0 + 256 : N;
            float acc[256];
            for (uint32_t n = n0; n < n1; ++n) acc[n - n0] = 0.0f;
            for (uint32_t kk = 0; kk < K; ++kk) {
                float xv = h2f(x[kk]);
                const uint16_t* wr = W + (uint64_t)kk * ldw;
                for (uint32_t n = n0; n < n1; ++n) acc[n - n0] += xv * h2f(wr[n]);
            }
            for (uint32_t n = n0; n < n1; ++n) scratch[n] = acc[n - n0];
        }
    }
    for (uint32_t n = 0; n < N; ++n) y[n] = f2h(scratch[n]);
}

/* Runs tokens[0..n) at positions pos0.. through the model, appending to the  */
/* cache; after the last token writes logits (fp16, vocab) and returns the     */
/* greedy id.                                                                 */
EXPORT uint32_t orc_model_forward(const orc_model_cfg* c, const uint16_t* w, uint16_t* cache,
                                  const uint16_t* tokens, uint32_t n, uint32_t pos0,
                                  uint16_t* logits) {
    const uint32_t d = c->d, hid = c->hidden, V = c->vocab;
    const uint64_t per = (uint64_t)d * 3 * d + (uint64_t)d * d + (uint64_t)d * hid + (uint64_t)hid * d;
    const uint16_t* E = w;
    const uint16_t* Wout = w + (uint64_t)V * d + c->layers * per;
    uint16_t* x = (uint16_t*)malloc(2 * d);
    uint16_t* hbuf = (uint16_t*)malloc(2 * d);
    uint16_t* qkv = (uint16_t*)malloc(2 * 3 * d);
    uint16_t* qk_r = (uint16_t*)malloc(2 * 2 * d);
    uint16_t* att = (uint16_t*)malloc(2 * d);
    uint16_t* tmp = (uint16_t*)malloc(2 * d);
    uint16_t* hh = (uint16_t*)malloc(2 * hid);
    uint16_t* hg = (uint16_t*)malloc(2 * hid);
    uint32_t big = V > 3 * d ? V : 3 * d;
    if (hid > big) big = hid;
    float* scratch = (float*)malloc(sizeof(float) * big);
    uint32_t last = 0;
    for (uint32_t t = 0; t < n; ++t) {
        uint32_t pos = pos0 + t;
        orc_embed(E, tokens + t, x, 1, d);
        for (uint32_t l = 0; l < c->layers; ++l) {
            const uint16_t* Wqkv = w + (uint64_t)V * d + l * per;
            const uint16_t* Wo = Wqkv + (uint64_t)d * 3 * d;
            const uint16_t* W1 = Wo + (uint64_t)d * d;
            const uint16_t* W2 = W1 + (uint64_t)d * hid;
            uint16_t* Kc = cache + (uint64_t)l * 2 * c->max_seq * d;
            uint16_t* Vc = Kc + (uint64_t)c->max_seq * d;
            orc_rms_norm(x, hbuf, 1, d, c->eps);
            gemv16(hbuf, Wqkv, qkv, d, 3 * d, 3 * d, scratch);
            /* rope on q and k (heads of dh channels) at absolute position pos */
            orc_rope(qkv, qk_r, 1, 1, d, c->rope_base, pos, c->dh);
            orc_rope(qkv + d, qk_r + d, 1, 1, d, c->rope_base, pos, c->dh);
            memcpy(Kc + (uint64_t)pos * d, qk_r + d, 2 * d);
            memcpy(Vc + (uint64_t)pos * d, qkv + 2 * d, 2 * d);
            orc_sq_attention(qk_r, Kc, Vc, att, c->heads, c->dh, pos + 1, d);
            gemv16(att, Wo, tmp, d, d, d, scratch);
            orc_add(x, tmp, x, d);
            orc_rms_norm(x, hbuf, 1, d, c->eps);
            gemv16(hbuf, W1, hh, d, hid, hid, scratch);
            orc_gelu(hh, hg, hid);
            gemv16(hg, W2, tmp, hid, d, d, scratch);
            orc_add(x, tmp, x, d);
        }
        if (t + 1 == n) {
            orc_rms_norm(x, hbuf, 1, d, c->eps);
            gemv16(hbuf, Wout, logits, d, V, V, scratch);
            last = orc_greedy_row(logits, 0, V);
        }
    }
    free(x); free(hbuf); free(qkv); free(qk_r); free(att); free(tmp); free(hh); free(hg);
    free(scratch);
    return last;
}

/* Prefill tokens[0..n_prompt) then `steps` greedy steps; ids_out gets the    */
/* steps+1 generated ids (the first comes from the prompt's last position).   */
EXPORT void orc_model_generate(const orc_model_cfg* c, const uint16_t* w, uint16_t* cache,
                               const uint16_t* prompt, uint32_t n_prompt, uint32_t steps,
                               uint16_t* ids_out, uint16_t* logits_all /* (steps+1,vocab) or NULL */) {
    uint16_t* lg = (uint16_t*)malloc(2 * (uint64_t)c->vocab);
    uint32_t id = orc_model_forward(c, w, cache, prompt, n_prompt, 0, lg);
    ids_out[0] = (uint16_t)id;
    if (logits_all) memcpy(logits_all, lg, 2 * (uint64_t)c->vocab);
    for (uint32_t s = 0; s < steps; ++s) {
        uint16_t tok = (uint16_t)id;
        id = orc_model_forward(c, w, cache, &tok, 1, n_prompt + s, lg);
        ids_out[s + 1] = (uint16_t)id;
        if (logits_all) memcpy(logits_all + (uint64_t)(s + 1) * c->vocab, lg, 2 * (uint64_t)c->vocab);
    }
    free(lg);
}

/* One decode step from an existing cache (position pos); used by the         */
/* full-size parity test, which starts from the GPU's prefilled cache.        */
EXPORT uint32_t orc_model_step(const orc_model_cfg* c, const uint16_t* w, uint16_t* cache,
                               uint16_t token, uint32_t pos, uint16_t* logits) {
    return orc_model_forward(c, w, cache, &token, 1, pos, logits);
}

/* ======================================================================== */
/* Training ops (the reference's non-inference shaders).  In-place outputs   */
/* (gradients the shader accumulates into, optimiser state) are updated in   */
/* the caller's arrays.                                                      */
/* ======================================================================== */

/* scale.comp:14-20 */
EXPORT void orc_scale(uint16_t* x, float s, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) x[i] = f2h(h2f(x[i]) * s);
}

/* relu.comp:14-20 */
EXPORT void orc_relu(const uint16_t* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        float v = h2f(in[i]);
        out[i] = f2h(v > 0.0f ? v : 0.0f);
    }
}

/* relu_bwd.comp:15-23 */
EXPORT void orc_relu_bwd(const uint16_t* gout, const uint16_t* in, uint16_t* gin, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        gin[i] = f2h(h2f(gin[i]) + (h2f(in[i]) > 0.0f ? h2f(gout[i]) : 0.0f));
}

/* gelu_bwd.comp:16-27: derivative of the tanh GELU */
EXPORT float orc_gelu_grad_f32(float x) {
    const float a = 0.7978845608028654f, b = 0.044715f;
    float x2 = x * x, x3 = x2 * x;
    float t = tanhf(a * (x + b * x3));
    float sech2 = 1.0f - t * t;
    float du = a * (1.0f + 3.0f * b * x2);
    return 0.5f * (1.0f + t) + 0.5f * x * sech2 * du;
}

/* gelu_bwd.comp:29-37 */
EXPORT void orc_gelu_bwd(const uint16_t* gout, const uint16_t* in, uint16_t* gin, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        gin[i] = f2h(h2f(gin[i]) + h2f(gout[i]) * orc_gelu_grad_f32(h2f(in[i])));
}

/* sgd.comp:15-24 */
EXPORT void orc_sgd(uint16_t* param, const uint16_t* grad, float lr, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) param[i] = f2h(h2f(param[i]) - lr * h2f(grad[i]));
}

/* adam.comp:32-84 with the host's bias corrections (evk_ai.cpp:541-545):
 * state m = m / rms, v = log2(rms) + 41 (0 = rms 0), fp16 */
EXPORT void orc_adam(uint16_t* param, const uint16_t* grad, uint16_t* m_s, uint16_t* v_s, uint64_t n,
                     float lr, float b1, float b2, float c1inv, float c2inv, float eps) {
    for (uint64_t i = 0; i < n; ++i) {
        float g = h2f(grad[i]);
        float stored = h2f(v_s[i]);
        float rms = stored > 0.0f ? exp2f(stored - 41.0f) : 0.0f;
        float m = h2f(m_s[i]) * rms, v = rms * rms;
        if (isnan(g) || isinf(g)) continue;
        m = b1 * m + (1.0f - b1) * g;
        v = b2 * v + (1.0f - b2) * g * g;
        rms = sqrtf(v > 0.0f ? v : 0.0f);
        float mn = m / (rms > 1.0e-8f ? rms : 1.0e-8f);
        if (!isnan(mn) && !isinf(mn)) m_s[i] = f2h(mn);
        float lr2 = log2f(rms > 1.0e-12f ? rms : 1.0e-12f) + 41.0f;
        if (!isnan(lr2) && !isinf(lr2)) v_s[i] = f2h(lr2);
        float upd = lr * (m * c1inv) / (rms * sqrtf(c2inv) + eps);
        if (!isnan(upd) && !isinf(upd)) {
            float p = h2f(param[i]) - upd;
            p = p < -65504.0f ? -65504.0f : (p > 65504.0f ? 65504.0f : p);
            param[i] = f2h(p);
        }
    }
}

/* softmax.comp:21-69: per row of D, over in * scale; raw values <= -65504
 * are masked (output 0); sums in double here */
EXPORT void orc_softmax(const uint16_t* in, uint16_t* out, float scale, uint64_t rows, uint32_t D) {
    for (uint64_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * D;
        uint16_t* y = out + r * D;
        float mx = -3.402823466e+38f;
        for (uint32_t j = 0; j < D; ++j) {
            float v = h2f(x[j]);
            if (v > -65504.0f && v * scale > mx) mx = v * scale;
        }
        double sum = 0.0;
        for (uint32_t j = 0; j < D; ++j) {
            float v = h2f(x[j]);
            if (v > -65504.0f) sum += exp((double)(v * scale - mx));
        }
        double inv = 1.0 / (sum > 1e-20 ? sum : 1e-20);
        for (uint32_t j = 0; j < D; ++j) {
            float v = h2f(x[j]);
            y[j] = f2h(v > -65504.0f ? (float)(exp((double)(v * scale - mx)) * inv) : 0.0f);
        }
    }
}

/* softmax_bwd.comp:20-43: grad_in += p (g - p.g) scale per row */
EXPORT void orc_softmax_bwd(const uint16_t* probs, const uint16_t* gout, uint16_t* gin, float scale,
                            uint64_t rows, uint32_t D) {
    for (uint64_t r = 0; r < rows; ++r) {
        const uint16_t* p = probs + r * D;
        const uint16_t* g = gout + r * D;
        uint16_t* o = gin + r * D;
        double dot = 0.0;
        for (uint32_t j = 0; j < D; ++j) dot += (double)h2f(p[j]) * h2f(g[j]);
        for (uint32_t j = 0; j < D; ++j)
            o[j] = f2h(h2f(o[j]) + (float)((double)h2f(p[j]) * (h2f(g[j]) - dot) * scale));
    }
}

/* rms_norm_bwd.comp:24-70: grad_in += g/rms - x (g.y) / (D rms^2), y = x/rms,
 * rms = sqrt(mean(x^2) + eps), x clamped to the fp16 range */
EXPORT void orc_rms_norm_bwd(const uint16_t* in, const uint16_t* gout, uint16_t* gin, float eps,
                             uint64_t rows, uint32_t D) {
    for (uint64_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * D;
        const uint16_t* g = gout + r * D;
        uint16_t* o = gin + r * D;
        double ss = 0.0;
        for (uint32_t j = 0; j < D; ++j) {
            double v = fmin(fmax(h2f(x[j]), -65504.0), 65504.0);
            ss += v * v;
        }
        double inv = 1.0 / sqrt(ss / D + eps);
        double dot = 0.0;
        for (uint32_t j = 0; j < D; ++j) dot += h2f(g[j]) * (fmin(fmax(h2f(x[j]), -65504.0), 65504.0) * inv);
        double sc = dot / D;
        for (uint32_t j = 0; j < D; ++j) {
            double v = fmin(fmax(h2f(x[j]), -65504.0), 65504.0);
            o[j] = f2h((float)(h2f(o[j]) + (h2f(g[j]) * inv - v * inv * inv * sc)));
        }
    }
}

/* mse_loss.comp:23-48: grad = 2 (p - t) / n, result = sum (p - t)^2 / n */
EXPORT void orc_mse_loss(const uint16_t* pred, const uint16_t* tgt, uint16_t* grad, uint16_t* result, uint64_t n) {
    double s = 0.0;
    const float gs = 2.0f / (float)n;
    for (uint64_t i = 0; i < n; ++i) {
        float d = h2f(pred[i]) - h2f(tgt[i]);
        s += (double)d * d;
        grad[i] = f2h(gs * d);
    }
    result[0] = f2h((float)(s / (double)n));
}

/* cross_entropy_count.comp, cross_entropy.comp:27-106, cross_entropy_scale.comp:
 * targets 0 or >= V are ignored (zero gradient row); logits clamped to
 * +-65000; grad = (softmax - onehot) / n_valid; result = mean loss over the
 * valid rows (0 if none or not finite) */
EXPORT void orc_cross_entropy(const uint16_t* logits, const uint16_t* targets, uint16_t* grad, uint16_t* result,
                              uint64_t P, uint32_t V) {
    uint64_t valid = 0;
    for (uint64_t r = 0; r < P; ++r)
        if (targets[r] != 0 && targets[r] < V) ++valid;
    double total = 0.0;
    for (uint64_t r = 0; r < P; ++r) {
        const uint16_t* x = logits + r * V;
        uint16_t* g = grad + r * V;
        uint32_t t = targets[r];
        if (t == 0 || t >= V || valid == 0) {
            for (uint32_t j = 0; j < V; ++j) g[j] = 0;
            continue;
        }
        double inv_valid = 1.0 / (double)valid;
        double mx = -3.402823466e+38;
        for (uint32_t j = 0; j < V; ++j) {
            double v = fmin(fmax(h2f(x[j]), -65000.0), 65000.0);
            if (v > mx) mx = v;
        }
        double sum = 0.0;
        for (uint32_t j = 0; j < V; ++j) sum += exp(fmin(fmax(h2f(x[j]), -65000.0), 65000.0) - mx);
        if (sum < 1e-20) sum = 1e-20;
        for (uint32_t j = 0; j < V; ++j) {
            double v = fmin(fmax(h2f(x[j]), -65000.0), 65000.0);
            double gv = exp(v - mx) / sum * inv_valid;
            if (j == t) gv -= inv_valid;
            g[j] = f2h((float)gv);
        }
        double vt = fmin(fmax(h2f(x[t]), -65000.0), 65000.0);
        total += (mx + log(sum) - vt) * inv_valid;
    }
    float loss = valid > 0 ? (float)total : 0.0f;
    if (isnan(loss) || isinf(loss)) loss = 0.0f;
    result[0] = f2h(loss);
}

/* sum_batch.comp:14-24: out[i] = out[i] + sum_b in[b, i], one rounding */
EXPORT void orc_sum_batch(const uint16_t* in, uint16_t* out, uint32_t batch, uint64_t per) {
    for (uint64_t i = 0; i < per; ++i) {
        float s = h2f(out[i]);
        for (uint32_t b = 0; b < batch; ++b) s += h2f(in[(uint64_t)b * per + i]);
        out[i] = f2h(s);
    }
}

/* causal_mask.comp:13-30: scores[b, i, j] = -65504 for j > i */
EXPORT void orc_causal_mask(uint16_t* scores, uint64_t batch, uint32_t N) {
    const uint16_t neg = orc_f32_to_f16(-65504.0f);
    for (uint64_t b = 0; b < batch; ++b)
        for (uint32_t i = 0; i < N; ++i)
            for (uint32_t j = i + 1; j < N; ++j) scores[(b * N + i) * N + j] = neg;
}

/* position_add.comp:17-34 */
EXPORT void orc_position_add(const uint16_t* in, const uint16_t* pos, uint16_t* out, uint32_t B, uint64_t per) {
    for (uint32_t b = 0; b < B; ++b)
        for (uint64_t i = 0; i < per; ++i) out[b * per + i] = f2h(h2f(in[b * per + i]) + h2f(pos[i]));
}

/* position_add_bwd.comp:20-49, both modes */
EXPORT void orc_position_add_bwd(const uint16_t* gout, uint16_t* gin, uint16_t* gpos, uint32_t B, uint64_t per) {
    for (uint64_t i = 0; i < (uint64_t)B * per; ++i) gin[i] = f2h(h2f(gin[i]) + h2f(gout[i]));
    for (uint64_t i = 0; i < per; ++i) {
        float s = h2f(gpos[i]);
        for (uint32_t b = 0; b < B; ++b) s += h2f(gout[b * per + i]);
        gpos[i] = f2h(s);
    }
}

/* rope_bwd.comp:15-45: grad_in += R(t)^T grad_out per pair */
EXPORT void orc_rope_bwd(const uint16_t* gout, uint16_t* gin, uint32_t B, uint32_t S, uint32_t E, float base) {
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t t = 0; t < S; ++t)
            for (uint32_t p = 0; p < E / 2; ++p) {
                uint64_t i = ((uint64_t)b * S + t) * E + 2 * p;
                float g0 = h2f(gout[i]), g1 = h2f(gout[i + 1]);
                float inv_freq = powf(base, -2.0f * (float)p / (float)E);
                float c = cosf((float)t * inv_freq), s = sinf((float)t * inv_freq);
                gin[i] = f2h(h2f(gin[i]) + (g0 * c + g1 * s));
                gin[i + 1] = f2h(h2f(gin[i + 1]) + (-g0 * s + g1 * c));
            }
}

/* embed_bwd.comp:16-32: grad_emb[idx[r]] += grad_out[r] for r in order, one
 * fp16 rounding per addition; ids >= vocab skipped */
EXPORT void orc_embed_bwd(const uint16_t* gout, const uint16_t* idx, uint16_t* gemb, uint64_t n_idx, uint32_t dim,
                          uint32_t vocab) {
    for (uint64_t r = 0; r < n_idx; ++r) {
        uint32_t tok = idx[r];
        if (tok >= vocab) continue;
        for (uint32_t d = 0; d < dim; ++d) {
            uint16_t* dst = gemb + (uint64_t)tok * dim + d;
            *dst = f2h(h2f(*dst) + h2f(gout[r * dim + d]));
        }
    }
}
