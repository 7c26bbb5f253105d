// Persistent greedy decode: every stage of every decode step in one
// persistent launch (the decode loop of the reference's caller,
// example/main_llm.cpp:622-654, in the KV-cached form of model.hip).
//
// Why: a decode step of the C4 model is 61 dependent matrix-vector stages
// of 1-5 MB each.  Launched as kernels, each stage pays a launch boundary
// (about 1.6 us on MI355X) plus the reload of its input from memory; here
// the stages hand their outputs to each other inside one launch, and every
// stage's weights are requested before the stage waits for its input.
//
// Hand-over ("mailboxes").  A stage writes its output as 64-bit words
// (payload: two fp16 or one fp32; high half: the stage's epoch tag) with
// agent-scope stores, which the hardware writes through to the device
// coherence point; a consumer polls the words with agent-scope loads until
// each carries the tag it expects, so the data and the "ready" flag arrive
// in one single-copy-atomic word and no separate barrier or fence is
// needed.  Tags grow by one per stage; a launch takes its base from ctl[0]
// and moves it past its own tags as soon as every workgroup has read it, so
// that graph replays of one launch, and launches after one that gave up, use
// new tags.  Every poll is bounded: on timeout the workgroup raises
// EVKHIP_STATUS_WAIT_TIMEOUT and leaves, and so, bounded in turn, do the
// workgroups waiting on it.
//
// Weights are taken pre-packed (evkhip_model_pack): each matrix transposed to
// (N, K), so that one output column's weights are one contiguous row and a
// stage's output columns need no cross-workgroup reduction.
//
// Stages of layer l (parity p = l & 1 selects a mailbox copy; a copy is
// rewritten two layers later, after stages that every workgroup takes part
// in, so its readers are done with it):
//   S1 all: x <- poll X2[p^1] (or the embedding row of the step's token, from
//      the previous step's LM-head candidates), h = rms_norm(x); columns of
//      h.Wqkv in pairs, rope on q and k -> QKV[p] (per head: q, k, v); k, v
//      rows of the cache at pos (written through).
//   S2 H*S workgroups: head h, key split s: q, (k, v of pos) <- poll; the
//      split's (m, l, o/l) -> ATT[p].
//   S3 G3 workgroups: attn = merge of the splits; x1 = x + attn.Wo (columns in
//      pairs) -> X1[p].
//   S4 all: x1 <- poll; gelu(rms_norm(x1).W1) -> GH[p].
//   S5 G5 workgroups: x2 = x1 + GH.W2 -> X2[p].
//   head all: x <- poll X2; logits = rms_norm(x).Wout; the workgroup's greedy
//      candidate -> CAND; the next step's S1 (or workgroup 0 after the last
//      step) picks the winner in the greedy_sample order.
#include "kernels.h"

#include <math.h>

#define DEV_HOST_INLINE __host__ __device__ __forceinline__

namespace evkhip {
namespace {

constexpr int PNT = 512;           // threads per workgroup
constexpr int PWV = PNT / 64;      // waves
constexpr int NPOLL = 256;         // waves 0-3 poll and write outputs; waves 4-7 stream weights
constexpr int PMAXW = 16;          // mailbox words one polling thread takes (<= 16 * NPOLL per poll)
constexpr int NBUF = 3;            // LDS weight slots: a stage's slice is requested two stages ahead
constexpr int KSPL = 128;          // keys per attention split
constexpr uint32_t kWrapAt = 0xFFF00000u;
constexpr int RSQ = 32;            // red[RSQ, RSQ + 4): the polling waves' sums of squares
constexpr int YO = 144;            // stage output floats (>= head rows per slot, >= dh + 2)

__device__ unsigned g_dec_status;

#ifdef EVKHIP_DECODE_TRACE
// Stage timestamps of one step and two consecutive layers (a separate trace
// build of the library, evk_amd/build.py --decode-trace): per layer,
// workgroup and stage kind S1..S5, the 100 MHz wall clock when the stage
// starts, when its input has arrived and when its outputs are stored.
constexpr int kTraceStep = 3, kTraceLayer = 2;  // layers kTraceLayer - 1 and kTraceLayer
__device__ unsigned long long g_dec_trace[2][1024][5][3];
#define DEC_TRACE(c, i)                                                                                     \
    do {                                                                                                    \
        if (threadIdx.x == 0 && (c).t == kTraceStep && ((c).l == kTraceLayer || (c).l == kTraceLayer - 1) && \
            (c).k < K_HEAD)                                                                                 \
            g_dec_trace[(c).l - kTraceLayer + 1][blockIdx.x][(c).k][(i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define DEC_TRACE(c, i) \
    do {                \
    } while (0)
#endif

struct PArgs {
    int d, H, dh, hid, V, L;
    int max_seq;
    float eps, rope_base;
    const f16* E;         // (V, d)
    const f16* lay;       // packed layers: WqkvT (3d,d), WoT (d,d), W1T (hid,d), W2T (d,hid)
    uint64_t per_layer;   // elements per packed layer
    const f16* WoutT;     // (V, d)
    f16* cache;           // per layer K (max_seq, d), V (max_seq, d)
    uint16_t* tok;        // token_io
    f16* logits;
    int n, pos0;
    uint64_t* mb;         // mailbox words
    uint32_t* ctl;        // [0] epoch base, [1] arrivals, [2] [3] wrap barrier count, generation
    int o_qkv, o_att, o_x1, o_gh, o_x2, par, o_cand, mb_words;
    int S_max;
    int G3, R3, G5, R5;
    int bufb;             // bytes of one LDS weight slot
    int hr;               // LM-head rows per slot
    int spin_limit;
};

// The thread index, opaque to the optimiser: values derived from it are
// formed where a stage uses them instead of being hoisted out of the step
// and layer loops (all stages' lane masks and offsets held at once exhaust
// the scalar and vector registers).
DEV int tid_now() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// A buffer descriptor from wave-uniform inputs, built in scalar registers
// (the DMA instructions take the descriptor only from there)
DEV __amdgpu_buffer_rsrc_t buf_rsrc_u(const void* base, uint32_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b), hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    return buf_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
DEV uint64_t mb_ld(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void mb_st(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV uint32_t pack2(float a, float b) { return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16); }
DEV float lo_h(uint32_t w) { return h2f((uint16_t)(w & 0xFFFFu)); }
DEV float hi_h(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
DEV half2v as_h2(uint32_t w) { return __builtin_bit_cast(half2v, w); }
// Sum over groups of L = 16, 32 or 64 lanes, complete in each group's last
// lane: DPP within rows of 16, then row_bcast:15 and row_bcast:31 (no LDS
// round trip, unlike a cross-row shuffle).
template <int L>
DEV float lanes_sum_last(float x) {
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
    if (L >= 32) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
    if (L >= 64) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x143, 0xC, 0xF, false));
    return x;
}
// the wave's sum, in every lane (wave-uniform)
DEV float wave_total(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lanes_sum_last<64>(x)), 63));
}
// the wave's maximum, in every lane (rows not in a row_bcast's mask keep x)
template <int CTL, int ROWS>
DEV float dpp_keep(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), CTL,
                                                                 ROWS, 0xF, false));
}
DEV float wave_maximum(float x) {
    x = fmaxf(x, dpp_keep<0xB1, 0xF>(x));
    x = fmaxf(x, dpp_keep<0x4E, 0xF>(x));
    x = fmaxf(x, dpp_keep<0x141, 0xF>(x));
    x = fmaxf(x, dpp_keep<0x140, 0xF>(x));
    x = fmaxf(x, dpp_keep<0x142, 0xA>(x));
    x = fmaxf(x, dpp_keep<0x143, 0xC>(x));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
// groups of L = 2, 4, 8 or 16 lanes, L uniform
DEV float group_sum(float x, int L) {
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
    if (L >= 4) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
    if (L >= 8) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
    if (L >= 16) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
    return x;
}
// groups of L = 1, 2, 4, ..., 64 lanes, L uniform
DEV float group_sum64(float x, int L) {
    if (L >= 2) x = group_sum(x, L);
    if (L >= 32) x += __shfl_xor(x, 16, 64);
    if (L >= 64) x += __shfl_xor(x, 32, 64);
    return x;
}
DEV float group_max64(float x, int L) {
    if (L >= 2) x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false)));
    if (L >= 4) x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false)));
    if (L >= 8) x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false)));
    if (L >= 16) x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false)));
    if (L >= 32) x = fmaxf(x, __shfl_xor(x, 16, 64));
    if (L >= 64) x = fmaxf(x, __shfl_xor(x, 32, 64));
    return x;
}

// Waits until words [0, n) of `box` carry `tag` and copies their payloads to
// dst[0, n) (LDS).  Called by the polling threads (tid < NPOLL); on timeout
// sets *s_fail.  The caller's next barrier publishes dst and the flag.
// A round requests all of a thread's words before it looks at any: volatile
// sc1 buffer loads (the compiler neither merges nor drops them, and issues
// them back to back; agent-scope atomic loads got a wait after each).  Each
// word is one naturally aligned 8-byte access, as the atomic load would be,
// so its tag and payload come from the same store.
// With SSQ, the waiting waves also form rms_norm's sum of squares of the
// words' fp16 values (clamped, rms_norm.comp): each thread over its own words
// in word order, then each wave's total into ssq[wave], so that the sum is
// the same on every run.
template <int NW, bool SSQ>  // words per thread and round: n <= NW * NPOLL
DEV void poll_n(const uint64_t* box, int n, uint32_t tag, uint32_t* dst, int limit, int* s_fail, float* ssq) {
    const int tid = tid_now();
    const __amdgpu_buffer_rsrc_t r = buf_rsrc_u(box, (uint32_t)n * 8u);
    uint32_t pend = 0;
#pragma unroll
    for (int u = 0; u < NW; ++u)
        if (tid + u * NPOLL < n) pend |= 1u << u;
    // Two rounds in flight: round r + 1 is requested before round r is looked
    // at, so a word is seen about half a load latency after it lands.  Every
    // round requests NW words (those past n read as zeros), so that the wait
    // for a round counts exactly the NW loads of the round after it.
    auto issue = [&](u32x2* w) {
        asm volatile("" ::: "memory");  // a new round: the words may have changed since the last one
#pragma unroll
        for (int u = 0; u < NW; ++u)
            w[u] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (uint32_t)tid * 8u,
                                                                              (uint32_t)(u * NPOLL * 8), 16 | (1 << 31)));
    };
    uint32_t val[NW];
#pragma unroll
    for (int u = 0; u < NW; ++u) val[u] = 0u;
    auto take = [&](const u32x2* w) {
#pragma unroll
        for (int u = 0; u < NW; ++u)
            if ((pend & (1u << u)) && w[u][1] == tag) {
                dst[tid + u * NPOLL] = w[u][0];
                if (SSQ) val[u] = w[u][0];
                pend &= ~(1u << u);
            }
    };
    u32x2 wa[NW], wb[NW];
    int it = 0;
    issue(wa);
    while (true) {
        issue(wb);
        take(wa);
        if (!__any(pend != 0) || ++it > limit) break;
        issue(wa);
        take(wb);
        if (!__any(pend != 0) || ++it > limit) break;
    }
    if (pend) *s_fail = 1;
    if (SSQ) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < NW; ++u) {  // words past n hold zero
            const half2v c = __builtin_elementwise_min(
                __builtin_elementwise_max(as_h2(val[u]), half2v{-65504.0f16, -65504.0f16}), half2v{65504.0f16, 65504.0f16});
            ss = __builtin_amdgcn_fdot2(c, c, ss, false);
        }
        ss = wave_total(ss);
        if ((tid & 63) == 0) ssq[tid >> 6] = ss;
    }
}
// ssq: see poll_n; given only for n <= 4 NPOLL
DEV void poll(const uint64_t* box, int n, uint32_t tag, uint32_t* dst, int limit, int* s_fail, float* ssq) {
    const int nw = (n + NPOLL - 1) / NPOLL;  // uniform
    if (ssq) {
        if (nw <= 2) poll_n<2, true>(box, n, tag, dst, limit, s_fail, ssq);
        else poll_n<4, true>(box, n, tag, dst, limit, s_fail, ssq);
    } else if (nw <= 1) {
        poll_n<1, false>(box, n, tag, dst, limit, s_fail, ssq);
    } else if (nw <= 2) {
        poll_n<2, false>(box, n, tag, dst, limit, s_fail, ssq);
    } else if (nw <= 4) {
        poll_n<4, false>(box, n, tag, dst, limit, s_fail, ssq);
    } else if (nw <= 8) {
        poll_n<8, false>(box, n, tag, dst, limit, s_fail, ssq);
    } else {
        poll_n<PMAXW, false>(box, n, tag, dst, limit, s_fail, ssq);
    }
}

// 16 bytes per lane from a buffer straight into LDS: lane i writes
// lds_base + 16 i.  Inline assembly, so that the compiler does not make the
// kernel's LDS reads wait for these loads; the streaming waves wait for them
// (vmcnt) before the barrier that publishes a slot.  M0 carries the LDS
// address; nothing else in this kernel keeps a value in M0.  sc1: read from
// the device coherence point (cache rows written during the launch).
typedef __attribute__((address_space(3))) void lds_void_t;
DEV uint32_t lds_u32(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void_t*)p);
}
DEV void dma16(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(res),
                 "s"(lds_base) : "memory");
}
DEV void dma16_sc1(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen sc1 lds" : : "v"(voff),
                 "s"(res), "s"(lds_base) : "memory");
}
// s_waitcnt vmcnt(m) for the largest listed m <= n (waiting for more loads
// than needed is always safe)
DEV void wait_vm_le(int n) {
#define EVK_VMW(v) if (n >= (v)) { __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | 0x0f70); return; }
    EVK_VMW(56) EVK_VMW(48) EVK_VMW(40) EVK_VMW(32) EVK_VMW(28) EVK_VMW(24) EVK_VMW(20) EVK_VMW(16)
    EVK_VMW(12) EVK_VMW(10) EVK_VMW(8) EVK_VMW(6) EVK_VMW(5) EVK_VMW(4) EVK_VMW(3) EVK_VMW(2) EVK_VMW(1)
#undef EVK_VMW
    __builtin_amdgcn_s_waitcnt(0x0f70);
}

// h = fp16(clamp(x) * inv) on a word of two fp16 values (rms_norm.comp's output)
DEV uint32_t norm_w(uint32_t w, float inv) {
    const float a = fminf(fmaxf(lo_h(w), -65504.0f), 65504.0f) * inv;
    const float b = fminf(fmaxf(hi_h(w), -65504.0f), 65504.0f) * inv;
    return pack2(a, b);
}

// out[row] = sum_k h[k] W[row][k] (fp32) for rows [0, nrows) of an LDS slice
// of (nrows, K) fp16 rows and an fp16 vector h (K / 2 words) in LDS; LPR lanes
// per row, all threads of the workgroup.  Products of fp16 pairs accumulate in
// fp32 (v_dot2_f32_f16).
// A lane takes chunks li + LPR j of 8 elements: j < full = k8n / LPR, then
// the partial last column (li < k8n % LPR).  Passes of KC chunks are issued
// before their first product, with a trip count fixed at compile time, which
// keeps the loads unmasked; the partial column's load goes out first.
template <int LPR, int KC>
DEV void dot_rows(const f16* W, int K, int nrows, const uint32_t* h, float* out) {
    const int tid = tid_now(), slot = tid / LPR, li = tid % LPR;
    constexpr int NS = PNT / LPR;
    const int k8n = K / 8, full = k8n / LPR, tail = full * LPR + li;
    auto dot4 = [&](float acc, u32x4v x, u32x4v y) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            acc = __builtin_amdgcn_fdot2(as_h2(x[e]), as_h2(y[e]), acc, false);
        return acc;
    };
    for (int r0 = 0; r0 < nrows; r0 += NS) {
        const int row = r0 + slot;
        float acc = 0.0f;
        if (row < nrows) {
            const f16* wr = W + (int64_t)row * K;
            u32x4v xt = u32x4v{0u, 0u, 0u, 0u}, yt = u32x4v{0u, 0u, 0u, 0u};
            if (tail < k8n) {
                xt = *reinterpret_cast<const u32x4v*>(wr + tail * 8);
                yt = *reinterpret_cast<const u32x4v*>(h + tail * 4);
            }
            int j0 = 0;
            for (; j0 + KC <= full; j0 += KC) {
                u32x4v x[KC], y[KC];
#pragma unroll
                for (int u = 0; u < KC; ++u) {
                    x[u] = *reinterpret_cast<const u32x4v*>(wr + (li + (j0 + u) * LPR) * 8);
                    y[u] = *reinterpret_cast<const u32x4v*>(h + (li + (j0 + u) * LPR) * 4);
                }
#pragma unroll
                for (int u = 0; u < KC; ++u) acc = dot4(acc, x[u], y[u]);
            }
            for (; j0 < full; ++j0)
                acc = dot4(acc, *reinterpret_cast<const u32x4v*>(wr + (li + j0 * LPR) * 8),
                           *reinterpret_cast<const u32x4v*>(h + (li + j0 * LPR) * 4));
            acc = dot4(acc, xt, yt);
        }
        acc = lanes_sum_last<LPR>(acc);
        if (li == LPR - 1 && row < nrows) out[row] = acc;
    }
}
template <int LPR>
DEV void dot_lds(const f16* W, int K, int nrows, const uint32_t* h, float* out) {
    static_assert(LPR == 16 || LPR == 32 || LPR == 64, "lanes per row");
    switch ((K / 8) / LPR) {  // uniform; the common counts, larger ones in passes of 8
        case 0:
        case 1: dot_rows<LPR, 1>(W, K, nrows, h, out); break;
        case 2: dot_rows<LPR, 2>(W, K, nrows, h, out); break;
        case 3: dot_rows<LPR, 3>(W, K, nrows, h, out); break;
        case 4: dot_rows<LPR, 4>(W, K, nrows, h, out); break;
        case 6: dot_rows<LPR, 6>(W, K, nrows, h, out); break;
        default: dot_rows<LPR, 8>(W, K, nrows, h, out); break;
    }
}

// 1 / sqrt(mean(clamp(x)^2) + eps) over the fp16 vector x (K / 2 words in
// LDS; rms_norm.comp), in every thread: each wave sums all of x itself (no
// barrier).  K is a multiple of 8.
DEV float rms_inv(const uint32_t* x, int K, float eps) {
    const int lane = tid_now() & 63;
    const int k8n = K / 8, full = k8n / 64, tail = full * 64 + lane;
    float ss = 0.0f;
    // packed: clamp two fp16 values at once, then both squares into fp32
    // (v_pk_min/max_f16, v_dot2_f32_f16)
    auto acc4 = [&](u32x4v v) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const half2v c = __builtin_elementwise_min(__builtin_elementwise_max(as_h2(v[e]), half2v{-65504.0f16, -65504.0f16}),
                                                       half2v{65504.0f16, 65504.0f16});
            ss = __builtin_amdgcn_fdot2(c, c, ss, false);
        }
    };
    u32x4v vt = u32x4v{0u, 0u, 0u, 0u};
    if (tail < k8n) vt = *reinterpret_cast<const u32x4v*>(x + tail * 4);
    int j0 = 0;
    for (; j0 + 4 <= full; j0 += 4) {
        u32x4v v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const u32x4v*>(x + (lane + (j0 + u) * 64) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc4(v[u]);
    }
    for (; j0 < full; ++j0) acc4(*reinterpret_cast<const u32x4v*>(x + (lane + j0 * 64) * 4));
    acc4(vt);
    return 1.0f / sqrtf(wave_total(ss) / (float)K + eps);
}

// hn = rms_norm(x) (fp16 words, rms_norm.comp) for the dots that follow;
// the caller's barrier publishes it.
DEV void rms_norm_words(const uint32_t* x, uint32_t* hn, int K, float eps) {
    const float inv = rms_inv(x, K, eps);
    for (int i = tid_now(); i < K / 2; i += PNT) hn[i] = norm_w(x[i], inv);
}
// the same from the four polling waves' sums of squares (poll_n with SSQ)
DEV void rms_norm_words_ssq(const uint32_t* x, uint32_t* hn, int K, float eps, const float* ssq) {
    const float ss = ((ssq[0] + ssq[1]) + ssq[2]) + ssq[3];
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    for (int i = tid_now(); i < K / 2; i += PNT) hn[i] = norm_w(x[i], inv);
}

// The greedy winner of the workgroup's (value, rank) pairs, in every thread.
DEV void block_best(float& bv, uint32_t& br, float* sv, uint32_t* sr) {
    const int tid = tid_now();
    // the order is total, so exchanges within quads, half rows and rows (DPP)
    // and then across rows leave the wave's best in every lane
    auto take = [&](float v2, uint32_t r2) {
        if (greedy_better(v2, r2, bv, br)) {
            bv = v2;
            br = r2;
        }
    };
#define EVK_DPP_TAKE(ctl)                                                                               \
    take(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, bv), ctl, 0xF, 0xF, false)), \
         (uint32_t)__builtin_amdgcn_update_dpp(0, (int)br, ctl, 0xF, 0xF, false))
    EVK_DPP_TAKE(0xB1);
    EVK_DPP_TAKE(0x4E);
    EVK_DPP_TAKE(0x141);
    EVK_DPP_TAKE(0x140);
#undef EVK_DPP_TAKE
    take(__shfl_xor(bv, 16, 64), __shfl_xor(br, 16, 64));
    take(__shfl_xor(bv, 32, 64), __shfl_xor(br, 32, 64));
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        sr[tid >> 6] = br;
    }
    __syncthreads();
    bv = sv[0];
    br = sr[0];
#pragma unroll
    for (int w = 1; w < PWV; ++w)
        if (greedy_better(sv[w], sr[w], bv, br)) {
            bv = sv[w];
            br = sr[w];
        }
    __syncthreads();
}

// LDS floats of the stage input: the longer input vector, or the attention's
// per-key-slot partial outputs
DEV_HOST_INLINE int hs_floats(int d, int hid, int dh) {
    const int m = d > hid ? d : hid;
    return ((m > PNT * 8 ? m : PNT * 8) + 3) & ~3;  // attention: (512 / (dh/8)) key slots x dh
}

// Stage kinds of a workgroup's sequence
enum { K_S1 = 0, K_S2 = 1, K_S3 = 2, K_S4 = 3, K_S5 = 4, K_HEAD = 5 };
struct Cur {
    int t, l, k, sub;  // step, layer, kind, LM-head slot
};

__global__ __launch_bounds__(PNT) void decode_persist(PArgs a) {
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    const int d = a.d, hid = a.hid, H = a.H, dh = a.dh, G = (int)gridDim.x, wid = (int)blockIdx.x;
    f16* ring = reinterpret_cast<f16*>(lds);                      // NBUF slots of bufb bytes
    uint32_t* xw = reinterpret_cast<uint32_t*>(lds + NBUF * a.bufb);  // d fp16: the residual stream x
    float* hs = reinterpret_cast<float*>(xw) + ((d + 3) & ~3);          // attention scratch (fp32)
    uint32_t* hw = reinterpret_cast<uint32_t*>(hs);                     // or a stage's fp16 input h
    float* yo = hs + hs_floats(d, hid, dh);                       // YO: stage outputs
    float* red = yo + YO;                                         // 64: reductions
    uint32_t* mbuf = reinterpret_cast<uint32_t*>(red + 64);      // polled payloads
    __shared__ int s_fail;
    __shared__ uint32_t s_tok;
    __shared__ float s_v[PWV];
    __shared__ uint32_t s_r[PWV];
    if (threadIdx.x == 0) s_fail = 0;

    auto fail = [&]() {
        if (threadIdx.x == 0)
            __hip_atomic_fetch_or(&g_dec_status, (unsigned)EVKHIP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    };

    // ---- epoch base ----
    // Every workgroup reads the base, then arrives on ctl[1]; the last to
    // arrive (all have read the base by then) resets the count and moves the
    // base past this launch's tags, so that the next launch (a graph replay
    // of this one, or a launch after one that gave up) uses new tags.  On the
    // rare wrap of the tags the mailboxes are cleared first, behind a
    // generation barrier on ctl[2] (count) and ctl[3] (generation).
    const int SPT = 5 * a.L + 1;
    const uint32_t need = (uint32_t)a.n * (uint32_t)SPT + 2u;
    uint32_t base = __hip_atomic_load(&a.ctl[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (base >= kWrapAt - need) {
        for (int i = wid * PNT + (int)threadIdx.x; i < a.mb_words; i += G * PNT) mb_st(a.mb + i, 0u, 0u);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t gen = __hip_atomic_load(&a.ctl[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);  // the generation is read before this arrival counts
            if (__hip_atomic_fetch_add(&a.ctl[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)G - 1u) {
                __hip_atomic_store(&a.ctl[2], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);
                __hip_atomic_store(&a.ctl[3], gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                int it = 0;
                while (__hip_atomic_load(&a.ctl[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
                    if (++it > a.spin_limit) {
                        s_fail = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
        }
        __syncthreads();
        base = 0u;
    }
    // every workgroup arrives, also one that gave up at the wrap barrier:
    // a partial count would make the first arrival of a later launch look
    // like the last one
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(&a.ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)G - 1u) {
        __hip_atomic_store(&a.ctl[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&a.ctl[0], base + need, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (s_fail) {
        fail();
        return;
    }
    auto tag_of = [&](int t, int k) { return base + 1u + (uint32_t)t * (uint32_t)SPT + (uint32_t)k; };
    const int HEAD = 5 * a.L;

    // this workgroup's columns of each stage
    const int np1 = 3 * d / 2, np4 = hid / 2;
    const int p1_lo = (int)((int64_t)wid * np1 / G), p1_hi = (int)((int64_t)(wid + 1) * np1 / G);
    const int p4_lo = (int)((int64_t)wid * np4 / G), p4_hi = (int)((int64_t)(wid + 1) * np4 / G);
    const int v_lo = (int)((int64_t)wid * a.V / G), v_hi = (int)((int64_t)(wid + 1) * a.V / G);
    const int nhead = (v_hi - v_lo + a.hr - 1) / a.hr;  // LM-head slots
    // Wo on the last G3 workgroups (the attention ones are the first H * S)
    const int w3 = wid - (G - a.G3), r3_lo = w3 * a.R3, r3_n = w3 >= 0 ? min(a.R3, d - r3_lo) : 0;
    const int r5_lo = wid * a.R5, r5_n = wid < a.G5 ? min(a.R5, d - r5_lo) : 0;
    const float att_scale = 1.0f / sqrtf((float)dh);
    const int PPK = dh / 8;                   // 16-byte pieces per key row
    const int ablk = dh / 2 + 2;              // words of one (head, split) partial
    auto splits = [&](int t) { return (a.pos0 + t + 1 + KSPL - 1) / KSPL; };

    // ---- this workgroup's sequence of stages ----
    auto takes = [&](const Cur& c) {
        switch (c.k) {
            case K_S2: return wid < H * splits(c.t);
            case K_S3: return r3_n > 0;
            case K_S5: return r5_n > 0;
            default: return true;
        }
    };
    auto step = [&](Cur c) {  // the next stage of the whole model
        if (c.k == K_HEAD) {
            if (c.sub + 1 < nhead) return Cur{c.t, c.l, K_HEAD, c.sub + 1};
            return Cur{c.t + 1, 0, K_S1, 0};
        }
        if (c.k < K_S5) return Cur{c.t, c.l, c.k + 1, 0};
        if (c.l + 1 < a.L) return Cur{c.t, c.l + 1, K_S1, 0};
        return Cur{c.t, c.l, K_HEAD, 0};
    };
    auto next = [&](Cur c) {  // the next stage this workgroup takes part in
        do c = step(c);
        while (c.t < a.n && !takes(c));
        return c;
    };

    // ---- streaming: the weight slice (or the split's cached K, V rows) of a
    // stage into a ring slot, by waves 4-7; returns this wave's load count ----
    auto stream = [&](const Cur& c, f16* slot) -> int {
        if (c.t >= a.n) return 0;
        const int tid = tid_now(), lane = tid & 63;
        const int sw = __builtin_amdgcn_readfirstlane((tid >> 6) - NPOLL / 64);  // streaming wave 0..3
        const f16* lw = a.lay + (uint64_t)c.l * a.per_layer;
        const f16* src = nullptr;
        int bytes = 0;
        if (c.k == K_S2) {
            const int pos = a.pos0 + c.t, S = splits(c.t), h = wid / S, s = wid % S;
            const int per = (pos + 1 + S - 1) / S;
            const int k_lo = s * per, kc_hi = min(min(pos + 1, k_lo + per), pos);
            const int nk = max(0, kc_hi - k_lo);
            const f16* Kc = a.cache + (uint64_t)c.l * 2 * a.max_seq * d;
            const f16* Vc = Kc + (uint64_t)a.max_seq * d;
            // rows [0, kc_hi) of the cache; a 1 KB load covers 1024 / (2 dh) keys
            const __amdgpu_buffer_rsrc_t kres = buf_rsrc_u(Kc, (uint32_t)kc_hi * (uint32_t)d * 2u);
            const __amdgpu_buffer_rsrc_t vres = buf_rsrc_u(Vc, (uint32_t)kc_hi * (uint32_t)d * 2u);
            const int kpi = 64 / PPK, nq = (nk + kpi - 1) / kpi;
            int cnt = 0;
            for (int q = sw; q < nq; q += 4) {
                const int key = k_lo + q * kpi + lane / PPK;
                const uint32_t off = oob_or(key < kc_hi, (uint32_t)(key * d + h * dh + (lane % PPK) * 8) * 2u);
                dma16_sc1(kres, off, lds_u32(slot + q * 512));
                dma16_sc1(vres, off, lds_u32(slot + KSPL * dh + q * 512));
                cnt += 2;
            }
            return cnt;
        }
        switch (c.k) {
            case K_S1: src = lw + (uint64_t)2 * p1_lo * d; bytes = 2 * (p1_hi - p1_lo) * d * 2; break;
            case K_S3: src = lw + (uint64_t)3 * d * d + (uint64_t)r3_lo * d; bytes = r3_n * d * 2; break;
            case K_S4: src = lw + (uint64_t)4 * d * d + (uint64_t)2 * p4_lo * d; bytes = 2 * (p4_hi - p4_lo) * d * 2; break;
            case K_S5:
                src = lw + (uint64_t)4 * d * d + (uint64_t)hid * d + (uint64_t)r5_lo * hid;
                bytes = r5_n * hid * 2;
                break;
            default: {
                const int r0 = v_lo + c.sub * a.hr, nr = min(a.hr, v_hi - r0);
                src = a.WoutT + (uint64_t)r0 * d;
                bytes = nr * d * 2;
            }
        }
        const __amdgpu_buffer_rsrc_t res = buf_rsrc_u(src, (uint32_t)bytes);
        int cnt = 0;
        for (int q = sw; q * 1024 < bytes; q += 4) {
            dma16(res, (uint32_t)(q * 1024 + lane * 16), lds_u32(slot + q * 512));
            ++cnt;
        }
        return cnt;
    };

    const bool streamer = (int)threadIdx.x >= NPOLL;
    // rms_norm's sums of squares formed by the polls of x (up to 4 words a poller)
    const bool ssq_poll = d / 2 <= 4 * NPOLL;
    static_assert(NPOLL == 4 * 64, "four polling waves");
    Cur cur{0, 0, K_S1, 0};
    Cur c1 = next(cur), c2 = next(c1);
    // this wave's loads of the stage, the next one and the one after
    int n0 = 0, n1 = 0, n2 = 0;
    if (streamer) {
        n0 = stream(cur, ring);
        n1 = stream(c1, ring + (a.bufb / 2));
    }
    float hbv = -3.402823466e+38f;  // LM head: this thread's candidate over the step's slots
    uint32_t hbr = 0u;
    float rcs = 1.0f, rsn = 0.0f;  // this thread's rotary pair at the step's position (q, k columns)

#pragma unroll 1
    for (int si = 0; cur.t < a.n; ++si) {
        const int b0 = si % NBUF;
        f16* W = ring + (size_t)b0 * (a.bufb / 2);
        // the stage two ahead into the slot the previous stage used
        if (streamer) n2 = stream(c2, ring + (size_t)((si + 2) % NBUF) * (a.bufb / 2));
        const int t = cur.t, l = cur.l, p = l & 1, k0 = l * 5, pos = a.pos0 + t;
        const int S = splits(t);
        DEC_TRACE(cur, 0);
        // ---- the stage's input ----
        if (!streamer) {
            // the stage's input words (one poll call site keeps the kernel's code small)
            const uint64_t* box = nullptr;
            int nw = 0;
            uint32_t tg = 0;
            uint32_t* dst = mbuf;
            float* sq = nullptr;  // rms_norm's sum of squares of x, formed while polling
            switch (cur.k) {
                case K_S1:
                    if (l > 0) {
                        box = a.mb + a.o_x2 + (p ^ 1) * a.par, nw = d / 2, tg = tag_of(t, k0 - 1), dst = xw;
                        sq = ssq_poll ? red + RSQ : nullptr;
                    } else if (t > 0) {
                        box = a.mb + a.o_cand, nw = 2 * G, tg = tag_of(t - 1, HEAD);
                    }
                    break;
                case K_S2: {
                    const int h = wid / S, s = wid % S;
                    const int per = (pos + 1 + S - 1) / S;
                    // the head's q (and, for the split that takes key pos, its new k, v)
                    const bool has_new = min(pos + 1, s * per + per) == pos + 1;
                    box = a.mb + a.o_qkv + p * a.par + h * (3 * dh / 2), nw = has_new ? 3 * dh / 2 : dh / 2;
                    tg = tag_of(t, k0);
                    break;
                }
                case K_S3: box = a.mb + a.o_att + p * a.par, nw = S * H * ablk, tg = tag_of(t, k0 + 1); break;
                case K_S4:
                    box = a.mb + a.o_x1 + p * a.par, nw = d / 2, tg = tag_of(t, k0 + 2), dst = xw;
                    sq = ssq_poll ? red + RSQ : nullptr;
                    break;
                case K_S5: box = a.mb + a.o_gh + p * a.par, nw = hid / 2, tg = tag_of(t, k0 + 3), dst = hw; break;
                default:
                    if (cur.sub == 0) {
                        box = a.mb + a.o_x2 + ((a.L - 1) & 1) * a.par, nw = d / 2, tg = tag_of(t, HEAD - 1), dst = xw;
                        sq = ssq_poll ? red + RSQ : nullptr;
                    }
            }
            if (nw > 0) poll(box, nw, tg, dst, a.spin_limit, &s_fail, sq);
        } else {
            // this stage's slice is in LDS once only the two later ones are in flight
            wait_vm_le(n1 + n2);
        }
        __syncthreads();
        if (s_fail) {
            fail();
            return;
        }
        DEC_TRACE(cur, 1);
        const int tid = tid_now(), lane = tid & 63, wave = tid >> 6;

        // ---- the stage ----
        if (cur.k == K_S1) {
            if (l == 0) {
                // the step's token: the previous step's candidates, or token_io[0]
                if (tid == 0) {
                    uint32_t tk = a.tok[0];
                    s_tok = tk;
                }
                if (t > 0) {
                    float bv = -3.402823466e+38f;
                    uint32_t br = 0u;
                    for (int i = tid; i < G; i += PNT) {
                        const float v = __builtin_bit_cast(float, mbuf[2 * i]);
                        const uint32_t r = mbuf[2 * i + 1];
                        if (greedy_better(v, r, bv, br)) {
                            bv = v;
                            br = r;
                        }
                    }
                    block_best(bv, br, s_v, s_r);
                    if (tid == 0) {
                        s_tok = greedy_index(br);
                        if (wid == 0) a.tok[t] = (uint16_t)s_tok;
                    }
                }
                __syncthreads();
                const f16* er = a.E + (int64_t)min((int)s_tok, a.V - 1) * d;
                if (!streamer)  // the streaming waves keep their loads for the slices
                    for (int i = tid; i < d / 2; i += NPOLL) xw[i] = reinterpret_cast<const uint32_t*>(er)[i];
                __syncthreads();
            }  // (otherwise the poll wrote x to xw)
            if (l > 0 && ssq_poll) rms_norm_words_ssq(xw, hw, d, a.eps, red + RSQ);
            else rms_norm_words(xw, hw, d, a.eps);
            __syncthreads();
            dot_lds<32>(W, d, 2 * (p1_hi - p1_lo), hw, yo);
            __syncthreads();
            const uint32_t tg = tag_of(t, k0);
            if (tid < p1_hi - p1_lo) {
                f16* Kc = a.cache + (uint64_t)l * 2 * a.max_seq * d;
                f16* Vc = Kc + (uint64_t)a.max_seq * d;
                const int col = 2 * (p1_lo + tid), which = col / d, c = col % d;
                float y0 = (float)(f16)yo[2 * tid], y1 = (float)(f16)yo[2 * tid + 1];
                if (which < 2) {
                    // the column range is the same in every layer: the angle once per step
                    if (cur.l == 0) {
                        const float inv_freq = powf(a.rope_base, -2.0f * (float)((c % dh) / 2) / (float)dh);
                        sincosf((float)pos * inv_freq, &rsn, &rcs);
                    }
                    const float r0 = y0 * rcs - y1 * rsn, r1 = y0 * rsn + y1 * rcs;
                    y0 = r0;
                    y1 = r1;
                }
                const uint32_t w = pack2(y0, y1);
                // per head: q, k, v words back to back
                mb_st(a.mb + a.o_qkv + p * a.par + (c / dh) * (3 * dh / 2) + which * (dh / 2) + (c % dh) / 2, tg, w);
                if (which > 0) {
                    // this step's attention takes k, v of pos from the mailbox; the
                    // cache row (written through) is read from the next step on.
                    // This wave's next poll waits for all of its stores (vmcnt
                    // counts stores), so the row is complete before any word the
                    // wave writes after it, and before the next step starts.
                    f16* row = (which == 1 ? Kc : Vc) + (int64_t)pos * d + c;
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(row), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        } else if (cur.k == K_S2) {
            // attention of head h over key split s; the split's cached K and V rows
            // are in W ([key][dh] each, rows past the cached ones unused).  Wave w
            // scores keys 16w..16w+15 (four lanes a key, dh/4 dimensions a lane)
            // and forms its own softmax partial (m_w, l_w, o_w) with its lanes on
            // the output dimensions; after one barrier the lanes of wave 0 merge
            // the eight partials and the new key's term and store the block.
            const int h = wid / S, s = wid % S;
            const int per = (pos + 1 + S - 1) / S;
            const int k_lo = s * per, k_hi = min(pos + 1, k_lo + per), kc_hi = min(k_hi, pos);
            const bool has_new = k_hi == pos + 1;
            const int nk = max(0, kc_hi - k_lo);  // cached keys of the split
            const f16* Ks = W;
            const f16* Vs = W + KSPL * dh;
            const float c2 = att_scale * 1.4426950408889634f;  // scores in the base-2 domain
            const int kb = (KSPL / PWV) * wave, kl = kb + (lane >> 2), part = lane & 3, dq = dh / 4;
            float sc = 0.0f;
            {
                const f16* kr = Ks + kl * dh + part * dq;
                const uint32_t* qw = mbuf + part * (dq / 2);
                if (dq >= 8) {
                    u32x4v kk[4], qq[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int jj = j < dq / 8 ? j : 0;
                        kk[j] = *reinterpret_cast<const u32x4v*>(kr + 8 * jj);
                        qq[j] = *reinterpret_cast<const u32x4v*>(qw + 4 * jj);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float dj = 0.0f;
#pragma unroll
                        for (int e = 0; e < 4; ++e) dj = __builtin_amdgcn_fdot2(as_h2(qq[j][e]), as_h2(kk[j][e]), dj, false);
                        sc += j < dq / 8 ? dj : 0.0f;
                    }
                } else {  // dh = 16: four dimensions a lane
                    const uint2 kk = *reinterpret_cast<const uint2*>(kr);
                    sc = __builtin_amdgcn_fdot2(as_h2(qw[0]), as_h2(kk.x), 0.0f, false);
                    sc = __builtin_amdgcn_fdot2(as_h2(qw[1]), as_h2(kk.y), sc, false);
                }
            }
            sc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sc), 0xB1, 0xF, 0xF, false));
            sc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sc), 0x4E, 0xF, 0xF, false));
            const bool live = kl < nk;
            sc = live ? sc * c2 : -INFINITY;
            const float mw = wave_maximum(sc);
            const float pk = live ? __builtin_amdgcn_exp2f(sc - mw) : 0.0f;
            const float lw = wave_total(part == 0 ? pk : 0.0f);
            // p . v over the wave's keys: lane on dimension lane (dh <= 64) or on
            // dimensions 2 lane, 2 lane + 1 (dh = 128); each key's p from its lanes
            float o0 = 0.0f, o1 = 0.0f;
            if (dh == 128) {
                uint32_t vv[KSPL / PWV];
#pragma unroll
                for (int k = 0; k < KSPL / PWV; ++k) vv[k] = *reinterpret_cast<const uint32_t*>(Vs + (kb + k) * dh + 2 * lane);
#pragma unroll
                for (int k = 0; k < KSPL / PWV; ++k) {
                    const float pkk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pk), 4 * k));
                    const bool kv = kb + k < nk;
                    o0 = __builtin_fmaf(pkk, kv ? lo_h(vv[k]) : 0.0f, o0);
                    o1 = __builtin_fmaf(pkk, kv ? hi_h(vv[k]) : 0.0f, o1);
                }
            } else {
                const int dl = lane < dh ? lane : 0;
                f16 vv[KSPL / PWV];
#pragma unroll
                for (int k = 0; k < KSPL / PWV; ++k) vv[k] = Vs[(kb + k) * dh + dl];
#pragma unroll
                for (int k = 0; k < KSPL / PWV; ++k) {
                    const float pkk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pk), 4 * k));
                    o0 = __builtin_fmaf(pkk, kb + k < nk ? (float)vv[k] : 0.0f, o0);
                }
            }
            float* ow = hs;  // [PWV][dh] partial outputs
            const int d0 = dh == 128 ? 2 * lane : lane;
            if (lane == 0) {
                red[wave] = mw;
                red[PWV + wave] = lw;
            }
            if (lane < dh) ow[wave * dh + d0] = o0;
            if (dh == 128) ow[wave * dh + d0 + 1] = o1;
            // the new key's score (q . k of pos), in every wave
            float s_new = -INFINITY;
            if (has_new) {
                float acc = 0.0f;
                if (lane < dh) acc = (d0 & 1 ? hi_h(mbuf[d0 / 2]) : lo_h(mbuf[d0 / 2])) *
                                     (d0 & 1 ? hi_h(mbuf[dh / 2 + d0 / 2]) : lo_h(mbuf[dh / 2 + d0 / 2]));
                if (dh == 128) acc += hi_h(mbuf[d0 / 2]) * hi_h(mbuf[dh / 2 + d0 / 2]);
                s_new = wave_total(acc) * c2;
            }
            __syncthreads();
            if (tid < min(dh, 64)) {
                // every partial requested at once, then trees (no serial chains)
                float mw8[PWV], lw8[PWV], oa[PWV], ob[PWV];
#pragma unroll
                for (int w = 0; w < PWV; ++w) {
                    mw8[w] = red[w];
                    lw8[w] = red[PWV + w];
                    oa[w] = ow[w * dh + d0];
                    ob[w] = dh == 128 ? ow[w * dh + d0 + 1] : 0.0f;
                }
                float mm[PWV];
#pragma unroll
                for (int w = 0; w < PWV; ++w) mm[w] = lw8[w] > 0.0f ? mw8[w] : -INFINITY;
                const float M = fmaxf(fmaxf(fmaxf(fmaxf(mm[0], mm[1]), fmaxf(mm[2], mm[3])),
                                            fmaxf(fmaxf(mm[4], mm[5]), fmaxf(mm[6], mm[7]))),
                                      s_new);
                float lf[PWV], af[PWV], bf[PWV];
#pragma unroll
                for (int w = 0; w < PWV; ++w) {
                    const float f = lw8[w] > 0.0f ? __builtin_amdgcn_exp2f(mw8[w] - M) : 0.0f;
                    lf[w] = lw8[w] * f;
                    af[w] = f * oa[w];
                    bf[w] = f * ob[w];
                }
                auto tree = [](const float* v) {
                    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                };
                static_assert(PWV == 8, "eight waves");
                float l = tree(lf), a0 = tree(af), a1 = tree(bf);
                if (has_new) {
                    const float pn = __builtin_amdgcn_exp2f(s_new - M);
                    const uint32_t vw = mbuf[dh + d0 / 2];
                    a0 = __builtin_fmaf(pn, d0 & 1 ? hi_h(vw) : lo_h(vw), a0);
                    if (dh == 128) a1 = __builtin_fmaf(pn, hi_h(vw), a1);
                    l += pn;
                }
                const float r0 = l > 0.0f ? a0 / l : 0.0f, r1 = l > 0.0f ? a1 / l : 0.0f;
                uint64_t* blk = a.mb + a.o_att + p * a.par + (s * H + h) * ablk;
                const uint32_t tg = tag_of(t, k0 + 1);
                if (dh == 128) {
                    mb_st(blk + 2 + tid, tg, pack2(r0, r1));
                } else {
                    // dimension pairs: the odd lane's value to its even neighbour
                    const float nb = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, r0), 0xB1, 0xF, 0xF, false));
                    if (!(tid & 1)) mb_st(blk + 2 + tid / 2, tg, pack2(r0, nb));
                }
                if (tid == 0) {
                    mb_st(blk, tg, __builtin_bit_cast(uint32_t, M * 0.6931471805599453f));  // natural-log maximum
                    mb_st(blk + 1, tg, __builtin_bit_cast(uint32_t, l));
                }
            }
        } else if (cur.k == K_S3) {
            // merge the splits; x1 = x + attn . Wo.  Split s of head h weighs
            // l_s e^(m_s - M_h) / sum over the head's splits (one exponential per
            // (head, split), in red2 = yo); then each element is a weighted sum.
            float* wts = yo;  // H * S <= YO weights
            {
                // thread (head hh, split ss) at hh * SG + ss, SG = the power of
                // two >= S (H * SG <= 2 H S_max <= PNT); every thread takes
                // part in the group reductions
                int SG = 1;
                while (SG < S) SG <<= 1;
                const int hh = tid / SG, ss = tid % SG;
                const bool ok = hh < H && ss < S;
                const uint32_t* b = mbuf + (ok ? ss * H + hh : 0) * ablk;
                const float ms = __builtin_bit_cast(float, b[0]), ls = __builtin_bit_cast(float, b[1]);
                const bool live = ok && ls > 0.0f;
                const float M = group_max64(live ? ms : -INFINITY, SG);
                const float w = live ? ls * __builtin_amdgcn_exp2f((ms - M) * 1.4426950408889634f) : 0.0f;
                const float den = group_sum64(w, SG);
                if (ok) wts[ss * H + hh] = den > 0.0f ? w * (1.0f / den) : 0.0f;
            }
            __syncthreads();
            // word cw = columns 2cw, 2cw + 1 (one head): sum over the splits,
            // eight splits' words requested at a time
            for (int cw = tid; cw < d / 2; cw += PNT) {
                const int h = (2 * cw) / dh, jw = ((2 * cw) % dh) / 2;
                float n0 = 0.0f, n1 = 0.0f;
                for (int s0 = 0; s0 < S; s0 += 8) {
                    uint32_t ow[8];
                    float wv[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int s2 = min(s0 + u, S - 1);
                        ow[u] = mbuf[(s2 * H + h) * ablk + 2 + jw];
                        wv[u] = wts[s2 * H + h];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float wu = s0 + u < S ? wv[u] : 0.0f;
                        n0 = __builtin_fmaf(wu, lo_h(ow[u]), n0);
                        n1 = __builtin_fmaf(wu, hi_h(ow[u]), n1);
                    }
                }
                hw[cw] = pack2(n0, n1);
            }
            __syncthreads();
            dot_lds<32>(W, d, r3_n, hw, yo);
            __syncthreads();
            if (tid < r3_n / 2) {
                const int c = r3_lo + 2 * tid;
                const float x0 = (float)(f16)(lo_h(xw[c / 2]) + (float)(f16)yo[2 * tid]);
                const float x1 = (float)(f16)(hi_h(xw[c / 2]) + (float)(f16)yo[2 * tid + 1]);
                mb_st(a.mb + a.o_x1 + p * a.par + c / 2, tag_of(t, k0 + 2), pack2(x0, x1));
            }
        } else if (cur.k == K_S4) {
            // x1 (in xw from the poll), rms_norm, gelu(h . W1)
            if (ssq_poll) rms_norm_words_ssq(xw, hw, d, a.eps, red + RSQ);
            else rms_norm_words(xw, hw, d, a.eps);
            __syncthreads();
            dot_lds<32>(W, d, 2 * (p4_hi - p4_lo), hw, yo);
            __syncthreads();
            if (tid < p4_hi - p4_lo) {
                const float g0 = gelu_f((float)(f16)yo[2 * tid]), g1 = gelu_f((float)(f16)yo[2 * tid + 1]);
                mb_st(a.mb + a.o_gh + p * a.par + p4_lo + tid, tag_of(t, k0 + 3), pack2(g0, g1));
            }
        } else if (cur.k == K_S5) {
            // x2 = x1 + gelu . W2 (gelu in hw from the poll)
            dot_lds<64>(W, hid, r5_n, hw, yo);
            __syncthreads();
            if (tid < r5_n / 2) {
                const int c = r5_lo + 2 * tid;
                const float x0 = (float)(f16)(lo_h(xw[c / 2]) + (float)(f16)yo[2 * tid]);
                const float x1 = (float)(f16)(hi_h(xw[c / 2]) + (float)(f16)yo[2 * tid + 1]);
                mb_st(a.mb + a.o_x2 + p * a.par + c / 2, tag_of(t, k0 + 4), pack2(x0, x1));
            }
        } else {
            // LM head slot: logits of rows [r0, r0 + nr); the step's candidate
            // after the last slot
            if (cur.sub == 0) {  // x2 in xw from the poll; hw keeps rms_norm(x2) over the slots
                if (ssq_poll) rms_norm_words_ssq(xw, hw, d, a.eps, red + RSQ);
                else rms_norm_words(xw, hw, d, a.eps);
                __syncthreads();
                hbv = -3.402823466e+38f;
                hbr = 0u;
            }
            const int r0 = v_lo + cur.sub * a.hr, nr = min(a.hr, v_hi - r0);
            dot_lds<32>(W, d, nr, hw, yo);
            __syncthreads();
            if (tid < nr) {
                const f16 lg = (f16)yo[tid];
                a.logits[r0 + tid] = lg;
                const float v = (float)lg;
                const uint32_t r = greedy_rank((uint32_t)(r0 + tid));
                if (v > -3.402823466e+38f && greedy_better(v, r, hbv, hbr)) {
                    hbv = v;
                    hbr = r;
                }
            }
            if (cur.sub + 1 == nhead) {
                float bv = hbv;
                uint32_t br = hbr;
                block_best(bv, br, s_v, s_r);
                if (tid == 0) {
                    const uint32_t tg = tag_of(t, HEAD);
                    mb_st(a.mb + a.o_cand + 2 * wid, tg, __builtin_bit_cast(uint32_t, bv));
                    mb_st(a.mb + a.o_cand + 2 * wid + 1, tg, br);
                }
            }
        }
        __syncthreads();  // the slot, mbuf and yo are reused by the next stages
        DEC_TRACE(cur, 2);
        cur = c1;
        c1 = c2;
        c2 = next(c2);
        n0 = n1;
        n1 = n2;
    }

    // ---- the last step's token ----
    if (wid == 0) {
        if (!streamer) poll(a.mb + a.o_cand, 2 * G, tag_of(a.n - 1, HEAD), mbuf, a.spin_limit, &s_fail, nullptr);
        __syncthreads();
        if (s_fail) {
            fail();
            return;
        }
        const int tid = tid_now();
        float bv = -3.402823466e+38f;
        uint32_t br = 0u;
        for (int i = tid; i < G; i += PNT) {
            const float v = __builtin_bit_cast(float, mbuf[2 * i]);
            const uint32_t r = mbuf[2 * i + 1];
            if (greedy_better(v, r, bv, br)) {
                bv = v;
                br = r;
            }
        }
        block_best(bv, br, s_v, s_r);
        if (tid == 0) a.tok[a.n] = (uint16_t)greedy_index(br);
    }
}

// (K, N) row-major -> (N, K) row-major, 64 x 64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_k(const f16* src, f16* dst, int K, int N) {
    __shared__ f16 tile[64][65];
    const int n0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int r = i / 64, c = i % 64;  // r: k, c: n
        if (k0 + r < K && n0 + c < N) tile[r][c] = src[(int64_t)(k0 + r) * N + n0 + c];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int r = i / 64, c = i % 64;  // r: n, c: k
        if (n0 + r < N && k0 + c < K) dst[(int64_t)(n0 + r) * K + k0 + c] = tile[c][r];
    }
}

hipError_t transpose(const f16* src, f16* dst, int K, int N, hipStream_t st) {
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((K + 63) / 64));
    hipLaunchKernelGGL(transpose_k, grid, dim3(256), 0, st, src, dst, K, N);
    return hipGetLastError();
}

// Mailboxes and the epoch words (grow-only, zeroed on growth); and the
// device's CU count.
struct PersistWs {
    void* buf = nullptr;
    size_t bytes = 0;
};
PersistWs g_pws;

struct Plan {
    int G, S_max, G3, R3, G5, R5, bufb, hr, lds;
    int o_qkv, o_att, o_x1, o_gh, o_x2, par, o_cand, words;
};

// The launch shape for cfg on a GPU of `cus` compute units and `lds_max`
// bytes of LDS per workgroup, or an error.
int plan_for(const evkhip_model_cfg& c, int cus, int lds_max, Plan* out) {
    const int d = (int)c.d, hid = (int)c.hidden, H = (int)c.heads, dh = (int)c.dh;
    EVK_RETURN_IF(d % 8 || hid % 8 || (dh != 16 && dh != 32 && dh != 64 && dh != 128), EVKHIP_ERR_UNSUPPORTED,
                  "model_decode_packed: needs d, hidden multiples of 8 and dh in {16,32,64,128}");
    Plan p{};
    // every workgroup writes at least one word in S1, S4 and the head
    p.G = std::min(std::min(cus, 3 * d / 2), std::min(hid / 2, (int)c.vocab));
    p.S_max = ((int)c.max_seq + KSPL - 1) / KSPL;
    // Wo and W2 columns: 16 (Wo) and 6 (W2) per workgroup, in pairs.  Fewer
    // S3 workgroups poll the large attention mailbox (measured: 16 beats 8,
    // 12 and 24 at C4); a W2 slice of 6 rows x hidden already fills a slot.
    p.R3 = 16;
    p.G3 = (d + p.R3 - 1) / p.R3;
    p.R5 = 6;
    p.G5 = (d + p.R5 - 1) / p.R5;
    EVK_RETURN_IF(p.G < 1 || H * p.S_max > p.G || H * p.S_max > YO || p.G3 > p.G || p.G5 > p.G, EVKHIP_ERR_UNSUPPORTED,
                  "model_decode_packed: %d heads x %d key splits do not fit %d workgroups", H, p.S_max, p.G);
    // a head's splits are merged within one wave
    EVK_RETURN_IF(p.S_max > 64, EVKHIP_ERR_UNSUPPORTED, "model_decode_packed: max_seq %u exceeds %d", c.max_seq,
                  64 * KSPL);
    const int np1 = 3 * d / 2, np4 = hid / 2;
    const int r1 = 2 * ((np1 + p.G - 1) / p.G), r4 = 2 * ((np4 + p.G - 1) / p.G);
    // one LDS slot holds any stage's slice
    int bytes = std::max(std::max(r1 * d, r4 * d), std::max(p.R3 * d, p.R5 * hid)) * 2;
    bytes = std::max(bytes, 2 * KSPL * dh * 2);
    bytes = std::max(bytes, 24 * d * 2);  // at least 24 LM-head rows
    p.bufb = (bytes + 1023) & ~1023;
    p.hr = std::min(YO, p.bufb / (d * 2));
    const int ablk = dh / 2 + 2;
    const int att_w = H * p.S_max * ablk;
    EVK_RETURN_IF(att_w > PMAXW * NPOLL || hid / 2 > PMAXW * NPOLL || 2 * p.G > PMAXW * NPOLL || d / 2 > PMAXW * NPOLL,
                  EVKHIP_ERR_UNSUPPORTED, "model_decode_packed: a stage input exceeds the poll capacity");
    // mailbox words: per parity QKV (per head: q, k, v), ATT, X1, GH, X2; then CAND
    p.o_qkv = 0;
    p.o_att = p.o_qkv + 3 * d / 2;
    p.o_x1 = p.o_att + att_w;
    p.o_gh = p.o_x1 + d / 2;
    p.o_x2 = p.o_gh + hid / 2;
    p.par = p.o_x2 + d / 2;
    p.o_cand = 2 * p.par;
    p.words = p.o_cand + 2 * p.G;
    const int xs = (d + 3) & ~3, hs = hs_floats(d, hid, dh);
    const int mw = std::max(std::max(att_w, hid / 2), std::max(2 * p.G, std::max(d / 2, 2 * dh)));
    p.lds = NBUF * p.bufb + (xs + hs + YO + 64) * 4 + mw * 4;
    EVK_RETURN_IF(p.lds > lds_max, EVKHIP_ERR_UNSUPPORTED,
                  "model_decode_packed: needs %d bytes of LDS per workgroup, the GPU has %d", p.lds, lds_max);
    *out = p;
    return EVKHIP_OK;
}

}  // namespace

int decode_status(uint32_t* flags, bool clear) {
    unsigned v = 0;
    EVK_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_dec_status), sizeof(v), 0, hipMemcpyDeviceToHost));
    *flags = v;
    if (clear && v) {
        const unsigned zero = 0;
        EVK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_dec_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice));
    }
    return EVKHIP_OK;
}

void decode_persist_free_workspace() {
    if (g_pws.buf) (void)hipFree(g_pws.buf);
    g_pws = PersistWs{};
}

}  // namespace evkhip

using namespace evkhip;

extern "C" {

uint64_t evkhip_model_packed_elems(const evkhip_model_cfg* c) { return evkhip_model_weight_elems(c); }

int evkhip_model_pack(const evkhip_model_cfg* cfg, const void* weights, void* packed, void* stream) {
    EVK_RETURN_IF(!cfg || !weights || !packed, EVKHIP_ERR_INVALID_ARG, "model_pack: null argument");
    const evkhip_model_cfg c = *cfg;
    EVK_RETURN_IF(c.vocab == 0 || c.d == 0 || c.layers == 0 || c.hidden == 0, EVKHIP_ERR_INVALID_ARG,
                  "model_pack: empty model dimension");
    EVK_RETURN_IF(weights == packed, EVKHIP_ERR_INVALID_ARG, "model_pack: packing in place is not supported");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int d = (int)c.d, hid = (int)c.hidden, V = (int)c.vocab;
    const f16* src = static_cast<const f16*>(weights);
    f16* dst = static_cast<f16*>(packed);
    const uint64_t per = (uint64_t)d * 3 * d + (uint64_t)d * d + 2 * (uint64_t)d * hid;
    EVK_HIP(hipMemcpyAsync(dst, src, (size_t)V * d * 2, hipMemcpyDeviceToDevice, st));
    for (uint32_t l = 0; l < c.layers; ++l) {
        const f16* s = src + (uint64_t)V * d + l * per;
        f16* o = dst + (uint64_t)V * d + l * per;
        EVK_HIP(transpose(s, o, d, 3 * d, st));                                         // Wqkv (d, 3d)
        EVK_HIP(transpose(s + (uint64_t)3 * d * d, o + (uint64_t)3 * d * d, d, d, st));  // Wo (d, d)
        EVK_HIP(transpose(s + (uint64_t)4 * d * d, o + (uint64_t)4 * d * d, d, hid, st));  // W1 (d, hid)
        EVK_HIP(transpose(s + (uint64_t)4 * d * d + (uint64_t)d * hid, o + (uint64_t)4 * d * d + (uint64_t)d * hid,
                          hid, d, st));                                                  // W2 (hid, d)
    }
    const uint64_t wo = (uint64_t)V * d + c.layers * per;
    EVK_HIP(transpose(src + wo, dst + wo, d, V, st));  // Wout (d, V)
    return EVKHIP_OK;
}

int evkhip_debug_decode_set_epoch(uint32_t distance) {
    EVK_RETURN_IF(!g_pws.buf, EVKHIP_ERR_INVALID_ARG,
                  "debug_decode_set_epoch: no persistent decode has run on this device yet");
    EVK_RETURN_IF(distance >= kWrapAt, EVKHIP_ERR_INVALID_ARG, "debug_decode_set_epoch: distance %u too large",
                  distance);
    const uint32_t base = kWrapAt - distance;
    EVK_HIP(hipDeviceSynchronize());
    EVK_HIP(hipMemcpy(g_pws.buf, &base, sizeof(base), hipMemcpyHostToDevice));
    return EVKHIP_OK;
}

#ifdef EVKHIP_DECODE_TRACE
// The trace of the last launch (trace build only): 2 x 1024 x 5 x 3 uint64.
int evkhip_debug_decode_trace(void* dst) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_dec_trace), sizeof(g_dec_trace), 0, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? EVKHIP_OK
               : EVKHIP_ERR_HIP;
}
#endif

int evkhip_model_decode_packed(const evkhip_model_cfg* cfg, const void* packed, void* cache, uint16_t* token_io,
                               uint32_t n_steps, uint32_t pos0, void* logits, void* stream) {
    EVK_RETURN_IF(!cfg || !packed || !cache || !token_io || !logits, EVKHIP_ERR_INVALID_ARG,
                  "model_decode_packed: null argument");
    const evkhip_model_cfg c = *cfg;
    EVK_RETURN_IF(c.vocab == 0 || c.vocab > 65536 || c.d == 0 || c.heads == 0 || c.layers == 0 || c.hidden == 0,
                  EVKHIP_ERR_INVALID_ARG, "model_decode_packed: empty model dimension");
    EVK_RETURN_IF(c.heads * c.dh != c.d, EVKHIP_ERR_SHAPE, "model_decode_packed: d=%u != heads*dh (%u*%u)", c.d,
                  c.heads, c.dh);
    EVK_RETURN_IF((uint64_t)pos0 + n_steps > c.max_seq, EVKHIP_ERR_SHAPE,
                  "model_decode_packed: positions %u..%u exceed max_seq %u", pos0, pos0 + n_steps, c.max_seq);
    EVK_RETURN_IF(!aligned16(packed) || !aligned16(cache) || c.vocab % 8, EVKHIP_ERR_UNSUPPORTED,
                  "model_decode_packed: needs 16-byte aligned weights and cache, vocab a multiple of 8");
    if (n_steps == 0) return EVKHIP_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int dev = 0, cus = 0;
    EVK_HIP(hipGetDevice(&dev));
    EVK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    int lds_max = 0;
    EVK_HIP(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    Plan pl{};
    const int rc = plan_for(c, cus, lds_max, &pl);
    if (rc != EVKHIP_OK) return rc;

    int per_cu = 0;
    EVK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(decode_persist), PNT,
                                                         (size_t)pl.lds));
    EVK_RETURN_IF(per_cu < 1 || pl.G > per_cu * cus, EVKHIP_ERR_UNSUPPORTED,
                  "model_decode_packed: %d workgroups cannot be resident at once", pl.G);
    // control words first (a fixed place for every model shape), mailboxes after
    const size_t need = 64 + (size_t)pl.words * 8;
    if (need > g_pws.bytes) {
        if (g_pws.buf) EVK_HIP(hipFree(g_pws.buf));
        g_pws = PersistWs{};
        EVK_HIP(hipMalloc(&g_pws.buf, need));
        EVK_HIP(hipMemsetAsync(g_pws.buf, 0, need, st));
        g_pws.bytes = need;
    }
    const f16* P = static_cast<const f16*>(packed);
    const uint64_t d = c.d, hid = c.hidden;
    const uint64_t per = d * 3 * d + d * d + 2 * d * hid;
    PArgs a{};
    a.d = (int)c.d; a.H = (int)c.heads; a.dh = (int)c.dh; a.hid = (int)c.hidden; a.V = (int)c.vocab;
    a.L = (int)c.layers; a.max_seq = (int)c.max_seq; a.eps = c.eps; a.rope_base = c.rope_base;
    a.E = P;
    a.lay = P + (uint64_t)c.vocab * d;
    a.per_layer = per;
    a.WoutT = a.lay + c.layers * per;
    a.cache = static_cast<f16*>(cache);
    a.tok = token_io;
    a.logits = static_cast<f16*>(logits);
    a.n = (int)n_steps;
    a.pos0 = (int)pos0;
    a.ctl = static_cast<uint32_t*>(g_pws.buf);
    a.mb = reinterpret_cast<uint64_t*>(static_cast<char*>(g_pws.buf) + 64);
    a.o_qkv = pl.o_qkv; a.o_att = pl.o_att; a.o_x1 = pl.o_x1; a.o_gh = pl.o_gh; a.o_x2 = pl.o_x2;
    a.par = pl.par; a.o_cand = pl.o_cand; a.mb_words = pl.words;
    a.S_max = pl.S_max;
    a.G3 = pl.G3; a.R3 = pl.R3; a.G5 = pl.G5; a.R5 = pl.R5;
    a.bufb = pl.bufb; a.hr = pl.hr;
    a.spin_limit = (int)std::min(flash_spin_limit(), 1u << 18);
    // An ordinary launch: the occupancy check above keeps all G workgroups
    // resident at once (one per CU), and every in-kernel wait is bounded, so
    // a workgroup that is held back (another stream's kernel on its CU)
    // delays the others or, at worst, ends the launch with
    // EVKHIP_STATUS_WAIT_TIMEOUT.  The cooperative launch API is not used:
    // the runtime state it creates was torn down after the profiler's own
    // finalisation at process exit and crashed rocprofv3 runs there.
    hipLaunchKernelGGL(decode_persist, dim3((unsigned)pl.G), dim3(PNT), (unsigned)pl.lds, st, a);
    EVK_HIP(hipGetLastError());
    return EVKHIP_OK;
}

}  // extern "C"
