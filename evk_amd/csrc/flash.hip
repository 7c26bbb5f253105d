// Flash attention forward/backward for gfx950: the kernels behind
// evk::ai::flash_attention / flash_attention_bwd (reference: evk_ai.cpp:332-473,
// shaders/flash_attention.comp, shaders/flash_attention_bwd.comp).
//
// Layout (reference MQA): Q,O,dO,dQ (B,N,H*Dh); K,V,dK,dV (B,N,Dh).  Per batch
// the query side is an (N*H) x Dh row-major matrix whose row r is query
// position r/H of head r%H, so all heads of a position share one K/V row and
// one K/V tile in LDS serves 8x more rows than multi-head attention would.
//
// MFMA mapping (v_mfma_f32_32x32x16_f16, see common.h):
//  forward / dQ : S^T = K Q^T (keys x queries).  The D layout gives every lane
//                 one query column and 16 keys, so the row max/sum is mostly
//                 lane-local, and the probabilities are already the B operand
//                 of O^T = V^T P^T.  K rows are fed to the MFMA in the order
//                 pi(m) (bits 2 and 3 of m swapped) so that element e of a lane
//                 holds key 16*(e/8) + 8*(l/32) + e%8: each 8-element half of
//                 the accumulator is 8 consecutive keys, i.e. one 16-byte LDS
//                 read of the transposed V (or K) tile.
//  dK/dV        : S = Q K^T (queries x keys) with Q rows in the order pi, so a
//                 lane owns one key column; dV^T += dO^T P and dK^T += Q^T dS
//                 read dO^T / Q^T from a per-wave transposed LDS tile.
// Softmax runs in the exp2 domain: s2 = s * scale * log2(e).
#include "kernels.h"

#include <algorithm>
#include <type_traits>

#include <math.h>

namespace evkhip {

// Status bits raised by the kernels of this file (EVKHIP_STATUS_*).
__device__ unsigned g_flash_status;

namespace {

// Default iterations (of s_sleep 1) of a bounded in-kernel wait.
constexpr int kDefaultSpinLimit = 1 << 22;
int g_spin_limit = kDefaultSpinLimit;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int BC = 64;   // keys per LDS stage
constexpr int BR = 128;  // query rows per workgroup (4 waves x 32)

// pi(m): swap bits 2 and 3 of a row index in 0..31.
DEV int pi32(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// Offset (halves) of 16-byte chunk c of row r in a tile of rows of W halves.
template <int W>
DEV int sw_off(int r, int c) {
    constexpr int KC = W / 8;
    return r * W + ((c ^ (r & (KC - 1))) << 3);
}

// Copy ROWS x DH (row-major, 16-byte chunks) from global rows [g0, g0+ROWS)
// into registers; rows >= nrows read as zero.
template <int ROWS, int DH, int NT>
struct RowTile {
    static constexpr int KC = DH / 8, CH = ROWS * KC, PER = (CH + NT - 1) / NT;
    u32x4 r[PER];
    DEV void load(const f16* src, int g0, int nrows) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int c = threadIdx.x + i * NT;
            int row = c / KC, kc = c % KC;
            u32x4 v = {0u, 0u, 0u, 0u};
            if ((CH % NT == 0 || c < CH) && g0 + row < nrows)
                v = *reinterpret_cast<const u32x4*>(src + (int64_t)(g0 + row) * DH + kc * 8);
            r[i] = v;
        }
    }
    DEV void store(f16* lds) const {  // [ROWS][DH] swizzled
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int c = threadIdx.x + i * NT;
            if (CH % NT == 0 || c < CH) {
                int row = c / KC, kc = c % KC;
                *reinterpret_cast<u32x4*>(lds + sw_off<DH>(row, kc)) = r[i];
            }
        }
    }
};

// Same rows, stored transposed in LDS as [DH][ROWS] (8x8 register transposes).
template <int ROWS, int DH, int NT>
struct TransTile {
    static constexpr int RB = ROWS / 8, DB = DH / 8, BLK = RB * DB, PER = (BLK + NT - 1) / NT;
    u32x4 r[PER][8];
    DEV void load(const f16* src, int g0, int nrows) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + i * NT;
            int db = q % DB, rb = q / DB;
            bool ok = (BLK % NT == 0 || q < BLK);
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                int g = g0 + rb * 8 + rr;
                u32x4 v = {0u, 0u, 0u, 0u};
                if (ok && g < nrows) v = *reinterpret_cast<const u32x4*>(src + (int64_t)g * DH + db * 8);
                r[i][rr] = v;
            }
        }
    }
    DEV void store(f16* lds) const {  // [DH][ROWS] swizzled
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + i * NT;
            if (BLK % NT == 0 || q < BLK) {
                int db = q % DB, rb = q / DB;
                u32x4 t[8];
                transpose8x8(r[i], t);
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    *reinterpret_cast<u32x4*>(lds + sw_off<ROWS>(db * 8 + c, rb)) = t[c];
            }
        }
    }
};

DEV half8 pack8(const float* x) {
    u32x4 u = {pack_h2(x[0], x[1]), pack_h2(x[2], x[3]), pack_h2(x[4], x[5]), pack_h2(x[6], x[7])};
    return as_half8(u);
}
// elements [off, off+8) of an accumulator
DEV half8 pack8v(const floatx16& x, int off) {
    u32x4 u = {pack_h2(x[off + 0], x[off + 1]), pack_h2(x[off + 2], x[off + 3]),
               pack_h2(x[off + 4], x[off + 5]), pack_h2(x[off + 6], x[off + 7])};
    return as_half8(u);
}

// ---------------------------------------------------------------------------
// Forward (MODE 0: O and public LSE) / statistics for the backward (MODE 1:
// lse2_rows and d_rows, with dP^T = V dO^T in place of the PV product).
//
// Workgroup: 4 waves x 16 query rows (64 rows) sharing row-major K and V
// tiles of 64 keys in LDS (double-buffered, rows padded by 32 bytes).  Each
// wave uses v_mfma_f32_16x16x32_f16:
//   S^T(16 keys x 16 q) = K(16 x 32dh) Q^T: lane l holds query l%16 and keys
//       4*(l/16)+j of each 16-key tile.
//   O^T(16 dh x 16 q) += V^T(16 dh x 32 keys) P^T: the probabilities already
//       sit in B-operand order (slot s <-> key 4*(l/16)+s of the first and
//       second 16-key tile), and V^T comes straight from the row-major V tile
//       through ds_read_tr16_b64 (4 consecutive key rows of one dh column per
//       lane).
// The softmax scale*log2(e) is folded into one FMA before v_exp_f32; the
// O rescale is skipped when no row maximum of the wave moved.
// Grid: ceil(N*H/64) * B workgroups; causal grids run heaviest rows first,
// in a zigzag so that the pairs of workgroups that share a CU carry about the
// same number of key tiles.
// ---------------------------------------------------------------------------
constexpr int FR = 64;  // query rows per workgroup (4 waves x 16)
constexpr int KT = 64;  // keys per LDS tile


DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maps a linear workgroup id to (row group, batch).  Causal: heaviest row
// groups first, alternate rounds of `round` groups reversed.
DEV void fwd_block_map(int bid, int nrg, int B, bool causal, int round, int* rg, int* b) {
    const int total = nrg * B;
    int idx = bid;
    if (causal) {
        const int r = bid / round, pos = bid % round;
        const int base = r * round;
        const int len = min(round, total - base);
        idx = (r & 1) ? base + (len - 1 - pos) : bid;
        *rg = nrg - 1 - idx / B;
    } else {
        *rg = idx / B;
    }
    *b = idx % B;
}

// Lazy rescaling: a wave keeps a reference maximum m_ref per query row and
// only re-normalises (O, l scaled by 2^(m_old-m_new)) when some score exceeds
// m_ref by more than 2^RESCALE_LOG2; in between, probabilities are
// 2^(s*c - m_ref) <= 2^RESCALE_LOG2, exact enough in fp16 and fp32 sums.
constexpr float RESCALE_LOG2 = 8.0f;

template <int DH, bool CAUSAL, int MODE>
__global__ __launch_bounds__(512) void flash_fwd(FlashArgs p, int round) {
    constexpr int KS = DH / 32;   // k-steps of QK^T (32 dh each)
    constexpr int DT = DH / 16;   // 16-row dh tiles of O^T
    constexpr int LW = DH + 8;    // LDS row stride in halves (16-byte pad)
    constexpr int TILE = KT * LW; // halves per K (or V) tile
    constexpr int CH = KT * DH / 8;  // 16-byte chunks per tile
    constexpr int PER = (CH + 255) / 256;
    // [stage][half][K tile, V tile]: the two wave sets take alternate tiles
    __shared__ __attribute__((aligned(16))) f16 smem[2 * 2 * 2 * TILE];

    const int H = p.H, N = p.N, NH = N * H;
    const int nrg = (NH + FR - 1) / FR;
    int rg, b;
    fwd_block_map(blockIdx.x, nrg, p.B, CAUSAL, round, &rg, &b);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int rw = wave & 3, half = wave >> 2;   // row wave, key half
    const int tid = threadIdx.x & 255;           // index within the half
    const int l16 = lane & 15, g = lane >> 4;
    const int R0 = rg * FR;
    const int rw0 = R0 + rw * 16;
    const int myrow = rw0 + l16;
    const bool row_ok = myrow < NH;
    const int qpos = min(myrow, NH - 1) / H;
    const int wpmax = min(rw0 + 15, NH - 1) / H;
    const int wpmin = min(rw0, NH - 1) / H;
    const int bpmax = min(R0 + FR - 1, NH - 1) / H;
    const int kend = CAUSAL ? min(N, bpmax + 1) : N;
    const float c2 = p.scale_log2;

    const f16* Qb = p.q + (int64_t)b * NH * DH;
    const f16* Kb = p.k + (int64_t)b * N * DH;
    const f16* Vb = p.v + (int64_t)b * N * DH;

    // B operand of S^T: lane holds query row myrow, dh [32ks + 8g, +8)
    half8 qf[KS], gf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u}, w = {0u, 0u, 0u, 0u};
        if (row_ok) {
            v = *reinterpret_cast<const u32x4*>(Qb + (int64_t)myrow * DH + ks * 32 + g * 8);
            if constexpr (MODE == 1)
                w = *reinterpret_cast<const u32x4*>(p.dO + (int64_t)b * NH * DH + (int64_t)myrow * DH +
                                                    ks * 32 + g * 8);
        }
        qf[ks] = as_half8(v);
        gf[ks] = as_half8(w);
    }
    // Drain the Q loads now: the main loop then only ever waits for the K/V
    // prefetch at the LDS store, never at the first MFMA of a tile.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    floatx4 oacc[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) oacc[d] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_ref = -INFINITY, t_part = 0.0f;
    floatx4 lacc = {0.0f, 0.0f, 0.0f, 0.0f};  // row sums (all 4 elements equal)
    const half8 ones8 = {(f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f,
                         (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f};

    // Each half stages its own tile (key tiles 2i and 2i+1 of pair i).
    // Rows past N load row N-1: those keys are masked to p = 0.
    u32x4 rr[2 * PER];
    auto gload = [&](int key0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = min(tid + i * 256, CH - 1);
            const int row = min(key0 + c / (DH / 8), N - 1), ch = c % (DH / 8);
            rr[i] = *reinterpret_cast<const u32x4*>(Kb + (int64_t)row * DH + ch * 8);
            rr[PER + i] = *reinterpret_cast<const u32x4*>(Vb + (int64_t)row * DH + ch * 8);
        }
    };
    auto lstore = [&](int stage) {
        f16* kb = smem + ((stage * 2 + half) * 2) * TILE;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = tid + i * 256;
            if (CH % 256 == 0 || c < CH) {
                const int row = c / (DH / 8), ch = c % (DH / 8);
                *reinterpret_cast<u32x4*>(kb + row * LW + ch * 8) = rr[i];
                *reinterpret_cast<u32x4*>(kb + TILE + row * LW + ch * 8) = rr[PER + i];
            }
        }
    };

    const int nkt = (kend + KT - 1) / KT;
    const int npair = (nkt + 1) / 2;
    if (npair > 0) {
        if (2 * 0 + half < nkt) gload(half * KT);
        lstore(0);
        if (npair > 1 && 2 + half < nkt) gload((2 + half) * KT);
    }
    __syncthreads();

    for (int pi = 0; pi < npair; ++pi) {
        const int stage = pi & 1;
        const int kt = 2 * pi + half;
        const int key0 = kt * KT;
        if (kt < nkt && (!CAUSAL || key0 <= wpmax)) {
            const f16* ks_ = smem + ((stage * 2 + half) * 2) * TILE;
            const f16* vs_ = ks_ + TILE;
            floatx4 s[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    half8 a = *reinterpret_cast<const half8*>(ks_ + (t * 16 + l16) * LW + ks * 32 + g * 8);
                    s[t] = mfma16(a, qf[ks], s[t]);
                }
            }
            floatx4 dp[4];
            if constexpr (MODE == 1) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    dp[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        half8 a = *reinterpret_cast<const half8*>(vs_ + (t * 16 + l16) * LW + ks * 32 + g * 8);
                        dp[t] = mfma16(a, gf[ks], dp[t]);
                    }
                }
            }
            // element j of s[t]: key key0 + 16t + 4g + j (raw, unscaled scores)
            if ((key0 + KT > N) || (CAUSAL && key0 + KT - 1 > wpmin)) {
                const int lim = (CAUSAL ? min(N - 1, qpos) : N - 1) - key0 - 4 * g;
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j) s[t][j] = (t * 16 + j > lim) ? -INFINITY : s[t][j];
            }
            float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                             fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
            mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(s[2][0], s[2][1]), fmaxf(s[2][2], s[2][3])),
                                 fmaxf(fmaxf(s[3][0], s[3][1]), fmaxf(s[3][2], s[3][3]))));
            mx *= c2;
            if (__any(mx > m_ref + RESCALE_LOG2)) {
                // new reference: the exact row maximum across the 4 lane groups
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float m_new = fmaxf(m_ref, mx);
                const float alpha = (m_ref == -INFINITY) ? 0.0f : fast_exp2(m_ref - m_new);
#pragma unroll
                for (int d = 0; d < DT; ++d) oacc[d] *= alpha;
                lacc *= alpha;
                t_part *= alpha;
                m_ref = m_new;
            }
            const float nbase = (m_ref == -INFINITY) ? 0.0f : -m_ref;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float pe = fast_exp2(__builtin_fmaf(s[t][j], c2, nbase));
                    if constexpr (MODE == 1) t_part += pe * dp[t][j];
                    s[t][j] = pe;
                }
            // P^T as B operands: k-step kk covers tiles 2kk, 2kk+1
            half8 pb[2];
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                u32x4 u = {pack_h2(s[2 * kk][0], s[2 * kk][1]), pack_h2(s[2 * kk][2], s[2 * kk][3]),
                           pack_h2(s[2 * kk + 1][0], s[2 * kk + 1][1]),
                           pack_h2(s[2 * kk + 1][2], s[2 * kk + 1][3])};
                pb[kk] = as_half8(u);
            }
            // row sums of the fp16 probabilities on the MFMA: ones(16x32) . P^T
            // leaves the full sum over the tile's keys in every element
            lacc = mfma16(ones8, pb[0], lacc);
            lacc = mfma16(ones8, pb[1], lacc);
            if constexpr (MODE == 0) {
                // this lane's ds_read_tr address within a 4-row x 16-col block
                const int trow = l16 >> 2, tcol = (l16 & 3) * 4;
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
                        const f16* base0 = vs_ + (kk * 32 + g * 4 + trow) * LW + d * 16 + tcol;
                        half4 lo = lds_read_tr(base0);
                        half4 hi = lds_read_tr(base0 + 16 * LW);
                        oacc[d] = mfma16(cat4(lo, hi), pb[kk], oacc[d]);
                    }
            }
        }
        if (pi + 1 < npair) {
            if (2 * (pi + 1) + half < nkt) lstore(stage ^ 1);
            if (pi + 2 < npair && 2 * (pi + 2) + half < nkt) gload((2 * (pi + 2) + half) * KT);
        }
        __syncthreads();
    }

    // Merge the two key halves through LDS (the stage buffers are free now).
    float* xch = reinterpret_cast<float*>(smem);
    constexpr int XW = DT * 4 + 3;  // floats per lane: O, m, l, t
    if (half == 1) {
        float* dst = xch + (rw * 64 + lane) * XW;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[d * 4 + j] = oacc[d][j];
        dst[DT * 4] = m_ref;
        dst[DT * 4 + 1] = lacc[0];
        dst[DT * 4 + 2] = t_part;
    }
    __syncthreads();
    if (half == 1) return;
    {
        const float* src = xch + (rw * 64 + lane) * XW;
        const float m2 = src[DT * 4];
        const float m_new = fmaxf(m_ref, m2);
        const float a1 = (m_ref == -INFINITY) ? 0.0f : fast_exp2(m_ref - m_new);
        const float a2 = (m2 == -INFINITY) ? 0.0f : fast_exp2(m2 - m_new);
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int j = 0; j < 4; ++j) oacc[d][j] = oacc[d][j] * a1 + src[d * 4 + j] * a2;
        lacc[0] = lacc[0] * a1 + src[DT * 4 + 1] * a2;
        t_part = t_part * a1 + src[DT * 4 + 2] * a2;
        m_ref = m_new;
    }

    // lacc already sums over all keys of the row; t is per lane group
    const float l_tot = lacc[0];
    float t_tot = t_part + __shfl_xor(t_part, 16, 64);
    t_tot += __shfl_xor(t_tot, 32, 64);
    const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (!row_ok) return;
    const int h = myrow % H;
    if constexpr (MODE == 0) {
        f16* Ob = p.out + (int64_t)b * NH * DH + (int64_t)myrow * DH;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            u32x2 w = {pack_h2(oacc[d][0] * inv_l, oacc[d][1] * inv_l),
                       pack_h2(oacc[d][2] * inv_l, oacc[d][3] * inv_l)};
            *reinterpret_cast<u32x2*>(Ob + d * 16 + g * 4) = w;
        }
        if (p.lse && g == 0) {
            const float lse = (l_tot > 0.0f) ? (m_ref + log2f(l_tot)) * kLn2 : -INFINITY;
            p.lse[((int64_t)b * H + h) * N + qpos] = lse;
        }
    } else {
        if (g == 0) {
            p.lse2_rows[(int64_t)b * NH + myrow] = (l_tot > 0.0f) ? m_ref + log2f(l_tot) : INFINITY;
            p.d_rows[(int64_t)b * NH + myrow] = t_tot * inv_l;
        }
    }
}

// ---------------------------------------------------------------------------
// Forward, key-split (O and the public LSE).
//
// Workgroup: two row tiles of 64 query rows, q and nrg-1-q of one batch (so
// that under the causal mask every workgroup carries about the same number
// of key chunks), 4 waves per tile.  Wave w of a tile owns key chunks w, w+4,
// ... (32 keys each) of the tile's key range, for all 64 rows: each wave runs
// its own online softmax over its keys and the four partial states
// (m, l, O) are merged once at the end.  No K/V tile is shared, so nothing
// is re-read from LDS by several waves and the main loop has no barrier:
//   S^T(32 keys x 64 q) = K Q^T with v_mfma_f32_16x16x32_f16: the K chunk is
//       loaded from global memory straight into A-operand registers; Q^T
//       (64 rows) stays in B-operand registers for the whole kernel.
//   O^T(DH x 64 q) += V^T P^T: the V chunk goes through a per-wave LDS slot
//       and comes back transposed by ds_read_b64_tr_b16; P^T is already in
//       B-operand order (slot s <-> key 4g+s for s < 4, 16+4g+s-4 after).
//   row sums: ones . P^T on the MFMA.
// The next chunk's V is requested once the current one is in its LDS slot,
// its K once the score MFMAs have read the current K registers (no register
// copies); a wave's last chunk requests nothing, so leaving the loop waits
// for no load.  Rescaling is lazy (RESCALE_LOG2), as in flash_fwd; the
// row maxima of a rescale cross the wave's 16-lane rows by permlane swaps.
// ---------------------------------------------------------------------------
constexpr int KC = 32;  // keys per chunk
#ifndef FWD_KS_QB
#define FWD_KS_QB 4  // 16-row query blocks per wave (rows per workgroup / 16)
#endif

// Maximum over the four 16-lane rows of a wave (lanes 16 and 32 apart):
// two row swaps on the VALU instead of cross-lane LDS permutes.
DEV float max_over_lane_rows(float m) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}

template <int DH, int QB>
struct KsLayout {
    static constexpr int ROWS = 16 * QB;         // query rows per workgroup
    static constexpr int KS = DH / 32;           // k-steps of QK^T
    static constexpr int DB = DH / 16;           // dh blocks of O^T
    static constexpr int VW = DH + 8;            // V slot row stride (halves)
    static constexpr int VSLOT = KC * VW;        // halves per wave slot
    static constexpr int VPER = KC * DH / 8 / 64;  // 16-byte V pieces per lane
    static constexpr int OW = DH + 4;            // merge row stride (floats)
    // the merge area follows the V slots: a wave stores its partials as soon
    // as its own loop ends, while other waves still use their slots.  Each
    // wave stores the three 16-row blocks it does not finish, and m, l of all
    // its rows.
    static constexpr int VBYTES = 4 * VSLOT * 2;
    static constexpr int MERGE = 4 * (QB - 1) * 16 * OW + 2 * 4 * ROWS;  // floats
    static constexpr int LDS_BYTES = VBYTES + MERGE * 4;
};

template <int DH, int QB, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void flash_fwd_ks(FlashArgs p) {
    using L = KsLayout<DH, QB>;
    constexpr int ROWS = L::ROWS;
    constexpr int KS = L::KS, DB = L::DB, VW = L::VW, VPER = L::VPER;
    __shared__ __attribute__((aligned(16))) float smem_all[2 * (L::LDS_BYTES / 4)];
    __shared__ int half_arrivals[2];  // barrier counters of the two halves
    if (threadIdx.x == 0) {
        half_arrivals[0] = 0;
        half_arrivals[1] = 0;
    }

    // a workgroup runs row tiles nrg-1-q (waves 0-3) and q (waves 4-7) of
    // one batch: under the causal mask every pair carries about the same
    // number of key chunks, and both halves share the CU's SIMDs
    const int H = p.H, N = p.N, NH = N * H;
    const int nrg = (NH + ROWS - 1) / ROWS;
    const int npair = (nrg + 1) / 2;
    // consecutive workgroups take consecutive batches: the workgroups an XCD
    // runs (id mod 8) then share the K/V of few batches in its L2
    const int b = blockIdx.x % p.B, pq = blockIdx.x / p.B;
    const int half = __builtin_amdgcn_readfirstlane(threadIdx.x >> 8);
    const int rg = half == 0 ? nrg - 1 - pq : pq;
    const bool active = half == 0 || rg != nrg - 1 - pq;  // odd nrg: the middle tile runs once
    float* smem_f = smem_all + half * (L::LDS_BYTES / 4);
    f16* vslot_all = reinterpret_cast<f16*>(smem_f);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3);
    const int l16 = lane & 15, g = lane >> 4;
    const int R0 = rg * ROWS;
    const int last = min(R0 + ROWS - 1, NH - 1);
    const int pmin = R0 / H, pmax = last / H;
    const int kend = CAUSAL ? min(N, pmax + 1) : N;
    const int nch = active ? (kend + KC - 1) / KC : 0;
    const float c2 = p.scale_log2;

    // K, V of this batch and Q of this row tile through buffer loads: rows
    // past the end read as zero (such keys are masked, such rows not stored)
    const f16* kb_ptr = p.k + (int64_t)b * N * DH;
    const f16* vb_ptr = p.v + (int64_t)b * N * DH;
    const __amdgpu_buffer_rsrc_t qres =
        buf_rsrc(p.q + ((int64_t)b * NH + R0) * DH, (uint32_t)(last - R0 + 1) * DH * 2);
    f16* vslot = vslot_all + wave * L::VSLOT;

    // chunk registers: K A-operands (key 16 kb + l16, dh 32 ks + 8 g) and this
    // lane's V pieces (16 bytes at byte lane*16 + i*1024 of the chunk).  Each
    // chunk gets descriptors over its own keys [c*KC, N), so keys past N read
    // as zeros.
    const uint32_t k_vo = (uint32_t)(l16 * DH + g * 8) * 2;
    const uint32_t v_vo = (uint32_t)lane * 16;
    u32x4 kr[2][KS], vr[VPER];
    // a chunk past the wave's last gets an empty descriptor: its loads
    // return zeros without touching memory (the start-up requests of the
    // late waves use this to stay branch-free)
    auto load_k = [&](int c) {
        const bool ok = c < nch;
        const uint32_t rem = ok ? (uint32_t)(N - c * KC) * DH * 2 : 0u;
        const __amdgpu_buffer_rsrc_t kres = buf_rsrc(kb_ptr + (ok ? (int64_t)c * KC * DH : 0), rem);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kr[kb][ks] = buf_load16(kres, k_vo + kb * 16 * DH * 2 + ks * 64, 0);
    };
    auto load_v = [&](int c) {
        const bool ok = c < nch;
        const uint32_t rem = ok ? (uint32_t)(N - c * KC) * DH * 2 : 0u;
        const __amdgpu_buffer_rsrc_t vres = buf_rsrc(vb_ptr + (ok ? (int64_t)c * KC * DH : 0), rem);
#pragma unroll
        for (int i = 0; i < VPER; ++i) vr[i] = buf_load16(vres, v_vo + i * 1024, 0);
    };
    auto load_chunk = [&](int c) {
        load_k(c);
        load_v(c);
    };

    // The heavy tile's first chunk goes out before the Q staging (K and V do
    // not depend on Q, so the two latencies overlap).  Under the causal mask
    // the light tile's waves issue theirs after the staging: the kernel's
    // start is bound by the burst of first requests from every CU, and the
    // heavy tile carries the workgroup's critical path (Q staged 2.4 -> 1.9
    // us, 13.0 -> 12.5 us per C2 launch).
    int c = wave;
    const bool late = CAUSAL && half == 1;
    // Every wave issues these requests (the late ones get the empty
    // descriptor): with no branch around them the staging's wait counts
    // stay exact, and the Q staging waits for the Q loads alone, not for the
    // first chunk's K and V behind them.
    load_k(late ? nch : c);

    // Q^T B operands: query R0 + 16 qb + l16, dh [32 ks + 8 g, +8)
    // the tile's Q goes through LDS once (each wave of the half loads a
    // quarter), then every wave reads its fragments from there
    half8 qf[QB][KS];
    int qpos[QB];
    {
        constexpr int QPIECES = ROWS * DH / 8;           // 16-byte pieces of the tile
        constexpr int QPER = QPIECES / 256;
        f16* qs = vslot_all;                              // [ROWS][DH + 8]
        const int ht = threadIdx.x & 255;
        u32x4 qv[QPER];
#pragma unroll
        for (int u = 0; u < QPER; ++u) {
            const int pc = ht + 256 * u, r = pc / (DH / 8), cc = (pc % (DH / 8)) * 8;
            qv[u] = buf_load16(qres, (uint32_t)(r * DH + cc) * 2, 0);
        }
        load_v(late ? nch : c);
#pragma unroll
        for (int u = 0; u < QPER; ++u) {
            const int pc = ht + 256 * u, r = pc / (DH / 8), cc = (pc % (DH / 8)) * 8;
            *reinterpret_cast<u32x4*>(qs + r * (DH + 8) + cc) = qv[u];
        }
        __syncthreads();
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            qpos[qb] = min(R0 + qb * 16 + l16, NH - 1) / H;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                qf[qb][ks] = *reinterpret_cast<const half8*>(qs + (qb * 16 + l16) * (DH + 8) + ks * 32 + g * 8);
        }
        __syncthreads();  // the V slots reuse this space
    }
    if (late) load_chunk(c);

    floatx4 oacc[DB][QB];
    floatx4 lacc[QB];
    // the running reference of a row is m_ref = -nbase once the row has one
    // (bit qb of refbits, per lane); nbase is 0 until then
    float nbase[QB];
    uint32_t refbits = 0;
    auto mref = [&](int qb) { return ((refbits >> qb) & 1) ? -nbase[qb] : -INFINITY; };
    bool fresh = true;           // some row of the wave may have no reference yet (wave-uniform)
    // no row has had a reference yet: O and l are still zero, so the first
    // rescale has nothing to scale (wave-uniform)
    bool any_ref = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int d = 0; d < DB; ++d) oacc[d][qb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        lacc[qb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        nbase[qb] = 0.0f;
    }
    const half8 ones8 = {(f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f,
                         (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f};

    const int trow = l16 >> 2, tcol = (l16 & 3) * 4;
    // chunks below cu need no mask (all keys in range and, causal, at or
    // before every row's position); the masked tail runs a separate body so
    // that the unmasked chunks carry no compare/select per score
    const int cu = CAUSAL ? min(N / KC, (pmin + 1) / KC) : N / KC;
    auto chunk = [&](int c, auto mtag) {
        constexpr bool MASK = decltype(mtag)::value;
        const int key0 = c * KC;
        // V chunk into this wave's slot (LDS ops of a wave complete in order,
        // so the previous chunk's transposed reads are done)
#pragma unroll
        for (int i = 0; i < VPER; ++i) {
            const int idx = lane + 64 * i;
            *reinterpret_cast<u32x4*>(vslot + (idx / (DH / 8)) * VW + (idx % (DH / 8)) * 8) = vr[i];
        }
        if (c + 4 < nch) load_v(c + 4);
        // V^T fragments read back at once (after the slot's writes, in
        // order): their latency hides behind the score MFMAs
        half8 vt[DB];
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const f16* base0 = vslot + (g * 4 + trow) * VW + d * 16 + tcol;
            vt[d] = cat4(lds_read_tr(base0), lds_read_tr(base0 + 16 * VW));
        }

        floatx4 s[2][QB];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    s[kb][qb] = mfma16(as_half8(kr[kb][ks]), qf[qb][ks], ks == 0 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : s[kb][qb]);
        // the K registers are free once the score MFMAs have read them: the
        // next chunk's K goes straight into them (no copy)
        if (c + 4 < nch) load_k(c + 4);
        // element j of s[kb][qb]: key key0 + 16 kb + 4 g + j, query row R0 + 16 qb + l16
        if constexpr (MASK) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int lim = (CAUSAL ? min(N - 1, qpos[qb]) : N - 1) - key0 - 4 * g;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        s[kb][qb][j] = (kb * 16 + j > lim) ? -INFINITY : s[kb][qb][j];
            }
        }
        // probabilities against the current references first.  A reference
        // only moves (rare, a real branch) when its row has none yet or some
        // probability of the chunk exceeds 2^RESCALE_LOG2; the packed fp16
        // maximum of the probabilities shows the latter (values past the fp16
        // range convert to inf), at half the instructions of an fp32 row max
        half8 pb[QB];
        auto make_p = [&]() {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                float e[2][4];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) e[kb][j] = fast_exp2(__builtin_fmaf(s[kb][qb][j], c2, nbase[qb]));
                u32x4 u = {pack_h2(e[0][0], e[0][1]), pack_h2(e[0][2], e[0][3]),
                           pack_h2(e[1][0], e[1][1]), pack_h2(e[1][2], e[1][3])};
                pb[qb] = as_half8(u);
            }
        };
        // while some row of the wave has no reference the rescale below runs
        // anyway and forms the probabilities itself
        bool need = fresh;
        if (!fresh) {
            make_p();
            half2_t hv[4 * QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int i = 0; i < 4; ++i) hv[qb * 4 + i] = half2_t{pb[qb][2 * i], pb[qb][2 * i + 1]};
            // three-input maxima (v_pk_maximum3_f16)
            auto mx3 = [](half2_t a, half2_t b, half2_t c) {
                return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
            };
            static_assert(QB == 4, "16 packed values");
            const half2_t h5[6] = {mx3(hv[0], hv[1], hv[2]), mx3(hv[3], hv[4], hv[5]), mx3(hv[6], hv[7], hv[8]),
                                   mx3(hv[9], hv[10], hv[11]), mx3(hv[12], hv[13], hv[14]), hv[15]};
            const half2_t h = mx3(mx3(h5[0], h5[1], h5[2]), mx3(h5[3], h5[4], h5[5]), h5[0]);
            need |= __builtin_fmaxf((float)h[0], (float)h[1]) > (float)(1 << (int)RESCALE_LOG2);
        }
        if (__builtin_expect(__any(need), 0)) {
            asm volatile("" ::: "memory");
            float m_new[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const float m = fmaxf(fmaxf(fmaxf(s[0][qb][0], s[0][qb][1]), fmaxf(s[0][qb][2], s[0][qb][3])),
                                      fmaxf(fmaxf(s[1][qb][0], s[1][qb][1]), fmaxf(s[1][qb][2], s[1][qb][3]))) * c2;
                m_new[qb] = fmaxf(mref(qb), max_over_lane_rows(m));
            }
            if (any_ref) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    const float alpha = ((refbits >> qb) & 1) ? fast_exp2(-nbase[qb] - m_new[qb]) : 0.0f;
#pragma unroll
                    for (int d = 0; d < DB; ++d) oacc[d][qb] *= alpha;
                    lacc[qb] *= alpha;
                }
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const bool has = m_new[qb] != -INFINITY;
                nbase[qb] = has ? -m_new[qb] : 0.0f;
                refbits |= (uint32_t)has << qb;
            }
            // rows whose keys so far were all masked still have no reference
            fresh = __any(refbits != (1u << QB) - 1);
            any_ref = true;
            make_p();
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) lacc[qb] = mfma16(ones8, pb[qb], lacc[qb]);
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) oacc[d][qb] = mfma16(vt[d], pb[qb], oacc[d][qb]);
        }
    };
    const int c_mask = __builtin_amdgcn_readfirstlane(min(nch, cu));
    for (; c < c_mask; c += 4) chunk(c, std::false_type{});
    for (; c < nch; c += 4) chunk(c, std::true_type{});

    // ---- merge the four waves' partial softmax states ----
    // Each wave stores its state as it stands (m, l and O relative to its own
    // running max); after a barrier of the half's four waves the lanes that
    // write a row combine the four with weights 2^(m_w - m).  Merge addresses derive from an opaque
    // copy of the lane id, so the compiler computes them here instead of
    // keeping them live through the loop.
    int ml = lane;
    asm volatile("" : "+v"(ml));
    const int ml16 = ml & 15, mg = ml >> 4;
    // Barrier of the four waves of this half (a counter in LDS): the halves
    // finish their loops at different times, and neither waits for the other
    // to merge.  Every wave of the half arrives (the four waves of a
    // workgroup are resident together), but the wait is bounded anyway: a
    // wave that gives up raises EVKHIP_STATUS_WAIT_TIMEOUT in the device
    // status word, which the host reads with evkhip_device_status.
    auto half_sync = [&](int target) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&half_arrivals[half], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        bool met = false;
        for (int it = 0;; ++it) {
            met = __hip_atomic_load(&half_arrivals[half], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target;
            if (met || it >= p.spin_limit) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (!met && lane == 0)
            __hip_atomic_fetch_or(&g_flash_status, (unsigned)EVKHIP_STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    static_assert(QB == 4, "one 16-row block per wave of the half");
    float* ob = smem_f + L::VBYTES / 4;          // [wave][3 blocks][16][OW]
    float* mw = ob + 4 * (QB - 1) * 16 * L::OW;  // [wave][ROWS]
    float* lw = mw + 4 * ROWS;                   // [wave][ROWS]
    // wave w finishes the rows of its block qb = w; it stores the other
    // blocks' partial state for the waves that finish them (block qb in its
    // slot qb, or qb - 1 past its own) and keeps its own
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int q = qb * 16 + ml16;
        if (mg == 0) {
            mw[wave * ROWS + q] = mref(qb);
            lw[wave * ROWS + q] = lacc[qb][0];
        }
        if (qb != wave) {
            const int k = qb < wave ? qb : qb - 1;
#pragma unroll
            for (int d = 0; d < DB; ++d)
                *reinterpret_cast<floatx4*>(ob + ((wave * (QB - 1) + k) * 16 + ml16) * L::OW + d * 16 + mg * 4) =
                    oacc[d][qb];
        }
    }
    half_sync(4);
    // lane (mg, ml16): row q = 16 wave + ml16, dh 16 d + 4 mg + j.  Every LDS
    // read of the merge (m, l of the four waves, the three other waves'
    // blocks) is issued before any is used.
    const int q = wave * 16 + ml16;
    const float mo = mw[wave * ROWS + q], lo = lw[wave * ROWS + q];
    float mv[3], lv[3];
    floatx4 r[3][DB];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int w = j < wave ? j : j + 1;        // the j-th other wave
        const int k = wave < w ? wave : wave - 1;  // this block's slot in wave w
        mv[j] = mw[w * ROWS + q];
        lv[j] = lw[w * ROWS + q];
#pragma unroll
        for (int d = 0; d < DB; ++d)
            r[j][d] = *reinterpret_cast<const floatx4*>(ob + ((w * (QB - 1) + k) * 16 + ml16) * L::OW + d * 16 + mg * 4);
    }
    // the wave's own block qb = wave, from registers (static indices)
    floatx4 a[DB];
    static_for<QB>([&](auto qc) {
        constexpr int qb = decltype(qc)::value;
        if (wave == qb) {
#pragma unroll
            for (int d = 0; d < DB; ++d) a[d] = oacc[d][qb];
        }
    });
    const float m = fmaxf(fmaxf(mo, mv[0]), fmaxf(mv[1], mv[2]));
    const float so = mo == -INFINITY ? 0.0f : fast_exp2(mo - m);
    float l = so * lo;
#pragma unroll
    for (int d = 0; d < DB; ++d) a[d] *= so;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const float sc = mv[j] == -INFINITY ? 0.0f : fast_exp2(mv[j] - m);
        l += sc * lv[j];
#pragma unroll
        for (int d = 0; d < DB; ++d) a[d] += sc * r[j][d];
    }
    const int row = R0 + q;
    const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
    if (active && row < NH) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const uint2 o = {pack_h2(a[d][0] * inv_l, a[d][1] * inv_l), pack_h2(a[d][2] * inv_l, a[d][3] * inv_l)};
            *reinterpret_cast<uint2*>(p.out + ((int64_t)b * NH + row) * DH + d * 16 + mg * 4) = o;
        }
        if (p.lse && mg == 0) {
            const float lse = l > 0.0f ? (m + log2f(l)) * kLn2 : -INFINITY;
            p.lse[((int64_t)b * H + row % H) * N + row / H] = lse;
        }
    }
}

// ---------------------------------------------------------------------------
// Backward dK, dV for head dims 32 and 64.
//
// Workgroup: 4 waves and 128 keys; wave w owns keys [32w, 32w+32) of the
// block, with K^T and V^T as B-operand registers for the whole kernel.  The
// workgroup walks 32-row chunks of the flattened (position, head) query rows,
// so the MQA sum over heads happens inside the MFMA accumulation.  A chunk
// (Q and dO rows, and per row the base-2 LSE and D = rowsum(dO * O), formed
// while staging from the O rows) is staged once in LDS for all four waves:
//   S = Q K^T, dP = dO V^T (16 rows x 16 keys per v_mfma_f32_16x16x32_f16,
//       A = rows read from LDS): lane owns one key, 4 rows per 16-row block
//   P = 2^(S*scale*log2e - lse2_row), dS = P (dP - D_row)
//   dV += P^T dO, dK += dS^T Q: the probabilities of two 16-row blocks are
//       the A operand as they are (slot s <-> row 4g+s, 16+4g+s-4), and dO, Q
//       come transposed from the LDS chunk through ds_read_b64_tr_b16.
// The query rows of a key block are split into parts of at most PART_CHUNKS
// chunks, one part per workgroup, so that causal key blocks near the start
// (which see every row) do not serialise the grid.  A key block with one
// part writes dK, dV directly; otherwise every part stores an fp32 partial
// and flash_bwd_kv_reduce sums them in part order (deterministic).
// ---------------------------------------------------------------------------
typedef int intx4 __attribute__((ext_vector_type(4)));

// fp32 sum of the 8 products of two fp16 vectors
DEV float dot8(const half8& x, const half8& y) {
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf((float)x[e], (float)y[e], acc);
    return acc;
}

constexpr int BKB = 128;       // keys per workgroup (4 waves x 32)
constexpr int BRC = 32;        // flattened query rows per chunk
constexpr int PART_CHUNKS = 16;

// Chunks of flattened rows that key block kb of a batch interacts with.
__host__ __device__ inline int bwd_kv_chunks(int kb, int N, int H, bool causal) {
    const int64_t r_lo = causal ? (int64_t)kb * BKB * H : 0;
    return (int)(((int64_t)N * H - r_lo + BRC - 1) / BRC);
}
__host__ __device__ inline int bwd_kv_parts(int kb, int N, int H, bool causal) {
    return (bwd_kv_chunks(kb, N, H, causal) + PART_CHUNKS - 1) / PART_CHUNKS;
}

template <int DH>
struct KvLayout {
    static constexpr int RW = DH + 8;             // chunk row stride (halves)
    static constexpr int CHUNK = BRC * RW;        // halves per Q (or dO) chunk
    static constexpr int STAGE = 2 * CHUNK;       // Q and dO
    static constexpr int STATS = 2 * BRC;         // floats: lse2, D per row
    static constexpr int CHUNK_BYTES = 2 * STAGE * 2;   // two stages
    static constexpr int STATS_BYTES = 2 * STATS * 4;
    static constexpr int LDS_BYTES = CHUNK_BYTES + STATS_BYTES + 2 * BRC * 4;
};

template <int DH, bool CAUSAL>
DEV void bwd_kv_body(const FlashArgs& p, float* part_ws, int parts_per_batch, int blk, char* lds) {
    using L = KvLayout<DH>;
    constexpr int KS = DH / 32, DB = DH / 16, RW = L::RW;
    constexpr int PIECES = BRC * DH / 8;              // 16-byte pieces of a chunk
    constexpr int PPT = (2 * PIECES + 255) / 256;     // per thread (Q and dO)
    f16* chunk_s = reinterpret_cast<f16*>(lds);
    float* stats_s = reinterpret_cast<float*>(lds + L::CHUNK_BYTES);
    int* pos_s = reinterpret_cast<int*>(lds + L::CHUNK_BYTES + L::STATS_BYTES);  // position of each row

    const int H = p.H, N = p.N, NH = N * H;
    const int nkb = (N + BKB - 1) / BKB;
    // workgroup -> (batch, key block, part); heavy key blocks first
    const int b = blk / parts_per_batch;
    int rem = blk % parts_per_batch, kb = 0, nparts = 0, slot0 = 0;
    for (; kb < nkb; ++kb) {
        nparts = bwd_kv_parts(kb, N, H, CAUSAL);
        if (rem < nparts) break;
        rem -= nparts;
        slot0 += nparts;
    }
    const int part = rem;
    const int nch_all = bwd_kv_chunks(kb, N, H, CAUSAL);
    const int c_lo = part * PART_CHUNKS, c_hi = min(nch_all, c_lo + PART_CHUNKS);
    const int r_lo = CAUSAL ? kb * BKB * H : 0;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int k0 = kb * BKB + wave * 32;  // this wave's first key
    const float c2 = p.scale_log2;

    // K^T, V^T B operands: key k0 + 16 kb2 + l16, dh [32 ks + 8 g, +8)
    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(p.k + (int64_t)b * N * DH, (uint32_t)N * DH * 2);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(p.v + (int64_t)b * N * DH, (uint32_t)N * DH * 2);
    half8 kt[2][KS], vt[2][KS];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint32_t off = (uint32_t)((k0 + 16 * k2 + l16) * DH + ks * 32 + g * 8) * 2;
            kt[k2][ks] = as_half8(buf_load16(kres, off, 0));
            vt[k2][ks] = as_half8(buf_load16(vres, off, 0));
        }

    floatx4 dk[2][DB], dv[2][DB];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            dk[k2][d] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            dv[k2][d] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }

    // chunk staging: thread t moves 16-byte pieces t, t+256, ... of [Q rows | dO rows]
    const __amdgpu_buffer_rsrc_t qres = buf_rsrc(p.q + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2);
    const __amdgpu_buffer_rsrc_t gres = buf_rsrc(p.dO + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2);
    const __amdgpu_buffer_rsrc_t ores = buf_rsrc(p.o + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2);
    const __amdgpu_buffer_rsrc_t lres = buf_rsrc(p.lse + (int64_t)b * H * N, (uint32_t)(H * N) * 4u);
    // A thread holds at most one dO piece (DH <= 64); with it the O piece at
    // the same place, so that D = rowsum(dO * O) comes from the DH/8 lanes
    // of a row.  Rows past NH read as zeros: D = 0, lse2 = 0 (their Q and
    // dO rows are zero too, so they add nothing).
    u32x4 pr[PPT], po = {0u, 0u, 0u, 0u};
    float sr = 0.0f;
    int spos = 0;
    // Row (position, head) of thread t's statistics row (t mod BRC), advanced
    // by BRC rows per chunk without dividing: gload(c) is called for c_lo,
    // c_lo + 1, ... in order.
    const int h_step = BRC % H, p_step = BRC / H;
    int st_head, st_pos;
    {
        const int row = r_lo + c_lo * BRC + (int)(threadIdx.x % BRC);
        st_head = row % H;
        st_pos = row / H;
    }
    int st_next = c_lo;
    // The LSE value is kept as loaded (lstore scales it), so that nothing
    // waits for the load here.
    auto gload = [&](int c) {
        const uint32_t row0 = (uint32_t)(r_lo + c * BRC);
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + 256 * i;
            // PIECES is a multiple of 64, so `which` is uniform across the
            // wave; said explicitly, the descriptor choice stays scalar (a
            // per-lane choice costs a loop over descriptors, after which the
            // compiler can no longer count the loads in flight and waits for
            // all of them, the next chunk's included, before the MFMAs)
            const int which = __builtin_amdgcn_readfirstlane(pc / PIECES), pi = pc % PIECES;
            const uint32_t off = (row0 * DH + pi * 8) * 2;
            if (2 * PIECES % 256 == 0 || pc < 2 * PIECES) {
                if (which) {
                    pr[i] = buf_load16(gres, off, 0);
                    po = buf_load16(ores, off, 0);
                } else {
                    pr[i] = buf_load16(qres, off, 0);
                }
            }
        }
        for (; st_next < c; ++st_next) {
            st_head += h_step;
            st_pos += p_step;
            if (st_head >= H) {
                st_head -= H;
                st_pos += 1;
            }
        }
        // LSE of row row0 + t (t < BRC), from the (B, H, N) LSE; every
        // thread issues the (predicated) load and uses it below, so that no
        // path leaves it in flight
        sr = buf_load_f32(lres, oob_or(threadIdx.x < BRC && row0 + threadIdx.x < (uint32_t)NH,
                                       (uint32_t)(st_head * N + st_pos) * 4u));
        if (threadIdx.x >= BRC && threadIdx.x < 2 * BRC) spos = st_pos;
    };
    auto lstore = [&](int stage) {
        f16* cs = chunk_s + stage * L::STAGE;
        float dsum = 0.0f;
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + 256 * i;
            const int which = __builtin_amdgcn_readfirstlane(pc / PIECES), pi = pc % PIECES;
            if (2 * PIECES % 256 == 0 || pc < 2 * PIECES) {
                *reinterpret_cast<u32x4*>(cs + which * L::CHUNK + (pi / (DH / 8)) * RW + (pi % (DH / 8)) * 8) = pr[i];
                if (which) dsum = dot8(as_half8(pr[i]), as_half8(po));
            }
        }
        // the DH/8 lanes of a row are adjacent (a quad or two): DPP sums
        dsum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dsum), 0xB1, 0xF, 0xF, false));
        if (DH / 8 >= 4)
            dsum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dsum), 0x4E, 0xF, 0xF, false));
        if (DH / 8 >= 8)
            dsum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dsum), 0x141, 0xF, 0xF, false));
        static_assert(DH / 8 <= 8, "a row's lanes within a half row");
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + 256 * i;
            const int pi = pc % PIECES;
            if (pc >= PIECES && pc < 2 * PIECES && pi % (DH / 8) == 0)
                stats_s[stage * L::STATS + BRC + pi / (DH / 8)] = dsum;
        }
        const float l2 = sr * kLog2e;  // base-2 LSE
        if (threadIdx.x < BRC) stats_s[stage * L::STATS + threadIdx.x] = l2;
        else if (threadIdx.x < 2 * BRC) pos_s[stage * BRC + threadIdx.x - BRC] = spos;
    };

    if (c_lo < c_hi) {
        gload(c_lo);
        lstore(0);
    }
    // nothing in flight from here on (the K^T, V^T operands included): the
    // loop's waits then cover only its own loads
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    const int trow = l16 >> 2, tcol = (l16 & 3) * 4;
    for (int c = c_lo; c < c_hi; ++c) {
        const int stage = (c - c_lo) & 1;
        // the next chunk is requested and staged unconditionally (past the
        // part's last chunk the rows are either past NH, reading zeros, or
        // rows nothing reads, staged into the stage nothing reads): with
        // every load of an iteration consumed in that iteration, the
        // compiler knows no load is in flight at the loop head
        gload(c + 1);
        const int row0 = r_lo + c * BRC;
        // rows of this chunk hold positions row0/H .. (row0+31)/H
        const bool live = !CAUSAL || (row0 + BRC - 1) / H >= k0;
        if (live && k0 < N) {
            const f16* qs = chunk_s + stage * L::STAGE;
            const f16* gs = qs + L::CHUNK;
            const float* st = stats_s + stage * L::STATS;
            // row statistics of the chunk, read before the MFMAs so that the
            // LDS latency hides behind them
            const int* ps_ = pos_s + stage * BRC;
            floatx4 l2v[2], ddv[2];
            intx4 psv[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                l2v[rb] = *reinterpret_cast<const floatx4*>(st + rb * 16 + 4 * g);
                ddv[rb] = *reinterpret_cast<const floatx4*>(st + BRC + rb * 16 + 4 * g);
                psv[rb] = *reinterpret_cast<const intx4*>(ps_ + rb * 16 + 4 * g);
            }
            const int pos_min = ps_[0];
            floatx4 s[2][2], dp[2][2];  // [row block][key block]
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                half8 qa[KS], ga[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    qa[ks] = *reinterpret_cast<const half8*>(qs + (rb * 16 + l16) * RW + ks * 32 + g * 8);
                    ga[ks] = *reinterpret_cast<const half8*>(gs + (rb * 16 + l16) * RW + ks * 32 + g * 8);
                }
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    s[rb][k2] = mfma16(qa[0], kt[k2][0], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
                    dp[rb][k2] = mfma16(ga[0], vt[k2][0], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                    for (int ks = 1; ks < KS; ++ks) {
                        s[rb][k2] = mfma16(qa[ks], kt[k2][ks], s[rb][k2]);
                        dp[rb][k2] = mfma16(ga[ks], vt[k2][ks], dp[rb][k2]);
                    }
                }
            }
            // element j of s[rb][k2]: row row0 + 16 rb + 4 g + j, key k0 + 16 k2 + l16
            // masking only where some key of this wave can exceed some row's
            // position (or lie past N)
            const bool edge = (CAUSAL && pos_min < k0 + 31) || k0 + 31 >= N;
            half8 pa[2], da[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int key = k0 + 16 * k2 + l16;
                float pv[2][4], dsv[2][4];
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const floatx4 l2 = l2v[rb], dd = ddv[rb];
                    const intx4 ps = psv[rb];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float pe = fast_exp2(__builtin_fmaf(s[rb][k2][j], c2, -l2[j]));
                        if (edge && ((CAUSAL && key > ps[j]) || key >= N)) pe = 0.0f;
                        pv[rb][j] = pe;
                        dsv[rb][j] = pe * (dp[rb][k2][j] - dd[j]);
                    }
                }
                u32x4 u = {pack_h2(pv[0][0], pv[0][1]), pack_h2(pv[0][2], pv[0][3]),
                           pack_h2(pv[1][0], pv[1][1]), pack_h2(pv[1][2], pv[1][3])};
                u32x4 w = {pack_h2(dsv[0][0], dsv[0][1]), pack_h2(dsv[0][2], dsv[0][3]),
                           pack_h2(dsv[1][0], dsv[1][1]), pack_h2(dsv[1][2], dsv[1][3])};
                pa[k2] = as_half8(u);
                da[k2] = as_half8(w);
            }
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const f16* gb = gs + (g * 4 + trow) * RW + d * 16 + tcol;
                const f16* qb_ = qs + (g * 4 + trow) * RW + d * 16 + tcol;
                const half8 gt = cat4(lds_read_tr(gb), lds_read_tr(gb + 16 * RW));
                const half8 qt = cat4(lds_read_tr(qb_), lds_read_tr(qb_ + 16 * RW));
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    dv[k2][d] = mfma16(pa[k2], gt, dv[k2][d]);
                    dk[k2][d] = mfma16(da[k2], qt, dk[k2][d]);
                }
            }
        }
        lstore(stage ^ 1);
        __syncthreads();
    }

    // element j of dk[k2][d]: key k0 + 16 k2 + 4 g + j, dh 16 d + l16
    auto store_f16 = [&](const floatx4 (&acc)[2][DB], f16* out, float scale) {
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = k0 + 16 * k2 + 4 * g + j;
                if (key < N) {
#pragma unroll
                    for (int d = 0; d < DB; ++d)
                        out[((int64_t)b * N + key) * DH + d * 16 + l16] = (f16)(acc[k2][d][j] * scale);
                }
            }
    };
    if (nparts == 1) {
        store_f16(dk, p.dK, p.scale);
        store_f16(dv, p.dV, 1.0f);
        return;
    }
    // fp32 partial of this part, lane-major: [slot][wave][dk|dv][k2][d][lane] floatx4
    constexpr int PW = 2 * 2 * DB;
    const int64_t slot = (int64_t)b * parts_per_batch + slot0 + part;
    floatx4* mine = reinterpret_cast<floatx4*>(part_ws) + (slot * 4 + wave) * PW * 64;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            // nontemporal: written once here, read once by the reduce kernel
            __builtin_nontemporal_store(dk[k2][d], mine + ((0 * 2 + k2) * DB + d) * 64 + lane);
            __builtin_nontemporal_store(dv[k2][d], mine + ((1 * 2 + k2) * DB + d) * 64 + lane);
        }
}

// Sums the fp32 partials of key blocks with several row parts, in part
// order, and writes dK (times the softmax scale) and dV.  Grid: one
// workgroup per (batch, key block) x 16 slices of its 4096 floatx4.
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256) void flash_bwd_kv_reduce(FlashArgs p, const float* part_ws, int parts_per_batch) {
    constexpr int DB = DH / 16, PW = 2 * 2 * DB, SLOT = 4 * PW * 64;  // floatx4 per slot
    const int N = p.N, H = p.H;
    const int nkb = (N + BKB - 1) / BKB;
    const int bk = blockIdx.x / 16, slice = blockIdx.x % 16;
    const int b = bk / nkb, kb = bk % nkb;
    int slot0 = 0;
    for (int k = 0; k < kb; ++k) slot0 += bwd_kv_parts(k, N, H, CAUSAL);
    const int nparts = bwd_kv_parts(kb, N, H, CAUSAL);
    if (nparts == 1) return;  // written directly by its only part
    for (int e = slice * 256 + threadIdx.x; e < SLOT; e += 16 * 256) {
        const floatx4* src = reinterpret_cast<const floatx4*>(part_ws) + ((int64_t)b * parts_per_batch + slot0) * SLOT + e;
        // part order as written; up to 16 loads go out together (predicated,
        // no serial tail) so that their latencies overlap
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int q = 0; q < nparts; q += 16) {
            floatx4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (q + u < nparts) v[u] = __builtin_nontemporal_load(src + (int64_t)(q + u) * SLOT);
            if (q == 0) acc = v[0];
            else acc += v[0];
#pragma unroll
            for (int u = 1; u < 16; ++u)
                if (q + u < nparts) acc += v[u];
        }
        // e = ((wave * 2 + which) * 2 + k2) * DB + d) * 64 + lane
        const int lane = e % 64, d = (e / 64) % DB, k2 = (e / (64 * DB)) % 2, which = (e / (64 * DB * 2)) % 2,
                  wave = e / (64 * PW);
        const int key0 = kb * BKB + wave * 32 + 16 * k2 + 4 * (lane >> 4);
        const int dh = d * 16 + (lane & 15);
        f16* out = which ? p.dV : p.dK;
        const float sc = which ? 1.0f : p.scale;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (key0 + j < N) out[((int64_t)b * N + key0 + j) * DH + dh] = (f16)(acc[j] * sc);
    }
}

// ---------------------------------------------------------------------------
// Backward dQ for head dims 32 and 64: the key-split forward's structure
// without the online softmax (P comes from the saved row statistics).
// Workgroup: 64 flattened query rows, 4 waves; wave w takes 32-key chunks
// w, w+4, ... for all 64 rows:
//   S^T = K Q^T, dP^T = V dO^T (K and V chunks straight into A-operand
//       registers; Q^T, dO^T held as B operands)
//   P^T = 2^(S^T*scale*log2e - lse2), dS^T = P^T (dP^T - D)
//   dQ^T += K^T dS^T: K goes through a per-wave LDS slot and comes back
//       transposed (ds_read_b64_tr_b16); dS^T is already in B-operand order.
// The four partial dQ^T are summed through LDS and scaled by the softmax
// scale.
// ---------------------------------------------------------------------------
template <int DH>
struct DqLayout {
    static constexpr int KW = DH + 8;             // K slot row stride (halves)
    static constexpr int KSLOT = KC * KW;         // halves per wave slot
    static constexpr int OW = DH + 4;             // merge row stride (floats)
    static constexpr int MERGE = 4 * 64 * OW;     // floats
    static constexpr int LDS_BYTES = (MERGE * 4 > 4 * KSLOT * 2) ? MERGE * 4 : 4 * KSLOT * 2;
};

template <int DH, bool CAUSAL>
DEV void bwd_q_body(const FlashArgs& p, int blk, char* lds) {
    using L = DqLayout<DH>;
    constexpr int KS = DH / 32, DB = DH / 16, KW = L::KW, OW = L::OW;
    constexpr int KPER = KC * DH / 8 / 64;  // 16-byte K pieces per lane
    float* smem_f = reinterpret_cast<float*>(lds);
    f16* kslot = reinterpret_cast<f16*>(smem_f) + (threadIdx.x >> 6) * L::KSLOT;

    const int H = p.H, N = p.N, NH = N * H;
    const int nrg = (NH + 63) / 64;
    const int b = blk % p.B;
    const int rg = CAUSAL ? nrg - 1 - blk / p.B : blk / p.B;  // heavy rows first
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int R0 = rg * 64;
    const int last = min(R0 + 63, NH - 1);
    const int pmin = R0 / H, pmax = last / H;
    const int kend = CAUSAL ? min(N, pmax + 1) : N;
    const int nch = (kend + KC - 1) / KC;
    const float c2 = p.scale_log2;

    const f16* kb_ptr = p.k + (int64_t)b * N * DH;
    const f16* vb_ptr = p.v + (int64_t)b * N * DH;
    const uint32_t rows_bytes = (uint32_t)(last - R0 + 1) * DH * 2;
    const __amdgpu_buffer_rsrc_t qres = buf_rsrc(p.q + ((int64_t)b * NH + R0) * DH, rows_bytes);
    const __amdgpu_buffer_rsrc_t gres = buf_rsrc(p.dO + ((int64_t)b * NH + R0) * DH, rows_bytes);
    const __amdgpu_buffer_rsrc_t ores = buf_rsrc(p.o + ((int64_t)b * NH + R0) * DH, rows_bytes);

    // B operands: row R0 + 16 qb + l16, dh [32 ks + 8 g, +8); row statistics:
    // the base-2 LSE from the (B, H, N) LSE, and D = rowsum(dO * O) over the
    // row's four lane groups
    half8 qf[4][KS], gf[4][KS];
    float l2[4], dd[4];
    int qpos[4];
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
        const int row = min(R0 + qb * 16 + l16, NH - 1);
        qpos[qb] = row / H;
        l2[qb] = p.lse[((int64_t)b * H + row % H) * N + row / H] * kLog2e;
        float dsum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint32_t off = (uint32_t)((qb * 16 + l16) * DH + ks * 32 + g * 8) * 2;
            qf[qb][ks] = as_half8(buf_load16(qres, off, 0));
            gf[qb][ks] = as_half8(buf_load16(gres, off, 0));
            dsum += dot8(gf[qb][ks], as_half8(buf_load16(ores, off, 0)));
        }
        dsum += __shfl_xor(dsum, 16, 64);
        dd[qb] = dsum + __shfl_xor(dsum, 32, 64);
    }
    floatx4 acc[DB][4];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) acc[d][qb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t a_vo = (uint32_t)(l16 * DH + g * 8) * 2;  // + k2*16*DH*2 + ks*64
    const uint32_t p_vo = (uint32_t)lane * 16;                // + i*1024
    const int k_lo = (lane / (DH / 8)) * KW + (lane % (DH / 8)) * 8;
    u32x4 kp[KPER], va[2][KS];
    auto load_chunk = [&](int c) {  // descriptors over keys [c*KC, N): keys past N read as zeros
        const uint32_t rem = (uint32_t)(N - c * KC) * DH * 2;
        const __amdgpu_buffer_rsrc_t kres = buf_rsrc(kb_ptr + (int64_t)c * KC * DH, rem);
        const __amdgpu_buffer_rsrc_t vres = buf_rsrc(vb_ptr + (int64_t)c * KC * DH, rem);
#pragma unroll
        for (int i = 0; i < KPER; ++i) kp[i] = buf_load16(kres, p_vo + i * 1024, 0);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) va[k2][ks] = buf_load16(vres, a_vo + k2 * 16 * DH * 2 + ks * 64, 0);
    };
    const int trow = l16 >> 2, tcol = (l16 & 3) * 4;
    int c = wave;
    if (c < nch) load_chunk(c);
    for (; c < nch; c += 4) {
        const int key0 = c * KC;
        // K chunk into this wave's slot; its A operands and K^T come back from LDS
#pragma unroll
        for (int i = 0; i < KPER; ++i)
            *reinterpret_cast<u32x4*>(kslot + k_lo + i * (64 / (DH / 8)) * KW) = kp[i];
        half8 vf[2][KS];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) vf[k2][ks] = as_half8(va[k2][ks]);
        half8 kf[2][KS];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kf[k2][ks] = *reinterpret_cast<const half8*>(kslot + (k2 * 16 + l16) * KW + ks * 32 + g * 8);
        if (c + 4 < nch) load_chunk(c + 4);
        half8 db_[4];
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) {
            floatx4 s[2], dp[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                s[k2] = mfma16(kf[k2][0], qf[qb][0], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
                dp[k2] = mfma16(vf[k2][0], gf[qb][0], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                for (int ks = 1; ks < KS; ++ks) {
                    s[k2] = mfma16(kf[k2][ks], qf[qb][ks], s[k2]);
                    dp[k2] = mfma16(vf[k2][ks], gf[qb][ks], dp[k2]);
                }
            }
            // element j of s[k2]: key key0 + 16 k2 + 4 g + j, row R0 + 16 qb + l16
            const int lim = (CAUSAL ? min(N - 1, qpos[qb]) : N - 1) - key0 - 4 * g;
            const bool edge = key0 + KC > N || (CAUSAL && key0 + KC - 1 > pmin);
            float dsv[2][4];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float pe = fast_exp2(__builtin_fmaf(s[k2][j], c2, -l2[qb]));
                    if (edge && k2 * 16 + j > lim) pe = 0.0f;
                    dsv[k2][j] = pe * (dp[k2][j] - dd[qb]);
                }
            u32x4 u = {pack_h2(dsv[0][0], dsv[0][1]), pack_h2(dsv[0][2], dsv[0][3]),
                       pack_h2(dsv[1][0], dsv[1][1]), pack_h2(dsv[1][2], dsv[1][3])};
            db_[qb] = as_half8(u);
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const f16* base0 = kslot + (g * 4 + trow) * KW + d * 16 + tcol;
            const half8 kt = cat4(lds_read_tr(base0), lds_read_tr(base0 + 16 * KW));
#pragma unroll
            for (int qb = 0; qb < 4; ++qb) acc[d][qb] = mfma16(kt, db_[qb], acc[d][qb]);
        }
    }

    // sum the four waves' dQ^T through LDS
    int ml = lane;
    asm volatile("" : "+v"(ml));
    const int ml16 = ml & 15, mg = ml >> 4;
    __syncthreads();
    float* ob = smem_f;
#pragma unroll
    for (int qb = 0; qb < 4; ++qb)
#pragma unroll
        for (int d = 0; d < DB; ++d)
            *reinterpret_cast<floatx4*>(ob + (wave * 64 + qb * 16 + ml16) * OW + d * 16 + mg * 4) = acc[d][qb];
    __syncthreads();
    constexpr int CPR = DH / 8;
    for (int rr = ml / CPR; rr < 16; rr += 64 / CPR) {
        const int q = wave * 16 + rr;
        const int row = R0 + q;
        const int dc = (ml % CPR) * 8;
        floatx4 a0 = *reinterpret_cast<const floatx4*>(ob + q * OW + dc);
        floatx4 a1 = *reinterpret_cast<const floatx4*>(ob + q * OW + dc + 4);
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            a0 += *reinterpret_cast<const floatx4*>(ob + (w * 64 + q) * OW + dc);
            a1 += *reinterpret_cast<const floatx4*>(ob + (w * 64 + q) * OW + dc + 4);
        }
        if (row < NH) {
            const float sc = p.scale;
            u32x4 o = {pack_h2(a0[0] * sc, a0[1] * sc), pack_h2(a0[2] * sc, a0[3] * sc),
                       pack_h2(a1[0] * sc, a1[1] * sc), pack_h2(a1[2] * sc, a1[3] * sc)};
            __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(p.out + ((int64_t)b * NH + row) * DH + dc));
        }
    }
}

// dK/dV (key blocks x row parts) and dQ (row tiles) in one launch: the
// first n_kv workgroups run the former, heavy key blocks first, the rest
// the latter, heavy row tiles first.  The two halves are independent (both
// read only Q, K, V, dO and the row statistics), so the dQ tiles fill the
// CUs that the short dK/dV parts free.
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_bwd_kvq(FlashArgs p, float* part_ws, int parts_per_batch, int n_kv) {
    constexpr int KVB = KvLayout<DH>::LDS_BYTES, QB = DqLayout<DH>::LDS_BYTES;
    __shared__ __attribute__((aligned(16))) char lds[KVB > QB ? KVB : QB];
    if ((int)blockIdx.x < n_kv) {
        // Workgroup i runs on XCD i % 8.  When the batches divide the XCDs
        // evenly, XCD x takes the dK/dV parts of batch x / (8 / B) only
        // (every (8 / B)-th part, heavy key blocks first), so the key blocks
        // that re-read a batch's Q, dO and O rows find them in that XCD's L2.
        int blk = blockIdx.x;
        const int xpb = p.B > 0 && 8 % p.B == 0 ? 8 / p.B : 0;
        if (xpb > 0 && parts_per_batch % xpb == 0 && n_kv == p.B * parts_per_batch) {
            const int x = blk % 8, i = blk / 8;
            blk = (x / xpb) * parts_per_batch + i * xpb + x % xpb;
        }
        bwd_kv_body<DH, CAUSAL>(p, part_ws, parts_per_batch, blk, lds);
    } else {
        // the same XCD assignment for the dQ tiles: XCD x takes the row tiles
        // of batch x / (8 / B) (heavy first), so that one XCD's L2 holds the
        // Q, dO and O rows of one batch for both kinds of workgroup
        int blk = blockIdx.x - n_kv;
        const int nrg = (p.N * p.H + 63) / 64;
        const int xpb = p.B > 0 && 8 % p.B == 0 ? 8 / p.B : 0;
        if (xpb > 0 && n_kv % 8 == 0 && nrg % xpb == 0) {
            const int x = blk % 8, i = blk / 8;
            blk = (i * xpb + x % xpb) * p.B + x / xpb;  // bwd_q_body: batch blk % B, tile blk / B
        }
        bwd_q_body<DH, CAUSAL>(p, blk, lds);
    }
}

// lse2_rows / d_rows from a saved LSE and O: D_i = rowsum(dO_i * O_i).
// DH/8 lanes per row, one 16-byte piece of O and of dO each (coalesced),
// summed across the row's lanes with shuffles.
template <int DH>
__global__ __launch_bounds__(256) void flash_bwd_pre(FlashArgs p) {
    constexpr int LPR = DH / 8;  // lanes per row
    const int NH = p.N * p.H;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t idx = t / LPR;  // flattened (batch, row)
    const int part = (int)(t % LPR);
    const bool ok = idx < (int64_t)p.B * NH;
    float acc = 0.0f;
    if (ok) {
        const half8 x = *reinterpret_cast<const half8*>(p.o + idx * DH + part * 8);
        const half8 y = *reinterpret_cast<const half8*>(p.dO + idx * DH + part * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)x[e] * (float)y[e];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (ok && part == 0) {
        const int b = (int)(idx / NH), r = (int)(idx % NH);
        p.d_rows[idx] = acc;
        p.lse2_rows[idx] = p.lse[((int64_t)b * p.H + (r % p.H)) * p.N + r / p.H] * kLog2e;
    }
}

// ---------------------------------------------------------------------------
// dK, dV.  Grid: (ceil(N/32), B); 4 waves share a 32-key block whose K and V
// fragments stay in registers; the waves take 32-row query tiles round-robin
// and meet in LDS at the end.
// ---------------------------------------------------------------------------
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256) void flash_bwd_dkdv(FlashArgs p) {
    constexpr int KS = DH / 16, DT = DH / 32;
    // per wave: Q^T and dO^T tiles [DH][32]; reused as the fp32 reduction area
    constexpr int WAVE_HALVES = 2 * DH * 32;
    __shared__ __attribute__((aligned(16))) f16 smem[4 * WAVE_HALVES];

    const int H = p.H, N = p.N, NH = N * H;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, lg = lane >> 5;
    const int key0 = blockIdx.x * 32;
    const int mykey = key0 + l32;
    const bool key_ok = mykey < N;

    const f16* Qb = p.q + (int64_t)b * NH * DH;
    const f16* dOb = p.dO + (int64_t)b * NH * DH;
    const float* lse2 = p.lse2_rows + (int64_t)b * NH;
    const float* Dr = p.d_rows + (int64_t)b * NH;

    // K^T and V^T as B operands: lane holds key mykey, dh [16ks + 8lg, +8).
    half8 kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 a = {0u, 0u, 0u, 0u}, c = {0u, 0u, 0u, 0u};
        if (key_ok) {
            a = *reinterpret_cast<const u32x4*>(p.k + ((int64_t)b * N + mykey) * DH + ks * 16 + lg * 8);
            c = *reinterpret_cast<const u32x4*>(p.v + ((int64_t)b * N + mykey) * DH + ks * 16 + lg * 8);
        }
        kf[ks] = as_half8(a);
        vf[ks] = as_half8(c);
    }

    floatx16 dk[DT], dv[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) { dk[t][e] = 0.0f; dv[t][e] = 0.0f; }

    f16* sQt = smem + wave * WAVE_HALVES;  // [DH][32]
    f16* sDt = sQt + DH * 32;              // [DH][32]

    const int rstart = CAUSAL ? (key0 * H) / 32 * 32 : 0;
    const int ntile = (NH - rstart + 31) / 32;
    for (int ti = wave; ti < ntile; ti += 4) {
        const int q0 = rstart + ti * 32;
        // this lane's A-operand row: query q0 + pi(l32)
        const int arow = q0 + pi32(l32);
        const bool arow_ok = arow < NH;
        floatx16 s, dp;
#pragma unroll
        for (int e = 0; e < 16; ++e) { s[e] = 0.0f; dp[e] = 0.0f; }
        // Stage Q^T, dO^T for this tile: lane writes its row's 8 dh values.
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 qa = {0u, 0u, 0u, 0u}, ga = {0u, 0u, 0u, 0u};
            if (arow_ok) {
                qa = *reinterpret_cast<const u32x4*>(Qb + (int64_t)arow * DH + ks * 16 + lg * 8);
                ga = *reinterpret_cast<const u32x4*>(dOb + (int64_t)arow * DH + ks * 16 + lg * 8);
            }
            half8 qh = as_half8(qa), gh = as_half8(ga);
            s = mfma32(qh, kf[ks], s);
            dp = mfma32(gh, vf[ks], dp);
            // transposed store: column index = query offset pi(l32) within the tile
            const int qc = pi32(l32);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int dh = ks * 16 + lg * 8 + e;
                sQt[dh * 32 + qc] = qh[e];
                sDt[dh * 32 + qc] = gh[e];
            }
        }
        // element e: query q0 + 16*(e/8) + 8*lg + e%8, key mykey
        float pe[16], dse[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int qr = q0 + 16 * (e >> 3) + 8 * lg + (e & 7);
            float pv = 0.0f, dsv = 0.0f;
            if (qr < NH && key_ok && (!CAUSAL || mykey <= qr / H)) {
                pv = exp2f(s[e] * p.scale_log2 - lse2[qr]);
                dsv = pv * (dp[e] - Dr[qr]);
            }
            pe[e] = pv;
            dse[e] = dsv;
        }
        const half8 pb0 = pack8(&pe[0]), pb1 = pack8(&pe[8]);
        const half8 sb0 = pack8(&dse[0]), sb1 = pack8(&dse[8]);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS stores of this wave done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const int dh = t * 32 + l32;
            // A operand rows dh, slots = queries 16*kstep + 8*lg + (0..7)
            half8 g0 = *reinterpret_cast<const half8*>(sDt + dh * 32 + 0 + lg * 8);
            half8 g1 = *reinterpret_cast<const half8*>(sDt + dh * 32 + 16 + lg * 8);
            half8 q0h = *reinterpret_cast<const half8*>(sQt + dh * 32 + 0 + lg * 8);
            half8 q1h = *reinterpret_cast<const half8*>(sQt + dh * 32 + 16 + lg * 8);
            dv[t] = mfma32(g0, pb0, dv[t]);
            dv[t] = mfma32(g1, pb1, dv[t]);
            dk[t] = mfma32(q0h, sb0, dk[t]);
            dk[t] = mfma32(q1h, sb1, dk[t]);
        }
        __builtin_amdgcn_wave_barrier();
    }

    // Reduce the 4 waves: fp32 [wave][DT][16][64] for dk then dv.
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    constexpr int PERW = DT * 16 * 64;  // floats per wave per tensor
    static_assert(4 * PERW * 4 <= (int)sizeof(smem), "reduction area");
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                red[wave * PERW + (t * 16 + e) * 64 + lane] = pass == 0 ? dk[t][e] : dv[t][e];
        __syncthreads();
        if (wave == 0) {
            f16* dst = (pass == 0 ? p.dK : p.dV) + ((int64_t)b * N) * DH;
            const float sc = pass == 0 ? p.scale : 1.0f;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int i = (t * 16 + e) * 64 + lane;
                    float v = red[i] + red[PERW + i] + red[2 * PERW + i] + red[3 * PERW + i];
                    const int dh = t * 32 + 8 * (e >> 2) + 4 * lg + (e & 3);
                    if (key_ok) dst[(int64_t)mykey * DH + dh] = (f16)(v * sc);
                }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// dQ.  Grid: (ceil(N*H/128), B), like the forward.
// ---------------------------------------------------------------------------
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256) void flash_bwd_dq(FlashArgs p) {
    constexpr int KS = DH / 16, DT = DH / 32;
    __shared__ __attribute__((aligned(16))) f16 sK[2][BC * DH];   // K rows
    __shared__ __attribute__((aligned(16))) f16 sV[2][BC * DH];   // V rows
    __shared__ __attribute__((aligned(16))) f16 sKt[2][BC * DH];  // K^T [DH][BC]

    const int H = p.H, N = p.N, NH = N * H;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, lg = lane >> 5;
    const int R0 = blockIdx.x * BR;
    const int rw0 = R0 + wave * 32;
    const int myrow = rw0 + l32;
    const bool row_ok = myrow < NH;
    const int qpos = min(myrow, NH - 1) / H;
    const int wpmax = min(rw0 + 31, NH - 1) / H;
    const int wpmin = min(rw0, NH - 1) / H;
    const int bpmax = min(R0 + BR - 1, NH - 1) / H;
    const int kend = CAUSAL ? min(N, bpmax + 1) : N;

    const f16* Qb = p.q + (int64_t)b * NH * DH;
    const f16* dOb = p.dO + (int64_t)b * NH * DH;
    const f16* Kb = p.k + (int64_t)b * N * DH;
    const f16* Vb = p.v + (int64_t)b * N * DH;
    const float my_lse2 = row_ok ? p.lse2_rows[(int64_t)b * NH + myrow] : 0.0f;
    const float my_d = row_ok ? p.d_rows[(int64_t)b * NH + myrow] : 0.0f;

    half8 qf[KS], gf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 a = {0u, 0u, 0u, 0u}, c = {0u, 0u, 0u, 0u};
        if (row_ok) {
            a = *reinterpret_cast<const u32x4*>(Qb + (int64_t)myrow * DH + ks * 16 + lg * 8);
            c = *reinterpret_cast<const u32x4*>(dOb + (int64_t)myrow * DH + ks * 16 + lg * 8);
        }
        qf[ks] = as_half8(a);
        gf[ks] = as_half8(c);
    }
    floatx16 dq[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) dq[t][e] = 0.0f;

    RowTile<BC, DH, 256> lk, lv;
    TransTile<BC, DH, 256> lkt;
    const int nkt = (kend + BC - 1) / BC;
    if (nkt > 0) {
        lk.load(Kb, 0, N); lv.load(Vb, 0, N); lkt.load(Kb, 0, N);
        lk.store(sK[0]); lv.store(sV[0]); lkt.store(sKt[0]);
    }
    __syncthreads();
    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) {
            lk.load(Kb, (kt + 1) * BC, N);
            lv.load(Vb, (kt + 1) * BC, N);
            lkt.load(Kb, (kt + 1) * BC, N);
        }
#pragma unroll
        for (int sub = 0; sub < BC / 32; ++sub) {
            const int key0 = kt * BC + sub * 32;
            if (key0 < kend && (!CAUSAL || key0 <= wpmax)) {
                floatx16 s, dp;
#pragma unroll
                for (int e = 0; e < 16; ++e) { s[e] = 0.0f; dp[e] = 0.0f; }
                const int arow = sub * 32 + pi32(l32);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    half8 a = *reinterpret_cast<const half8*>(sK[cur] + sw_off<DH>(arow, ks * 2 + lg));
                    half8 c = *reinterpret_cast<const half8*>(sV[cur] + sw_off<DH>(arow, ks * 2 + lg));
                    s = mfma32(a, qf[ks], s);
                    dp = mfma32(c, gf[ks], dp);
                }
                const bool need_mask = (key0 + 32 > N) || (CAUSAL && key0 + 31 > wpmin) || !row_ok;
                float ds[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    float pe = exp2f(s[e] * p.scale_log2 - my_lse2);
                    if (need_mask) {
                        int key = key0 + 16 * (e >> 3) + 8 * lg + (e & 7);
                        if (key >= N || (CAUSAL && key > qpos) || !row_ok) pe = 0.0f;
                    }
                    ds[e] = pe * (dp[e] - my_d);
                }
                const half8 b0 = pack8(&ds[0]), b1 = pack8(&ds[8]);
#pragma unroll
                for (int t = 0; t < DT; ++t) {
                    const int krow = t * 32 + l32;  // dh
                    half8 a0 = *reinterpret_cast<const half8*>(sKt[cur] + sw_off<BC>(krow, sub * 4 + 0 + lg));
                    half8 a1 = *reinterpret_cast<const half8*>(sKt[cur] + sw_off<BC>(krow, sub * 4 + 2 + lg));
                    dq[t] = mfma32(a0, b0, dq[t]);
                    dq[t] = mfma32(a1, b1, dq[t]);
                }
            }
        }
        if (more) {
            lk.store(sK[cur ^ 1]); lv.store(sV[cur ^ 1]); lkt.store(sKt[cur ^ 1]);
        }
        __syncthreads();
    }
    if (!row_ok) return;
    f16* dQr = p.out + (int64_t)b * NH * DH + (int64_t)myrow * DH;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const int dh = t * 32 + 8 * e4 + 4 * lg;
            u32x2 w = {pack_h2(dq[t][4 * e4] * p.scale, dq[t][4 * e4 + 1] * p.scale),
                       pack_h2(dq[t][4 * e4 + 2] * p.scale, dq[t][4 * e4 + 3] * p.scale)};
            *reinterpret_cast<u32x2*>(dQr + dh) = w;
        }
}

// ---------------------------------------------------------------------------
// Scalar fallbacks for head sizes without an MFMA kernel (any Dh <= 256).
// One thread per query row (forward / stats / dQ) or per key (dK, dV).
// ---------------------------------------------------------------------------
constexpr int SC_MAXDH = 256;

__global__ __launch_bounds__(64) void flash_fwd_scalar(FlashArgs p, int Dh, int causal, int mode) {
    const int NH = p.N * p.H;
    const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (idx >= (int64_t)p.B * NH) return;
    const int b = (int)(idx / NH), r = (int)(idx % NH), pos = r / p.H, h = r % p.H;
    const f16* qr = p.q + idx * Dh;
    const f16* gr = mode ? p.dO + idx * Dh : nullptr;
    float acc[SC_MAXDH];
    for (int d = 0; d < Dh; ++d) acc[d] = 0.0f;
    float m = -INFINITY, l = 0.0f, t = 0.0f;
    const int L = causal ? pos + 1 : p.N;
    for (int j = 0; j < L; ++j) {
        const f16* kr = p.k + ((int64_t)b * p.N + j) * Dh;
        const f16* vr = p.v + ((int64_t)b * p.N + j) * Dh;
        float s = 0.0f, dpv = 0.0f;
        for (int d = 0; d < Dh; ++d) {
            s += (float)qr[d] * (float)kr[d];
            if (mode) dpv += (float)gr[d] * (float)vr[d];
        }
        s *= p.scale_log2;
        float mn = fmaxf(m, s);
        float al = exp2f(m - mn), pe = exp2f(s - mn);
        l = l * al + pe;
        t = t * al + pe * dpv;
        if (!mode)
            for (int d = 0; d < Dh; ++d) acc[d] = acc[d] * al + pe * (float)vr[d];
        m = mn;
    }
    const float il = l > 0.0f ? 1.0f / l : 0.0f;
    if (!mode) {
        for (int d = 0; d < Dh; ++d) p.out[idx * Dh + d] = (f16)(acc[d] * il);
        if (p.lse) p.lse[((int64_t)b * p.H + h) * p.N + pos] = (m + log2f(l)) * kLn2;
    } else {
        p.lse2_rows[idx] = m + log2f(l);
        p.d_rows[idx] = t * il;
    }
}

__global__ __launch_bounds__(64) void flash_dq_scalar(FlashArgs p, int Dh, int causal) {
    const int NH = p.N * p.H;
    const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (idx >= (int64_t)p.B * NH) return;
    const int b = (int)(idx / NH), r = (int)(idx % NH), pos = r / p.H;
    const f16* qr = p.q + idx * Dh;
    const f16* gr = p.dO + idx * Dh;
    float acc[SC_MAXDH];
    for (int d = 0; d < Dh; ++d) acc[d] = 0.0f;
    const float l2 = p.lse2_rows[idx], Di = p.d_rows[idx];
    const int L = causal ? pos + 1 : p.N;
    for (int j = 0; j < L; ++j) {
        const f16* kr = p.k + ((int64_t)b * p.N + j) * Dh;
        const f16* vr = p.v + ((int64_t)b * p.N + j) * Dh;
        float s = 0.0f, dpv = 0.0f;
        for (int d = 0; d < Dh; ++d) {
            s += (float)qr[d] * (float)kr[d];
            dpv += (float)gr[d] * (float)vr[d];
        }
        float pe = exp2f(s * p.scale_log2 - l2);
        float ds = pe * (dpv - Di);
        for (int d = 0; d < Dh; ++d) acc[d] += ds * (float)kr[d];
    }
    for (int d = 0; d < Dh; ++d) p.out[idx * Dh + d] = (f16)(acc[d] * p.scale);
}

__global__ __launch_bounds__(64) void flash_dkdv_scalar(FlashArgs p, int Dh, int causal) {
    const int NH = p.N * p.H;
    const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (idx >= (int64_t)p.B * p.N) return;
    const int b = (int)(idx / p.N), j = (int)(idx % p.N);
    const f16* kr = p.k + idx * Dh;
    const f16* vr = p.v + idx * Dh;
    float ak[SC_MAXDH], av[SC_MAXDH];
    for (int d = 0; d < Dh; ++d) { ak[d] = 0.0f; av[d] = 0.0f; }
    const int rs = causal ? j * p.H : 0;
    for (int r = rs; r < NH; ++r) {
        const int64_t ri = (int64_t)b * NH + r;
        const f16* qr = p.q + ri * Dh;
        const f16* gr = p.dO + ri * Dh;
        float s = 0.0f, dpv = 0.0f;
        for (int d = 0; d < Dh; ++d) {
            s += (float)qr[d] * (float)kr[d];
            dpv += (float)gr[d] * (float)vr[d];
        }
        float pe = exp2f(s * p.scale_log2 - p.lse2_rows[ri]);
        float ds = pe * (dpv - p.d_rows[ri]);
        for (int d = 0; d < Dh; ++d) {
            av[d] += pe * (float)gr[d];
            ak[d] += ds * (float)qr[d];
        }
    }
    for (int d = 0; d < Dh; ++d) {
        p.dK[idx * Dh + d] = (f16)(ak[d] * p.scale);
        p.dV[idx * Dh + d] = (f16)av[d];
    }
}

__global__ __launch_bounds__(256) void flash_bwd_pre_scalar(FlashArgs p, int Dh) {
    const int NH = p.N * p.H;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.B * NH) return;
    const int b = (int)(idx / NH), r = (int)(idx % NH);
    float acc = 0.0f;
    for (int d = 0; d < Dh; ++d) acc += (float)p.o[idx * Dh + d] * (float)p.dO[idx * Dh + d];
    p.d_rows[idx] = acc;
    p.lse2_rows[idx] = p.lse[((int64_t)b * p.H + (r % p.H)) * p.N + r / p.H] * kLog2e;
}

// Workspace for the backward statistics (grow-only).
// Backward workspace (grow-only byte arena): row statistics, fp32 dK/dV
// partials, and O / LSE of a recomputed forward.
char* g_bwd_ws = nullptr;
size_t g_bwd_ws_bytes = 0;

template <int DH>
hipError_t launch_fwd(const FlashArgs& a, bool causal, int mode, hipStream_t st) {
    const int nrg = (a.N * a.H + FR - 1) / FR;
    dim3 grid(nrg * a.B);
    // zigzag round = one workgroup per CU: round r+1 runs in reverse, so the
    // workgroups that land on the same CU pair heavy with light row groups
    const int round = device_cu_count();
    if constexpr (DH <= 64) {
        // buffer offsets are 32-bit: one batch of K (or V) must stay below 2 GiB
        if (mode == 0 && (int64_t)a.N * DH * 2 < (int64_t)INT32_MAX) {
            constexpr int QB = FWD_KS_QB;
            const int64_t nrg_ks = ((int64_t)a.N * a.H + 16 * QB - 1) / (16 * QB);
            dim3 gk((unsigned)((nrg_ks + 1) / 2 * a.B));
            if (causal) hipLaunchKernelGGL((flash_fwd_ks<DH, QB, true>), gk, dim3(512), 0, st, a);
            else hipLaunchKernelGGL((flash_fwd_ks<DH, QB, false>), gk, dim3(512), 0, st, a);
            return hipGetLastError();
        }
    }
    if (mode == 0) {
        if (causal) hipLaunchKernelGGL((flash_fwd<DH, true, 0>), grid, dim3(512), 0, st, a, round);
        else hipLaunchKernelGGL((flash_fwd<DH, false, 0>), grid, dim3(512), 0, st, a, round);
    } else {
        if (causal) hipLaunchKernelGGL((flash_fwd<DH, true, 1>), grid, dim3(512), 0, st, a, round);
        else hipLaunchKernelGGL((flash_fwd<DH, false, 1>), grid, dim3(512), 0, st, a, round);
    }
    return hipGetLastError();
}

template <int DH>
hipError_t launch_bwd(const FlashArgs& a, bool causal, bool have_lse, hipStream_t st) {
    const int NH = a.N * a.H;
    if (have_lse) {
        dim3 g((unsigned)(((int64_t)a.B * NH * (DH / 8) + 255) / 256));
        hipLaunchKernelGGL(flash_bwd_pre<DH>, g, dim3(256), 0, st, a);
    } else {
        hipError_t e = launch_fwd<DH>(a, causal, 1, st);
        if (e != hipSuccess) return e;
    }
    dim3 gk((a.N + 31) / 32, a.B);
    dim3 gq((NH + BR - 1) / BR, a.B);
    if (causal) {
        hipLaunchKernelGGL((flash_bwd_dkdv<DH, true>), gk, dim3(256), 0, st, a);
        hipLaunchKernelGGL((flash_bwd_dq<DH, true>), gq, dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((flash_bwd_dkdv<DH, false>), gk, dim3(256), 0, st, a);
        hipLaunchKernelGGL((flash_bwd_dq<DH, false>), gq, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// dK/dV by key blocks and row parts, then dQ by row tiles (head dims 32, 64).
template <int DH>
hipError_t launch_bwd_split(const FlashArgs& a, bool causal, float* parts, int parts_per_batch,
                            hipStream_t st) {
    const int NH = a.N * a.H;
    const int n_kv = a.B * parts_per_batch;
    dim3 gm((unsigned)(n_kv + (NH + 63) / 64 * a.B));
    const int nkb = (a.N + BKB - 1) / BKB;
    dim3 gr((unsigned)(a.B * nkb * 16));
    if (causal) {
        hipLaunchKernelGGL((flash_bwd_kvq<DH, true>), gm, dim3(256), 0, st, a, parts, parts_per_batch, n_kv);
        hipLaunchKernelGGL((flash_bwd_kv_reduce<DH, true>), gr, dim3(256), 0, st, a, parts, parts_per_batch);
    } else {
        hipLaunchKernelGGL((flash_bwd_kvq<DH, false>), gm, dim3(256), 0, st, a, parts, parts_per_batch, n_kv);
        hipLaunchKernelGGL((flash_bwd_kv_reduce<DH, false>), gr, dim3(256), 0, st, a, parts, parts_per_batch);
    }
    return hipGetLastError();
}

}  // namespace

int flash_status(uint32_t* flags, bool clear) {
    unsigned v = 0;
    EVK_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_flash_status), sizeof(v), 0, hipMemcpyDeviceToHost));
    if (clear && v) {
        const unsigned zero = 0;
        EVK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_flash_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice));
    }
    *flags = v;
    return EVKHIP_OK;
}

void flash_set_spin_limit(uint32_t n) {
    g_spin_limit = n == 0 ? kDefaultSpinLimit : (int)std::min<uint32_t>(n - 1, (uint32_t)INT32_MAX);
}

uint32_t flash_spin_limit() { return (uint32_t)g_spin_limit; }

void flash_free_workspace() {
    if (g_bwd_ws) (void)hipFree(g_bwd_ws);
    g_bwd_ws = nullptr;
    g_bwd_ws_bytes = 0;
}

int flash_forward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st) {
    a.spin_limit = g_spin_limit;
    a.scale = 1.0f / sqrtf((float)dh);
    a.scale_log2 = a.scale * kLog2e;
    hipError_t e;
    if (mfma && dh == 32) e = launch_fwd<32>(a, causal, 0, st);
    else if (mfma && dh == 64) e = launch_fwd<64>(a, causal, 0, st);
    else if (mfma && dh == 128) e = launch_fwd<128>(a, causal, 0, st);
    else if (mfma && flash_wide_head(dh) && flash_wide_fits(a.N, a.H, dh)) e = flash_forward_wide(a, dh, causal, st);
    else {
        dim3 g((unsigned)(((int64_t)a.B * a.N * a.H + 63) / 64));
        hipLaunchKernelGGL(flash_fwd_scalar, g, dim3(64), 0, st, a, dh, (int)causal, 0);
        e = hipGetLastError();
    }
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "flash forward launch");
}

int flash_backward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st) {
    a.spin_limit = g_spin_limit;
    a.scale = 1.0f / sqrtf((float)dh);
    a.scale_log2 = a.scale * kLog2e;
    const size_t rows = (size_t)a.B * a.N * a.H;
    const bool have_lse = a.lse != nullptr;
    const bool split = mfma && dh <= 64 && !flash_wide_head(dh) && (int64_t)a.N * a.H * dh * 2 < (int64_t)INT32_MAX;
    const bool wide = mfma && flash_wide_head(dh) && flash_wide_fits(a.N, a.H, dh);
    // arena layout (256-byte aligned pieces)
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int nkb = (a.N + BKB - 1) / BKB;
    int parts_per_batch = 0;
    if (split)
        for (int kb = 0; kb < nkb; ++kb) parts_per_batch += bwd_kv_parts(kb, a.N, a.H, causal);
    const size_t stats_b = (split || wide) ? 0 : al(2 * rows * sizeof(float));  // formed in-kernel
    const size_t part_b = split ? al((size_t)a.B * parts_per_batch * 4 * (2 * 2 * (dh / 16)) * 64 * 16) : 0;
    const size_t fwd_b = ((split || wide) && !have_lse) ? al(rows * dh * 2) + al(rows * sizeof(float)) : 0;
    const size_t need = stats_b + part_b + fwd_b;
    if (need > g_bwd_ws_bytes) {
        if (g_bwd_ws) EVK_HIP(hipFree(g_bwd_ws));
        g_bwd_ws = nullptr;
        g_bwd_ws_bytes = 0;
        EVK_HIP(hipMalloc(&g_bwd_ws, need));
        g_bwd_ws_bytes = need;
    }
    a.lse2_rows = split ? nullptr : reinterpret_cast<float*>(g_bwd_ws);
    a.d_rows = split ? nullptr : a.lse2_rows + rows;
    hipError_t e;
    if (split) {
        float* parts = reinterpret_cast<float*>(g_bwd_ws + stats_b);
        if (!have_lse) {
            // recompute the forward's O and LSE into the arena
            FlashArgs f = a;
            f16* o_ws = reinterpret_cast<f16*>(g_bwd_ws + stats_b + part_b);
            float* l_ws = reinterpret_cast<float*>(g_bwd_ws + stats_b + part_b + al(rows * dh * 2));
            f.out = o_ws;
            f.lse = l_ws;
            e = (dh == 32) ? launch_fwd<32>(f, causal, 0, st) : launch_fwd<64>(f, causal, 0, st);
            if (e != hipSuccess) return check_hip(e, "flash backward: forward recompute");
            a.o = o_ws;
            a.lse = l_ws;
        }
        e = (dh == 32) ? launch_bwd_split<32>(a, causal, parts, parts_per_batch, st)
                       : launch_bwd_split<64>(a, causal, parts, parts_per_batch, st);
    } else if (wide) {
        if (!have_lse) {
            // recompute the forward's O and LSE into the arena
            FlashArgs f = a;
            f.out = reinterpret_cast<f16*>(g_bwd_ws + stats_b);
            f.lse = reinterpret_cast<float*>(g_bwd_ws + stats_b + al(rows * dh * 2));
            e = flash_forward_wide(f, dh, causal, st);
            if (e != hipSuccess) return check_hip(e, "flash backward: forward recompute");
            a.o = f.out;
            a.lse = f.lse;
        }
        e = flash_backward_wide(a, dh, causal, st);
    } else if (mfma && dh == 32) {
        e = launch_bwd<32>(a, causal, have_lse, st);
    } else if (mfma && dh == 64) {
        e = launch_bwd<64>(a, causal, have_lse, st);
    } else if (mfma && dh == 128) {
        e = launch_bwd<128>(a, causal, have_lse, st);
    } else {
        dim3 g((unsigned)((rows + 63) / 64));
        if (have_lse) {
            hipLaunchKernelGGL(flash_bwd_pre_scalar, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                               a, dh);
        } else {
            hipLaunchKernelGGL(flash_fwd_scalar, g, dim3(64), 0, st, a, dh, (int)causal, 1);
        }
        hipLaunchKernelGGL(flash_dq_scalar, g, dim3(64), 0, st, a, dh, (int)causal);
        dim3 gk((unsigned)(((int64_t)a.B * a.N + 63) / 64));
        hipLaunchKernelGGL(flash_dkdv_scalar, gk, dim3(64), 0, st, a, dh, (int)causal);
        e = hipGetLastError();
    }
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "flash backward launch");
}

}  // namespace evkhip
