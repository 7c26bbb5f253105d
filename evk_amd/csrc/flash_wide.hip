// Flash attention forward / backward on the MFMA for head sizes the
// specialised kernels of flash.hip do not cover: any multiple of 16 up to
// 256 (the reference's flash shader takes Dh <= 256, flash_attention.comp:46;
// its only training caller runs one head of 256, example/main_llm.cpp:694-702
// through Graph::causal_attention, evk_ai.h:961-1007).
//
// Layout as in flash.hip (reference MQA): Q,O,dO,dQ (B,N,H*Dh); K,V,dK,dV
// (B,N,Dh); per batch the query side is an (N*H) x Dh matrix whose row r is
// position r/H of head r%H.
//
// MFMA forms (lane l, g = l/16, l16 = l%16):
//   contractions over Dh: v_mfma_f32_16x16x32_f16 per 32 dims (A row l16,
//       B column l16, k = 8g..8g+7 of the step; the A fragment is one
//       16-byte LDS read), and for Dh an odd multiple of 16 one
//       v_mfma_f32_16x16x16_f16 for the last 16 (k = 4g..4g+3); D column
//       l16, rows 4g+j.
//   v_mfma_f32_16x16x32_f16 for contractions over 32 keys or 32 rows:
//       operand slot s of lane l holds k = 4g+s (s < 4) or 16+4g+s-4, which
//       is exactly how two 16-wide D blocks lay out their rows, so
//       probabilities go from one MFMA's result to the next one's operand
//       without moving; the other operand comes from a row-major LDS tile
//       through ds_read_b64_tr_b16 (rows 4g.. and 16+4g.., 16 columns).
// Every score is scaled in fp32 (s * scale * log2(e), exp2 domain).
#include "kernels.h"

#include <math.h>

namespace evkhip {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int WKC = 32;   // keys (or rows) per chunk

DEV floatx4 mfma_k16(const half4& a, const half4& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
DEV half8 pack_slots(const floatx4& x0, const floatx4& x1) {
    u32x4 u = {pack_h2(x0[0], x0[1]), pack_h2(x0[2], x0[3]), pack_h2(x1[0], x1[1]), pack_h2(x1[2], x1[3])};
    return as_half8(u);
}

// WKC rows x DH halves of a (rows, DH) row-major matrix, loaded into
// registers by the workgroup's 256 threads and stored into an LDS tile with
// rows of DH + 8 halves (the next tile's loads fly during the current one).
// Rows outside the buffer descriptor read as zeros.
template <int DH>
struct WideTile {
    static constexpr int W = DH + 8;
    static constexpr int PIECES = WKC * DH / 8;  // 16-byte pieces
    static constexpr int PER = (PIECES + 255) / 256;
    u32x4 r[PER];
    DEV void load(__amdgpu_buffer_rsrc_t res, int row0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int pc = threadIdx.x + 256 * i;
            const int row = pc / (DH / 8), col = (pc % (DH / 8)) * 8;
            const bool ok = PIECES % 256 == 0 || pc < PIECES;
            r[i] = buf_load16(res, oob_or(ok, (uint32_t)((row0 + row) * DH + col) * 2u), 0);
        }
    }
    DEV void store(f16* lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int pc = threadIdx.x + 256 * i;
            if (PIECES % 256 == 0 || pc < PIECES) {
                const int row = pc / (DH / 8), col = (pc % (DH / 8)) * 8;
                *reinterpret_cast<u32x4*>(lds + row * W + col) = r[i];
            }
        }
    }
};

// 4 halves at element `elem` through a buffer descriptor (zeros unless ok)
DEV half4 ld_h4(__amdgpu_buffer_rsrc_t res, bool ok, int elem) {
    const uint32_t off = oob_or(ok, (uint32_t)elem * 2u);
    return __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(res, off, 0, 0));
}

// A operand of a 16x16x32 MFMA from a row-major LDS tile (rows of W
// halves): column c0 + l16 of rows {4g..4g+3, 16+4g..16+4g+3} (slot order).
template <int W>
DEV half8 tile_tr(const f16* t, int c0, int g, int trow, int tcol) {
    const f16* base = t + (4 * g + trow) * W + c0 + tcol;
    return cat4(lds_read_tr(base), lds_read_tr(base + 16 * W));
}

// One row of DH halves (a query, key or dO row) as B fragments of the Dh
// contraction: m[ks] holds dims 32 ks + 8 g .. +7, t the tail dims
// 32 K32 + 4 g .. +3 when DH is an odd multiple of 16.
template <int DH>
struct RowFrag {
    static constexpr int K32 = DH / 32;
    static constexpr bool TAIL = DH % 32 != 0;
    half8 m[K32 > 0 ? K32 : 1];
    half4 t;
    DEV void load(__amdgpu_buffer_rsrc_t res, bool ok, int row, int g) {
#pragma unroll
        for (int ks = 0; ks < K32; ++ks)
            m[ks] = as_half8(buf_load16(res, oob_or(ok, (uint32_t)(row * DH + 32 * ks + 8 * g) * 2u), 0));
        if (TAIL) t = ld_h4(res, ok, row * DH + 32 * K32 + 4 * g);
    }
};

// One 16 x 16 block of D = A B^T contracted over the 32-wide steps
// [S0, S1) of DH, plus the 16-wide tail when TAIL: A rows r0 + l16 of the
// LDS tile a (rows of W halves; W * 2 bytes is an odd multiple of 16, so
// the 16 rows of a 16-byte read hit distinct banks), B fragments bf; D
// element j: row r0 + 4 g + j, column l16.  Every A fragment is requested
// before the first MFMA.
template <int DH, int W, int S0, int S1, bool TAIL>
DEV floatx4 contract_steps(const f16* a, int r0, const RowFrag<DH>& bf, int l16, int g) {
    const f16* row = a + (r0 + l16) * W;
    half8 fr[S1 > S0 ? S1 - S0 : 1];
    half4 tl;
#pragma unroll
    for (int ks = S0; ks < S1; ++ks) fr[ks - S0] = *reinterpret_cast<const half8*>(row + 32 * ks + 8 * g);
    if (TAIL) tl = *reinterpret_cast<const half4*>(row + 32 * RowFrag<DH>::K32 + 4 * g);
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = S0; ks < S1; ++ks) acc = mfma16(fr[ks - S0], bf.m[ks], acc);
    if (TAIL) {
        // the tail goes to an accumulator of its own: a 16x16x16 MFMA that
        // takes a 16x16x32 MFMA's result as its C operand right behind it
        // read wrong values on MI355X
        const floatx4 t = mfma_k16(tl, bf.t, floatx4{0.f, 0.f, 0.f, 0.f});
        acc = (S1 > S0) ? acc + t : t;
    }
    return acc;
}
template <int DH, int W>
DEV floatx4 contract_full(const f16* a, int r0, const RowFrag<DH>& bf, int l16, int g) {
    return contract_steps<DH, W, 0, RowFrag<DH>::K32, RowFrag<DH>::TAIL>(a, r0, bf, l16, g);
}

// The four waves of a workgroup hand 16 x 16 fp32 blocks to each other
// through LDS: wave w writes its block at x + 64 w lanes (16 bytes a lane,
// the same lane-to-element map in every wave), and after a barrier any wave
// reads block w' at the same lane.
DEV void xput(floatx4* x, int wave, int lane, const floatx4& v) { x[wave * 64 + lane] = v; }
DEV floatx4 xget(const floatx4* x, int w, int lane) { return x[w * 64 + lane]; }
constexpr int XBYTES = 4 * 64 * 16;

// dh blocks (16 wide) of a wave when four waves share DB of them
template <int DB>
struct DhShare {
    static constexpr int PER = (DB + 3) / 4;
};

// ---------------------------------------------------------------------------
// Forward: O and the public LSE.  Grid (ceil(N*H/16), B), 4 waves per
// workgroup for 16 query rows R0 + l16 (the B operand Q^T in registers).
// K and V come in 32-key tiles staged in LDS for the workgroup (double
// buffered).  The tile's scores are two 16 x 16 blocks (keys 0-15, 16-31);
// wave w contracts block w % 2 over one half of Dh (w / 2), the four parts
// go through LDS, and every wave adds them up and forms the probabilities
// itself, then multiplies them into dh blocks w, w+4, ... of the output:
//   S^T(16 keys x 16 q) = K Q^T   (contraction over Dh, split in halves)
//   O^T(16 dh x 16 q) += V^T P^T  (16x16x32, V^T by tr reads)
//   row sums: ones . P^T on the MFMA.
// Rescaling is lazy: a row's reference maximum moves only when a chunk has a
// score more than 2^8 above it.
// ---------------------------------------------------------------------------
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256) void flash_fwd_wide(FlashArgs p) {
    constexpr int DB = DH / 16, DPW = DhShare<DB>::PER, W = WideTile<DH>::W;
    __shared__ __attribute__((aligned(16))) f16 sK[2][WKC * W];
    __shared__ __attribute__((aligned(16))) f16 sV[2][WKC * W];
    __shared__ floatx4 sX[4 * 64];

    const int H = p.H, N = p.N, NH = N * H;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4, trow = l16 >> 2, tcol = (l16 & 3) * 4;
    constexpr int K32 = RowFrag<DH>::K32, HS = (K32 + 1) / 2;  // the first half: steps [0, HS)
    const int R0 = blockIdx.x * 16;
    const int myrow = R0 + l16;
    const bool row_ok = myrow < NH;
    const int qpos = min(myrow, NH - 1) / H;
    const int pmax = min(R0 + 15, NH - 1) / H, pmin = R0 / H;
    const int kend = CAUSAL ? min(N, pmax + 1) : N;
    const float c2 = p.scale_log2;

    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(p.k + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(p.v + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t qres = buf_rsrc(p.q + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);

    // the first tile's loads go out first (they do not depend on Q), then Q
    WideTile<DH> lk, lv;
    const int nkt = (kend + WKC - 1) / WKC;
    if (nkt > 0) {
        lk.load(kres, 0);
        lv.load(vres, 0);
    }
    RowFrag<DH> qf;
    qf.load(qres, row_ok, myrow, g);
    // drain these loads here: inside the loop the only loads in flight are
    // then the next tile's, which the loop waits for at its LDS store only
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    floatx4 oacc[DPW];
#pragma unroll
    for (int i = 0; i < DPW; ++i) oacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 lacc = {0.f, 0.f, 0.f, 0.f};
    float m_ref = -INFINITY;
    const half8 ones8 = {(f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f};

    if (nkt > 0) {
        lk.store(sK[0]);
        lv.store(sV[0]);
    }
    __syncthreads();
    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) {
            lk.load(kres, (kt + 1) * WKC);
            lv.load(vres, (kt + 1) * WKC);
        }
        const int key0 = kt * WKC;
        // element j of s[kb]: key key0 + 16 kb + 4 g + j, query myrow
        {
            const floatx4 part = (wave & 2) ? contract_steps<DH, W, HS, K32, RowFrag<DH>::TAIL>(sK[cur], 16 * (wave & 1), qf, l16, g)
                                            : contract_steps<DH, W, 0, HS, false>(sK[cur], 16 * (wave & 1), qf, l16, g);
            xput(sX, wave, lane, part);
        }
        __syncthreads();
        floatx4 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) s[kb] = xget(sX, kb, lane) + xget(sX, kb + 2, lane);
        if ((key0 + WKC > N) || (CAUSAL && key0 + WKC - 1 > pmin)) {
            const int lim = (CAUSAL ? min(N - 1, qpos) : N - 1) - key0 - 4 * g;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[kb][j] = (kb * 16 + j > lim) ? -INFINITY : s[kb][j];
        }
        float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3]))) * c2;
        if (__any(mx > m_ref + 8.0f)) {
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_ref, mx);
            const float alpha = (m_ref == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
#pragma unroll
            for (int i = 0; i < DPW; ++i) oacc[i] *= alpha;
            lacc *= alpha;
            m_ref = m_new;
        }
        const float nbase = (m_ref == -INFINITY) ? 0.0f : -m_ref;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) s[kb][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][j], c2, nbase));
        const half8 pb = pack_slots(s[0], s[1]);
        lacc = mfma16(ones8, pb, lacc);
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const int d = wave + 4 * i;
            if (DB % 4 == 0 || d < DB) oacc[i] = mfma16(tile_tr<W>(sV[cur], d * 16, g, trow, tcol), pb, oacc[i]);
        }
        if (more) {
            lk.store(sK[cur ^ 1]);
            lv.store(sV[cur ^ 1]);
        }
        __syncthreads();
    }
    if (!row_ok) return;
    const float l = lacc[0];
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    f16* orow = p.out + ((int64_t)b * NH + myrow) * DH;
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const int d = wave + 4 * i;
        if (DB % 4 == 0 || d < DB) {
            const u32x2 w2 = {pack_h2(oacc[i][0] * inv, oacc[i][1] * inv), pack_h2(oacc[i][2] * inv, oacc[i][3] * inv)};
            *reinterpret_cast<u32x2*>(orow + d * 16 + g * 4) = w2;
        }
    }
    if (p.lse && wave == 0 && g == 0)
        p.lse[((int64_t)b * H + myrow % H) * N + qpos] = l > 0.0f ? (m_ref + log2f(l)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// dK, dV (blocks of flash_bwd_wide).  4 waves; a workgroup owns 16 keys k0 + l16
// (K^T, V^T as B-operand registers) and walks every query row at or after
// k0 in 32-row tiles of Q and dO (with their lse2 and D) staged in LDS for
// the workgroup, so the MQA sum over heads happens in the accumulation.
// The tile's S and dP are four 16 x 16 blocks (rows 0-15, 16-31 of each);
// wave w contracts block w and hands it to the others through LDS.  Every
// wave forms the tile's P and dS itself; wave w accumulates dh blocks
// w, w+4, ... of dK and dV:
//   S, dP (16 rows x 16 keys) = Q K^T, dO V^T  (contractions over DH)
//   P = 2^(S c - lse2_row), dS = P (dP - D_row)
//   dV^T(16 dh x 16 keys) += dO^T P, dK^T += Q^T dS  (16x16x32 over rows)
// ---------------------------------------------------------------------------
// Dot product of two 16-byte pieces (8 halves each), in fp32.
DEV float dot8(const u32x4& a, const u32x4& b) {
    const half8 x = as_half8(a), y = as_half8(b);
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf((float)x[e], (float)y[e], acc);
    return acc;
}

// LDS of a flash_bwd_wide workgroup, either role: two double-buffered
// 32-row tiles, then (dK/dV) the tiles' lse2 and D, the block exchange and
// the per-piece dO . O products of the next tile
template <int DH>
constexpr int bwd_wide_lds() {
    return 2 * 2 * WKC * WideTile<DH>::W * 2 + 2 * 2 * WKC * 4 + XBYTES + WideTile<DH>::PIECES * 4;
}

template <int DH, bool CAUSAL>
__device__ void bwd_dkdv_wide(const FlashArgs& p, int bx, char* lds) {
    constexpr int DB = DH / 16, DPW = DhShare<DB>::PER, W = WideTile<DH>::W;
    f16 (*sQ)[WKC * W] = reinterpret_cast<f16 (*)[WKC * W]>(lds);
    f16 (*sG)[WKC * W] = reinterpret_cast<f16 (*)[WKC * W]>(lds + 2 * WKC * W * 2);
    float (*sL)[WKC] = reinterpret_cast<float (*)[WKC]>(lds + 4 * WKC * W * 2);
    float (*sD)[WKC] = reinterpret_cast<float (*)[WKC]>(lds + 4 * WKC * W * 2 + 2 * WKC * 4);
    floatx4* sX = reinterpret_cast<floatx4*>(lds + 4 * WKC * W * 2 + 4 * WKC * 4);
    float* sPart = reinterpret_cast<float*>(lds + 4 * WKC * W * 2 + 4 * WKC * 4 + XBYTES);

    const int H = p.H, N = p.N, NH = N * H;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4, trow = l16 >> 2, tcol = (l16 & 3) * 4;
    const int k0 = bx * 16;
    const int mykey = k0 + l16;
    const bool key_ok = mykey < N;
    const float c2 = p.scale_log2;

    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(p.k + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(p.v + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t qres = buf_rsrc(p.q + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t gres = buf_rsrc(p.dO + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t ores = buf_rsrc(p.o + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t lres = buf_rsrc(p.lse + (int64_t)b * H * N, (uint32_t)(H * N) * 4u);

    RowFrag<DH> kf, vf;
    kf.load(kres, key_ok, mykey, g);
    vf.load(vres, key_ok, mykey, g);
    floatx4 dk[DPW], dv[DPW];
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        dk[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        dv[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    // rows of positions >= k0 (causal), in tiles of 32
    const int rstart = CAUSAL ? min(NH, k0 * H) / WKC * WKC : 0;
    const int nrt = (NH - rstart + WKC - 1) / WKC;
    // per row of a tile: lse2 = LSE * log2(e) of (position, head), and
    // D = rowsum(dO * O).  The LSE is loaded as it is and scaled when it goes
    // to LDS: arithmetic on it at the load would make the wave wait there for
    // every load in flight, the next tile's included.  O comes in the dO
    // tile's piece layout; each thread stores the dot products of its pieces
    // and, after the next barrier, the first WKC threads add their row's
    // DH / 8 products in order.
    constexpr int PPR = DH / 8;  // pieces per row
    WideTile<DH> lq, lg, lo;
    float lsv = 0.0f;
    auto load_tile = [&](int t) {
        const int r0 = rstart + t * WKC;
        lq.load(qres, r0);
        lg.load(gres, r0);
        lo.load(ores, r0);
        const int r = r0 + (int)threadIdx.x;
        lsv = buf_load_f32(lres, oob_or(threadIdx.x < WKC && r < NH, (uint32_t)((r % H) * N + r / H) * 4u));
    };
    auto stage_tile = [&](int st) {
        lq.store(sQ[st]);
        lg.store(sG[st]);
#pragma unroll
        for (int i = 0; i < WideTile<DH>::PER; ++i) {
            const int pc = threadIdx.x + 256 * i;
            if (WideTile<DH>::PIECES % 256 == 0 || pc < WideTile<DH>::PIECES) sPart[pc] = dot8(lg.r[i], lo.r[i]);
        }
        if (threadIdx.x < WKC) sL[st][threadIdx.x] = lsv * kLog2e;
    };
    auto finish_d = [&](int st) {
        if (threadIdx.x < WKC) {
            float d = 0.0f;
#pragma unroll
            for (int c = 0; c < PPR; ++c) d += sPart[threadIdx.x * PPR + c];
            sD[st][threadIdx.x] = d;
        }
    };
    if (nrt > 0) load_tile(0);
    // drain the key operands' and the first tile's loads together: inside
    // the loop only the next tile's loads are then in flight (see
    // flash_fwd_wide)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    if (nrt > 0) stage_tile(0);
    __syncthreads();
    for (int rt = 0; rt < nrt; ++rt) {
        const int cur = rt & 1;
        const bool more = rt + 1 < nrt;
        if (more) load_tile(rt + 1);
        finish_d(cur);
        const int r0 = rstart + rt * WKC;
        // element j of s[rb]: row r0 + 16 rb + 4 g + j, key mykey
        // wave w: block w of S rows 0-15, 16-31, then dP rows 0-15, 16-31
        xput(sX, wave, lane, contract_full<DH, W>((wave & 2) ? sG[cur] : sQ[cur], 16 * (wave & 1),
                                                  (wave & 2) ? vf : kf, l16, g));
        __syncthreads();
        const floatx4 s[2] = {xget(sX, 0, lane), xget(sX, 1, lane)}, dp[2] = {xget(sX, 2, lane), xget(sX, 3, lane)};
        floatx4 pe[2], ds[2];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rl = rb * 16 + 4 * g + j, r = r0 + rl;
                const bool ok = r < NH && key_ok && (!CAUSAL || mykey <= r / H);
                const float pv = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[rb][j], c2, -sL[cur][rl])) : 0.0f;
                pe[rb][j] = pv;
                ds[rb][j] = pv * (dp[rb][j] - sD[cur][rl]);
            }
        const half8 pb = pack_slots(pe[0], pe[1]), sb = pack_slots(ds[0], ds[1]);
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const int d = wave + 4 * i;
            if (DB % 4 == 0 || d < DB) {
                dv[i] = mfma16(tile_tr<W>(sG[cur], d * 16, g, trow, tcol), pb, dv[i]);
                dk[i] = mfma16(tile_tr<W>(sQ[cur], d * 16, g, trow, tcol), sb, dk[i]);
            }
        }
        if (more) stage_tile(cur ^ 1);
        __syncthreads();
    }
    if (!key_ok) return;
    // element j of dk[i]: dh 16 d + 4 g + j of key mykey
    f16* kdst = p.dK + ((int64_t)b * N + mykey) * DH;
    f16* vdst = p.dV + ((int64_t)b * N + mykey) * DH;
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const int d = wave + 4 * i;
        if (DB % 4 == 0 || d < DB) {
            const u32x2 a = {pack_h2(dk[i][0] * p.scale, dk[i][1] * p.scale), pack_h2(dk[i][2] * p.scale, dk[i][3] * p.scale)};
            const u32x2 c = {pack_h2(dv[i][0], dv[i][1]), pack_h2(dv[i][2], dv[i][3])};
            *reinterpret_cast<u32x2*>(kdst + d * 16 + g * 4) = a;
            *reinterpret_cast<u32x2*>(vdst + d * 16 + g * 4) = c;
        }
    }
}

// ---------------------------------------------------------------------------
// dQ (blocks of flash_bwd_wide).  4 waves for 16 query rows (Q^T and dO^T as B
// operands); K and V in 32-key tiles staged in LDS as in the forward; the
// tile's S^T and dP^T are four 16 x 16 blocks, one per wave, handed over
// through LDS; every wave forms dS, wave w accumulates dh blocks w, w+4,
// ... of dQ:
//   S^T, dP^T (16 keys x 16 q) = K Q^T, V dO^T  (contractions over DH)
//   dS^T = P^T (dP^T - D), P = 2^(S c - lse2_row)
//   dQ^T(16 dh x 16 q) += K^T dS^T  (16x16x32 over keys, K^T by tr reads)
// ---------------------------------------------------------------------------
template <int DH, bool CAUSAL>
__device__ void bwd_dq_wide(const FlashArgs& p, int bx, char* lds) {
    constexpr int DB = DH / 16, DPW = DhShare<DB>::PER, W = WideTile<DH>::W;
    f16 (*sK)[WKC * W] = reinterpret_cast<f16 (*)[WKC * W]>(lds);
    f16 (*sV)[WKC * W] = reinterpret_cast<f16 (*)[WKC * W]>(lds + 2 * WKC * W * 2);
    floatx4* sX = reinterpret_cast<floatx4*>(lds + 4 * WKC * W * 2 + 4 * WKC * 4);

    const int H = p.H, N = p.N, NH = N * H;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4, trow = l16 >> 2, tcol = (l16 & 3) * 4;
    const int R0 = bx * 16;
    const int myrow = R0 + l16;
    const bool row_ok = myrow < NH;
    const int qpos = min(myrow, NH - 1) / H;
    const int pmax = min(R0 + 15, NH - 1) / H, pmin = R0 / H;
    const int kend = CAUSAL ? min(N, pmax + 1) : N;
    const float c2 = p.scale_log2;

    const __amdgpu_buffer_rsrc_t kres = buf_rsrc(p.k + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t vres = buf_rsrc(p.v + (int64_t)b * N * DH, (uint32_t)N * DH * 2u);
    const __amdgpu_buffer_rsrc_t qres = buf_rsrc(p.q + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t gres = buf_rsrc(p.dO + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t ores = buf_rsrc(p.o + (int64_t)b * NH * DH, (uint32_t)NH * DH * 2u);
    const __amdgpu_buffer_rsrc_t lres = buf_rsrc(p.lse + (int64_t)b * H * N, (uint32_t)(H * N) * 4u);
    const float my_lse = buf_load_f32(lres, oob_or(row_ok, (uint32_t)((myrow % H) * N + qpos) * 4u));

    WideTile<DH> lk, lv;
    const int nkt = (kend + WKC - 1) / WKC;
    if (nkt > 0) {  // before the row operands: they do not depend on each other
        lk.load(kres, 0);
        lv.load(vres, 0);
    }
    RowFrag<DH> qf, gf, of;
    qf.load(qres, row_ok, myrow, g);
    gf.load(gres, row_ok, myrow, g);
    of.load(ores, row_ok, myrow, g);
    float my_d = 0.0f;  // D = rowsum(dO * O): this lane's dims, then the row's four lane groups
#pragma unroll
    for (int ks = 0; ks < RowFrag<DH>::K32; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) my_d = __builtin_fmaf((float)of.m[ks][e], (float)gf.m[ks][e], my_d);
    if (RowFrag<DH>::TAIL) {
#pragma unroll
        for (int e = 0; e < 4; ++e) my_d = __builtin_fmaf((float)of.t[e], (float)gf.t[e], my_d);
    }
    my_d += __shfl_xor(my_d, 16, 64);
    my_d += __shfl_xor(my_d, 32, 64);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): see flash_fwd_wide
    const float my_lse2 = my_lse * kLog2e;
    floatx4 dq[DPW];
#pragma unroll
    for (int i = 0; i < DPW; ++i) dq[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (nkt > 0) {
        lk.store(sK[0]);
        lv.store(sV[0]);
    }
    __syncthreads();
    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) {
            lk.load(kres, (kt + 1) * WKC);
            lv.load(vres, (kt + 1) * WKC);
        }
        const int key0 = kt * WKC;
        // wave w: block w of S^T keys 0-15, 16-31, then dP^T keys 0-15, 16-31
        xput(sX, wave, lane, contract_full<DH, W>((wave & 2) ? sV[cur] : sK[cur], 16 * (wave & 1),
                                                  (wave & 2) ? gf : qf, l16, g));
        __syncthreads();
        const floatx4 s[2] = {xget(sX, 0, lane), xget(sX, 1, lane)}, dp[2] = {xget(sX, 2, lane), xget(sX, 3, lane)};
        const bool need_mask = (key0 + WKC > N) || (CAUSAL && key0 + WKC - 1 > pmin) || !row_ok;
        const int lim = (CAUSAL ? min(N - 1, qpos) : N - 1) - key0 - 4 * g;
        floatx4 ds[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = !need_mask || (row_ok && kb * 16 + j <= lim);
                const float pv = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][j], c2, -my_lse2)) : 0.0f;
                ds[kb][j] = pv * (dp[kb][j] - my_d);
            }
        const half8 sb = pack_slots(ds[0], ds[1]);
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const int d = wave + 4 * i;
            if (DB % 4 == 0 || d < DB) dq[i] = mfma16(tile_tr<W>(sK[cur], d * 16, g, trow, tcol), sb, dq[i]);
        }
        if (more) {
            lk.store(sK[cur ^ 1]);
            lv.store(sV[cur ^ 1]);
        }
        __syncthreads();
    }
    if (!row_ok) return;
    f16* qdst = p.out + ((int64_t)b * NH + myrow) * DH;
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const int d = wave + 4 * i;
        if (DB % 4 == 0 || d < DB) {
            const u32x2 w2 = {pack_h2(dq[i][0] * p.scale, dq[i][1] * p.scale), pack_h2(dq[i][2] * p.scale, dq[i][3] * p.scale)};
            *reinterpret_cast<u32x2*>(qdst + d * 16 + g * 4) = w2;
        }
    }
}

template <int DH>
hipError_t launch_fwd_wide(const FlashArgs& a, bool causal, hipStream_t st) {
    dim3 grid((unsigned)((a.N * a.H + 15) / 16), (unsigned)a.B);
    if (causal) hipLaunchKernelGGL((flash_fwd_wide<DH, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((flash_fwd_wide<DH, false>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// dK/dV and dQ in one launch: blocks [0, nkv) of a batch take 16 keys
// each, the rest 16 query rows each; the two roles share nothing, so their
// latency chains overlap on the GPU.
template <int DH, bool CAUSAL>
__global__ __launch_bounds__(256) void flash_bwd_wide(FlashArgs p, int nkv) {
    __shared__ __attribute__((aligned(16))) char lds[bwd_wide_lds<DH>()];
    if ((int)blockIdx.x < nkv) bwd_dkdv_wide<DH, CAUSAL>(p, blockIdx.x, lds);
    else bwd_dq_wide<DH, CAUSAL>(p, blockIdx.x - nkv, lds);
}

template <int DH>
hipError_t launch_bwd_wide(const FlashArgs& a, bool causal, hipStream_t st) {
    const int nkv = (a.N + 15) / 16, nq = (a.N * a.H + 15) / 16;
    dim3 grid((unsigned)(nkv + nq), (unsigned)a.B);
    if (causal) hipLaunchKernelGGL((flash_bwd_wide<DH, true>), grid, dim3(256), 0, st, a, nkv);
    else hipLaunchKernelGGL((flash_bwd_wide<DH, false>), grid, dim3(256), 0, st, a, nkv);
    return hipGetLastError();
}

// Head sizes with wide kernels (multiples of 16 up to 256 not covered by
// the specialised kernels): calls f.template operator()<DH>().
template <class F>
hipError_t wide_dispatch(int dh, F&& f) {
    switch (dh) {
        case 16: return f(std::integral_constant<int, 16>{});
        case 48: return f(std::integral_constant<int, 48>{});
        case 80: return f(std::integral_constant<int, 80>{});
        case 96: return f(std::integral_constant<int, 96>{});
        case 112: return f(std::integral_constant<int, 112>{});
        case 144: return f(std::integral_constant<int, 144>{});
        case 160: return f(std::integral_constant<int, 160>{});
        case 176: return f(std::integral_constant<int, 176>{});
        case 192: return f(std::integral_constant<int, 192>{});
        case 208: return f(std::integral_constant<int, 208>{});
        case 224: return f(std::integral_constant<int, 224>{});
        case 240: return f(std::integral_constant<int, 240>{});
        case 256: return f(std::integral_constant<int, 256>{});
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool flash_wide_head(uint32_t dh) {
    return dh % 16 == 0 && dh >= 16 && dh <= 256 && dh != 32 && dh != 64 && dh != 128;
}

hipError_t flash_forward_wide(const FlashArgs& a, int dh, bool causal, hipStream_t st) {
    return wide_dispatch(dh, [&](auto D) { return launch_fwd_wide<decltype(D)::value>(a, causal, st); });
}

hipError_t flash_backward_wide(const FlashArgs& a, int dh, bool causal, hipStream_t st) {
    return wide_dispatch(dh, [&](auto D) { return launch_bwd_wide<decltype(D)::value>(a, causal, st); });
}

}  // namespace evkhip
