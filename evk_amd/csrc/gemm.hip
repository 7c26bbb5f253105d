// fp16 GEMM / GEMV for gfx950: the kernels behind evk::ai::matmul
// (reference: evk_ai.cpp:254-330 host side, shaders/matmul.comp:44-141).
//
// Tiled kernel: a workgroup computes a BM x BN tile of C with 4 waves; each
// wave owns a (BM/WGM) x (BN/WGN) sub-tile made of 32x32 MFMA accumulators
// (v_mfma_f32_32x32x16_f16, fp32 accumulation).  A and B tiles of BK along
// K are staged in LDS, double-buffered, always stored k-contiguous
// ([row][k], 16-byte chunks XOR-swizzled by row).  Operands that arrive
// k-contiguous in memory (A row-major, B stored (N,K)) are copied as 16-byte
// chunks; operands that arrive m/n-contiguous (A stored (K,M), B row-major
// (K,N)) are transposed in registers in 8x8 blocks on the way to LDS.  The
// global loads of tile t+1 are issued before the MFMAs of tile t.
//
// Skinny kernel (M <= 16, B row-major): bandwidth-bound, streams B once with
// 16-byte coalesced loads, fp32 accumulation in registers, split-K across
// workgroups with a deterministic last-arriving-workgroup reduction.
#include "kernels.h"

#include <algorithm>
#include <utility>

namespace evkhip {

namespace {

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
    static constexpr int NT = WGM * WGN * 64;
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int TM = WM / 32, TN = WN / 32;
    static constexpr int KC = BK / 8;  // 16-byte chunks per LDS row
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 MFMA tile");
    static_assert(BK % 16 == 0 && KC <= 8, "BK must be 16..64");
};

// Element offset (in halves) of chunk `c` of LDS row `r` (rows of BK halves).
template <int BK>
DEV int lds_off(int r, int c) {
    constexpr int KC = BK / 8;
    return r * BK + ((c ^ (r & (KC - 1))) << 3);
}

// ---- k-contiguous operand: ROWS x BK tile, chunk copies --------------------
template <int ROWS, int BK, int NT>
struct DirectLoader {
    static constexpr int KC = BK / 8;
    static constexpr int CHUNKS = ROWS * KC;
    static constexpr int PER = (CHUNKS + NT - 1) / NT;
    u32x4 r[PER];

    DEV void load(const f16* __restrict__ src, int64_t ld, int row0, int nrows, int k0, int K) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int c = threadIdx.x + i * NT;
            int row = c / KC, kc = c % KC;
            int gr = row0 + row, gk = k0 + kc * 8;
            u32x4 v = {0u, 0u, 0u, 0u};
            if ((CHUNKS % NT == 0 || c < CHUNKS) && gr < nrows && gk < K)
                v = *reinterpret_cast<const u32x4*>(src + (int64_t)gr * ld + gk);
            r[i] = v;
        }
    }
    DEV void store(f16* lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int c = threadIdx.x + i * NT;
            if (CHUNKS % NT == 0 || c < CHUNKS) {
                int row = c / KC, kc = c % KC;
                *reinterpret_cast<u32x4*>(lds + lds_off<BK>(row, kc)) = r[i];
            }
        }
    }
};

// ---- m/n-contiguous operand: memory holds BK rows of ROWS contiguous halves;
// LDS wants ROWS rows of BK.  8x8 register transposes. ------------------------
template <int ROWS, int BK, int NT>
struct TransLoader {
    static constexpr int NB = ROWS / 8, KB = BK / 8;
    static constexpr int BLOCKS = NB * KB;
    static constexpr int PER = (BLOCKS + NT - 1) / NT;
    u32x4 r[PER][8];

    DEV void load(const f16* __restrict__ src, int64_t ld, int row0, int nrows, int k0, int K) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + i * NT;
            int kb = q / NB, nb = q % NB;
            int gn = row0 + nb * 8;
            bool okb = (BLOCKS % NT == 0 || q < BLOCKS) && gn < nrows;
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                int gk = k0 + kb * 8 + rr;
                u32x4 v = {0u, 0u, 0u, 0u};
                if (okb && gk < K) v = *reinterpret_cast<const u32x4*>(src + (int64_t)gk * ld + gn);
                r[i][rr] = v;
            }
        }
    }
    DEV void store(f16* lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + i * NT;
            if (BLOCKS % NT == 0 || q < BLOCKS) {
                int kb = q / NB, nb = q % NB;
                u32x4 t[8];
                transpose8x8(r[i], t);
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    *reinterpret_cast<u32x4*>(lds + lds_off<BK>(nb * 8 + c, kb)) = t[c];
            }
        }
    }
};

template <bool TRANS, int ROWS, int BK, int NT>
using LoaderFor = typename std::conditional<TRANS, TransLoader<ROWS, BK, NT>, DirectLoader<ROWS, BK, NT>>::type;

// TA: A stored (K,M).  TB: B stored (N,K).
template <class Cfg, bool TA, bool TB>
__global__ __launch_bounds__(Cfg::NT) void gemm_tiled(GemmArgs p) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NT = Cfg::NT;
    constexpr int TM = Cfg::TM, TN = Cfg::TN;
    __shared__ __attribute__((aligned(16))) f16 sA[2][BM * BK];
    __shared__ __attribute__((aligned(16))) f16 sB[2][BN * BK];

    const int M = p.M, N = p.N, K = p.K;
    const int bz = blockIdx.z;
    const f16* __restrict__ A = p.A + (int64_t)bz * p.sA;
    const f16* __restrict__ B = p.B + (int64_t)bz * p.sB;
    f16* __restrict__ Cp = p.C + (int64_t)bz * p.sC;

    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm0 = (wave / Cfg::WGN) * Cfg::WM, wn0 = (wave % Cfg::WGN) * Cfg::WN;
    const int l32 = lane & 31, lg = lane >> 5;

    // A: logical (M,K).  !TA: row-major ld=K, rows m.  TA: memory (K,M), ld=M.
    LoaderFor<TA, BM, BK, NT> la;
    LoaderFor<!TB, BN, BK, NT> lb;
    const int64_t ldA = TA ? M : K;
    const int64_t ldB = TB ? K : N;

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int KT = (K + BK - 1) / BK;
    la.load(A, ldA, m0, M, 0, K);
    lb.load(B, ldB, n0, N, 0, K);
    la.store(sA[0]);
    lb.store(sB[0]);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            la.load(A, ldA, m0, M, (kt + 1) * BK, K);
            lb.load(B, ldB, n0, N, (kt + 1) * BK, K);
        }
        const f16* a_s = sA[cur];
        const f16* b_s = sB[cur];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            half8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const half8*>(a_s + lds_off<BK>(wm0 + i * 32 + l32, ks * 2 + lg));
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const half8*>(b_s + lds_off<BK>(wn0 + j * 32 + l32, ks * 2 + lg));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(af[i], bf[j], acc[i][j]);
        }
        if (more) {
            la.store(sA[cur ^ 1]);
            lb.store(sB[cur ^ 1]);
        }
        __syncthreads();
    }

    // Epilogue: D element e of lane l -> row 8*(e/4)+4*lg+(e%4), col l32.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn0 + j * 32 + l32;
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm0 + i * 32 + 8 * (e >> 2) + 4 * lg + (e & 3);
                if (row < M) {
                    f16* dst = Cp + (int64_t)row * N + col;
                    float v = acc[i][j][e];
                    if (p.acc) v += (float)*dst;
                    *dst = (f16)v;
                }
            }
        }
}

// ---- MFMA kernel: BM x BN tiles; 4 waves of (BM/2) x (BN/2), or for 256x256
// tiles 8 waves of 128 x 64 (two waves per SIMD: one wave's LDS reads and
// waits overlap the other's MFMAs; measured 2-5 % faster than 4 waves of
// 128 x 128 at 4096^3 and QKV, while 4 waves of 64 x 128 were slower).
// 64x64 tiles of a grid that fits the CUs once with a long K run go as four
// K groups of 4 waves (16 waves), whose fp32 sums are added in group order
// in LDS, so the result does not depend on timing: 1024^3 8.6 -> 7.1 us ----
// v_mfma_f32_16x16x32_f16 (lane l: A row l%16 / B column l%16, k 8(l/16)..+8;
// D column l%16, rows 4(l/16)..+3).  Each operand tile of BK = 64 along K
// goes from global memory straight into LDS (buffer_load_dwordx4 ... lds: a
// wave instruction fills 1 KB, lane i the 16 bytes at i*16) as it lies in
// memory, with the 16-byte chunks of a row permuted so that the fragment
// reads hit distinct banks:
//   k-contiguous operand (A row-major, B stored (N,K)): rows of 64 halves,
//     chunk c of row r at slot c ^ (r & 7); fragments by ds_read_b128.
//   m/n-contiguous operand (A stored (K,M), B row-major): rows of BM / BN
//     halves, chunk c of row r at slot c ^ 2 (r & 3); fragments by
//     ds_read_b64_tr_b16 (4 consecutive k of one column per lane).
// The loads choose their global chunk per lane to realise the permutation;
// chunks outside the matrix read as zeros (buffer descriptors).  Two LDS
// stages for 256x256 tiles, four for smaller ones: the loads of the next
// tiles fly during the MFMAs of tile t; one barrier per tile.  Workgroups are ordered so that the
// ones an XCD runs (workgroup id mod 8) cover a compact block of C tiles and
// share A/B panels in that XCD's L2.  The epilogue stages each wave's fp16
// tile in LDS and writes 16-byte row chunks (accumulating calls add C per
// element instead, with one rounding of the fp32 sum).
constexpr int MB_K = 64;  // BK

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from a buffer straight into LDS: lane i writes
// lds_base + 16 i (lds_base: wave-uniform LDS byte address).  Written as
// inline assembly so that the compiler does not make every later LDS read
// wait for these loads (it cannot tell the two stages apart); the kernel
// waits for them itself (vmcnt) before the barrier that publishes a stage.
// M0 carries the LDS address; nothing else in the kernels that use this
// keeps a value in M0.
DEV void dma16(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(res), "s"(lds_base)
                 : "memory");
}
DEV uint32_t lds_addr(const f16* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void*)p);
}

// One operand tile (ROWS x COLS halves as stored in memory; the matrix is
// nr x nc with leading dimension ld, the tile starts at (r0, c0)) into LDS.
template <int ROWS, int COLS, bool KCONTIG, int NWV = 4>
DEV void tile_to_lds(__amdgpu_buffer_rsrc_t res, int64_t ld, int r0, int c0, int nr, int nc, f16* lds, int wave,
                     int lane) {
    constexpr int CPR = COLS / 8;     // chunks per row
    constexpr int RPI = 64 / CPR;     // rows per wave instruction
    constexpr int PER = ROWS / RPI / NWV;
    static_assert(PER >= 1 && CPR >= 8, "tile shape");
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int q = wave * PER + t;
        const int row = q * RPI + lane / CPR, slot = lane % CPR;
        const int ch = KCONTIG ? (slot ^ (row & 7)) : (slot ^ (2 * (row & 3)));
        const bool ok = r0 + row < nr && c0 + ch * 8 < nc;
        const uint32_t off = oob_or(ok, (uint32_t)(((int64_t)(r0 + row) * ld + c0 + ch * 8) * 2));
        dma16(res, off, lds_addr(lds + q * 512));
    }
}

// fragment of a k-contiguous tile: row r, k chunk kc (8 halves)
DEV half8 frag_k(const f16* t, int r, int kc) {
    return *reinterpret_cast<const half8*>(t + r * MB_K + ((kc ^ (r & 7)) << 3));
}
// fragment of an m/n-contiguous tile (rows of W halves): column block c0
// (multiple of 16), k rows k0 + 8 g .. +8, through two transposed reads
template <int W>
DEV half8 frag_t(const f16* t, int k0, int c0, int g, int trow, int tcol) {
    auto at = [&](int k) {
        const int c = c0 + tcol;
        return t + k * W + ((((c >> 3) ^ (2 * (k & 3))) << 3) | (c & 7));
    };
    const int k = k0 + 8 * g + trow;
    return cat4(lds_read_tr(at(k)), lds_read_tr(at(k + 4)));
}

DEV int xcd_tile(int w, int total) {
    if (total % 8) return w;
    return (w % 8) * (total / 8) + w / 8;  // XCD w%8 gets a contiguous range
}

// LDS stages of gemm_mfma: two for 256x256 tiles (128 KB), four for the
// smaller tiles, whose short K loops need more tiles in flight.
template <int BM>
constexpr int mfma_stages() { return BM >= 256 ? 2 : 4; }

// s_waitcnt with vmcnt(n) (n < 64) and the other counters left alone
DEV void wait_vmcnt(int n) {
    switch (n) {
#define EVK_VMCNT_CASE(v) \
    case v: __builtin_amdgcn_s_waitcnt(((v) & 15) | (((v) >> 4) << 14) | 0x0f70); break;
        EVK_VMCNT_CASE(0) EVK_VMCNT_CASE(4) EVK_VMCNT_CASE(8) EVK_VMCNT_CASE(12) EVK_VMCNT_CASE(16)
        EVK_VMCNT_CASE(24) EVK_VMCNT_CASE(32)
#undef EVK_VMCNT_CASE
        default: __builtin_amdgcn_s_waitcnt(0x0f70); break;
    }
}

template <int BM, int BN, bool TA, bool TB, int NWV = 4, int KG = 1>
__global__ __launch_bounds__(64 * NWV * KG, 1) void gemm_mfma(GemmArgs p, int tiles_m, int tiles_n) {
    constexpr int WGN = NWV / 2;  // waves along N (2 along M)
    constexpr int BK = MB_K, WM = BM / 2, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
    constexpr int A_EL = BM * BK, B_EL = BN * BK, STAGE = A_EL + B_EL;
    constexpr int NST = KG > 1 ? 2 : mfma_stages<BM>();  // per K group
    constexpr int LPT = (BM * BK / 512 + BN * BK / 512) / NWV;  // DMA loads per wave per tile
    constexpr int OUT_LD = WN + 8;
    constexpr int OUT_EL = NWV * WM * OUT_LD;
    constexpr int LDS_EL = OUT_EL > KG * NST * STAGE ? OUT_EL : KG * NST * STAGE;
    static_assert(KG == 1 || (KG - 1) * NWV * FM * FN * 64 * 8 <= KG * NST * STAGE,
                  "K-group partials fit in the stages");
    __shared__ __attribute__((aligned(1024))) f16 smem[LDS_EL];

    const int M = p.M, N = p.N, K = p.K;
    const int bz = blockIdx.z;
    const f16* A = p.A + (int64_t)bz * p.sA;
    const f16* B = p.B + (int64_t)bz * p.sB;
    f16* Cp = p.C + (int64_t)bz * p.sC;

    // tile order: XCD-contiguous ranges, then groups of 4 tile rows
    const int total = tiles_m * tiles_n;
    const int t = xcd_tile(blockIdx.x, total);
    constexpr int GM = 4;
    const int grp = t / (GM * tiles_n), first = grp * GM, gsz = min(GM, tiles_m - first);
    const int tm = first + (t % (GM * tiles_n)) % gsz, tn = (t % (GM * tiles_n)) / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63;
    // KG > 1: KG groups of NWV waves; group kg takes the kg-th range of the
    // K tiles in its own LDS stages, and the groups' fp32 sums meet in LDS
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kg = wave_all / NWV, wave = wave_all % NWV;
    const int l16 = lane & 15, g = lane >> 4;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int trow = l16 >> 2, tcol = (l16 & 3) * 4;

    const __amdgpu_buffer_rsrc_t ares = buf_rsrc(A, (uint32_t)((int64_t)M * K * 2));
    const __amdgpu_buffer_rsrc_t bres = buf_rsrc(B, (uint32_t)((int64_t)K * N * 2));
    auto issue = [&](int k0, f16* sa, f16* sb) {
        if (TA) tile_to_lds<BK, BM, false, NWV>(ares, M, k0, m0, K, M, sa, wave, lane);
        else tile_to_lds<BM, BK, true, NWV>(ares, K, m0, k0, M, K, sa, wave, lane);
        if (TB) tile_to_lds<BN, BK, true, NWV>(bres, K, n0, k0, N, K, sb, wave, lane);
        else tile_to_lds<BK, BN, false, NWV>(bres, N, k0, n0, K, N, sb, wave, lane);
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // One LDS tile: 2 k-steps x FM fragment rows, FN MFMAs per row, run as
    // 2 FM steps.  A fragments are read AD steps ahead (ring of AD + 1); the
    // B fragments of the second k-step are read during the first, one or
    // more per step; the scheduling groups pin that order so that the LDS
    // latency hides behind the MFMAs of earlier steps.
    constexpr int NA = TA ? 2 : 1, NB = TB ? 1 : 2;  // LDS reads per fragment
    constexpr int AD = FM >= 4 ? 3 : FM - 1;         // A prefetch distance
    constexpr int NS = 2 * FM;                       // steps per tile
    constexpr int BPS = (FN + FM - 1) / FM;          // next-B fragments per step
    auto ldA = [&](const f16* As, int ks, int i) {
        return TA ? frag_t<BM>(As, ks * 32, wm0 + 16 * i, g, trow, tcol) : frag_k(As, wm0 + 16 * i + l16, ks * 4 + g);
    };
    auto ldB = [&](const f16* Bs, int ks, int j) {
        return TB ? frag_k(Bs, wn0 + 16 * j + l16, ks * 4 + g) : frag_t<BN>(Bs, ks * 32, wn0 + 16 * j, g, trow, tcol);
    };
    auto compute = [&](const f16* As, const f16* Bs) {
        half8 bf[2][FN], af[AD + 1];
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[0][j] = ldB(Bs, 0, j);
#pragma unroll
        for (int s2 = 0; s2 < AD; ++s2) af[s2] = ldA(As, s2 / FM, s2 % FM);
        __builtin_amdgcn_sched_group_barrier(0x100, FN * NB + AD * NA, 0);
        static_for<NS>([&](auto stc) {
            constexpr int st = decltype(stc)::value, ks = st / FM, i = st % FM;
            constexpr bool pre_a = st + AD < NS;
            constexpr int nb = (ks == 0 && i * BPS < FN) ? (FN - i * BPS >= BPS ? BPS : FN - i * BPS) : 0;
            if constexpr (pre_a) af[(st + AD) % (AD + 1)] = ldA(As, (st + AD) / FM, (st + AD) % FM);
#pragma unroll
            for (int b2 = 0; b2 < nb; ++b2) bf[1][i * BPS + b2] = ldB(Bs, 1, i * BPS + b2);
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[st % (AD + 1)], bf[ks][j], acc[i][j]);
            // this step's LDS reads, then its MFMAs
            constexpr int nr = (pre_a ? NA : 0) + nb * NB;
            if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);
        });
    };

    // tile kt of the group's range lives in stage kt % NST; NST-1 tiles are
    // in flight.  Every group runs the same number of barrier steps.
    const int KT_ALL = (K + BK - 1) / BK, per = (KT_ALL + KG - 1) / KG;
    const int kt_base = kg * per, KT = max(0, min(KT_ALL - kt_base, per));
    f16* gsm = smem + kg * NST * STAGE;
#pragma unroll
    for (int t2 = 0; t2 < NST - 1; ++t2)
        if (t2 < KT) issue((kt_base + t2) * BK, gsm + t2 * STAGE, gsm + t2 * STAGE + A_EL);
    for (int kt = 0; kt < per; ++kt) {
        // this wave's loads of tile kt are in LDS once at most the loads of
        // the younger tiles in flight remain (loads complete in order)
        wait_vmcnt(LPT * max(0, min(NST - 2, KT - 1 - kt)));
        __syncthreads();  // everyone's; the stage of tile kt-1 is free again
        if (kt + NST - 1 < KT) {
            f16* nxt = gsm + ((kt + NST - 1) % NST) * STAGE;
            issue((kt_base + kt + NST - 1) * BK, nxt, nxt + A_EL);
        }
        if (kt >= KT) continue;
        const f16* cur = gsm + (kt % NST) * STAGE;
        compute(cur, cur + A_EL);
    }

    if constexpr (KG > 1) {
        // groups 1.. store their sums lane-major; group 0 adds them in group order
        __syncthreads();  // every group is done with its stages
        floatx4* red = reinterpret_cast<floatx4*>(smem);
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) red[((((kg - 1) * NWV + wave) * FM + i) * FN + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (kg == 0) {
            for (int q = 1; q < KG; ++q)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] += red[((((q - 1) * NWV + wave) * FM + i) * FN + j) * 64 + lane];
        }
    }
    if (p.acc) {  // C += A B: one rounding of the fp32 sum per element
        if (kg > 0) return;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = n0 + wn0 + 16 * j + l16;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = m0 + wm0 + 16 * i + 4 * g + e;
                    if (row < M && col < N) {
                        f16* dst = Cp + (int64_t)row * N + col;
                        *dst = (f16)(acc[i][j][e] + (float)*dst);
                    }
                }
            }
        return;
    }
    // stage the wave's tile as fp16 rows, then 16-byte row chunks to C; the
    // staging area overlaps the stages, which every wave has finished
    // reading once all have passed this barrier
    __syncthreads();
    if (kg > 0) return;  // past the last barrier: group 0 stores the tile
    f16* ot = smem + wave * WM * OUT_LD;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) ot[(16 * i + 4 * g + e) * OUT_LD + 16 * j + l16] = (f16)acc[i][j][e];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes
    __builtin_amdgcn_wave_barrier();
    constexpr int CPR = WN / 8;
#pragma unroll 4
    for (int q = lane; q < WM * CPR; q += 64) {
        const int r = q / CPR, cc = (q % CPR) * 8;
        const int row = m0 + wm0 + r, col = n0 + wn0 + cc;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ot + r * OUT_LD + cc);
        // nontemporal: C is written once (QKV shape 0.785 -> 0.763 ms)
        if (row < M && col < N) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(Cp + (int64_t)row * N + col));
    }
}

// ---- any-alignment fallback: one thread per C element, fp32 FMA ------------
__global__ __launch_bounds__(256) void gemm_scalar(GemmArgs p, int ta, int tb) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int bz = blockIdx.y;
    if (idx >= (int64_t)p.M * p.N) return;
    const int r = (int)(idx / p.N), c = (int)(idx % p.N);
    const f16* A = p.A + (int64_t)bz * p.sA;
    const f16* B = p.B + (int64_t)bz * p.sB;
    f16* Cp = p.C + (int64_t)bz * p.sC;
    float s = 0.0f;
    for (int k = 0; k < p.K; ++k) {
        float a = (float)(ta ? A[(int64_t)k * p.M + r] : A[(int64_t)r * p.K + k]);
        float b = (float)(tb ? B[(int64_t)c * p.K + k] : B[(int64_t)k * p.N + c]);
        s += a * b;
    }
    f16* dst = Cp + (int64_t)r * p.N + c;
    if (p.acc) s += (float)*dst;
    *dst = (f16)s;
}

// ---- skinny GEMV: C(M,N) = A(M,K) B(K,N), M <= 16, B row-major -------------
// Bandwidth-bound on B, which is read exactly once.  Workgroup (cb, ks) owns
// 64 columns (one 128-byte line of each B row) and the K range
// [ks*SK_KC, +SK_KC): its 256 threads are 8 column groups of 8 columns x 32
// row groups, and each thread requests all SK_LD of its 16-byte B loads
// before it waits, so the whole 64 KB slice is in flight at once.  A's slice
// is staged in LDS as floats [k][MR]; the A loads go out first and the B
// loads right after them (the prologue then waits for A only: loads complete
// in issue order).  The 32 row groups are summed through LDS; with one K
// range the workgroup writes C, otherwise fp32 partials that the column
// block's last-arriving workgroup adds in range order (deterministic).
constexpr int SK_CB = 64;                 // columns per workgroup
constexpr int SK_RG = 32;                 // row groups
constexpr int SK_LD = 16;                 // B loads per thread
constexpr int SK_KC = SK_RG * SK_LD;      // rows per K range (512)

// The K ranges of a column block meet in the workgroup that arrives last
// (agent-scope partial stores and counter, no fences); it adds the partials
// in range order, so the result does not depend on arrival order.
DEV void gemv_finish(const GemmArgs& p, float* part, unsigned* cnt, int c0) {
    const int M = p.M, N = p.N, bz = blockIdx.z, nks = gridDim.y;
    if (!arrive_last(cnt + bz * gridDim.x + blockIdx.x, nks)) return;
    f16* Cp = p.C + (int64_t)bz * p.sC;
    for (int idx = threadIdx.x; idx < M * SK_CB; idx += 256) {
        const int m = idx / SK_CB, gc = c0 + idx % SK_CB;
        if (gc >= N) continue;
        const float* src = part + ((int64_t)bz * nks * M + m) * N + gc;
        const int64_t stride = (int64_t)M * N;
        float v = 0.0f;
        for (int s0 = 0; s0 < nks; s0 += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = (s0 + u < nks) ? ld_ag(src + (s0 + u) * stride) : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        f16* dst = Cp + (int64_t)m * N + gc;
        *dst = (f16)(p.acc ? v + (float)*dst : v);
    }
}

// The same finish for up to 16 rows (the MFMA kernel), with 16-byte loads:
// thread t adds row t / 16, columns 4 (t % 16) .. +3 of the column block,
// every range's partial requested before any is added, in range order as
// in gemv_finish.  The loads carry the sc1 policy of ld_ag (served from the
// device coherence point).
DEV void gemv_finish_m16(const GemmArgs& p, float* part, unsigned* cnt, int c0) {
    const int M = p.M, N = p.N, bz = blockIdx.z, nks = gridDim.y;
    if (!arrive_last(cnt + bz * gridDim.x + blockIdx.x, nks)) return;
    static_assert(16 * SK_CB / 4 == 256, "one row quad per thread");
    const int m = threadIdx.x / (SK_CB / 4), gc = c0 + (threadIdx.x % (SK_CB / 4)) * 4;
    const bool ok = m < M && gc < N;  // N % 8 == 0: the quad is whole
    const __amdgpu_buffer_rsrc_t pres =
        buf_rsrc(part + (int64_t)bz * nks * M * N, (uint32_t)((int64_t)nks * M * N * 4));
    const uint32_t off0 = (uint32_t)(((int64_t)m * N + gc) * 4), step = (uint32_t)((int64_t)M * N * 4);
    constexpr int PB = 8;  // ranges per batch of loads
    floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < nks; s0 += PB) {
        u32x4 t[PB];
#pragma unroll
        for (int s = 0; s < PB; ++s)
            t[s] = __builtin_amdgcn_raw_buffer_load_b128(pres, oob_or(ok && s0 + s < nks, off0 + (s0 + s) * step), 0,
                                                         16 /* sc1 */);
#pragma unroll
        for (int s = 0; s < PB; ++s) v += __builtin_bit_cast(floatx4, t[s]);
    }
    if (ok) {
        f16* dst = p.C + (int64_t)bz * p.sC + (int64_t)m * N + gc;
        if (p.acc) {
            const uint2 o = *reinterpret_cast<const uint2*>(dst);
            const half2_t h0 = __builtin_bit_cast(half2_t, o.x), h1 = __builtin_bit_cast(half2_t, o.y);
            v[0] += (float)h0[0];
            v[1] += (float)h0[1];
            v[2] += (float)h1[0];
            v[3] += (float)h1[1];
        }
        *reinterpret_cast<uint2*>(dst) = uint2{pack_h2(v[0], v[1]), pack_h2(v[2], v[3])};
    }
}

template <int MR>
__global__ __launch_bounds__(256) void gemv_sk(GemmArgs p, float* __restrict__ part, unsigned* cnt) {
    // A's slice in LDS as fp16 pairs: pair P = rg + 32 v (v < SK_LD / 2) holds
    // k = rg + 64 v and k + 32 of the K range for each row m, the two B rows
    // that thread row group rg loads as its loads 2v and 2v+1
    __shared__ __attribute__((aligned(16))) uint32_t hv[(SK_KC / 2) * MR];
    __shared__ float red[SK_RG * 4 * SK_CB];
    const int M = p.M, N = p.N, K = p.K;
    const int bz = blockIdx.z, ks = blockIdx.y, nks = gridDim.y;
    const f16* A = p.A + (int64_t)bz * p.sA;
    const f16* B = p.B + (int64_t)bz * p.sB;
    f16* Cp = p.C + (int64_t)bz * p.sC;
    const int c0 = blockIdx.x * SK_CB, r_lo = ks * SK_KC, r_hi = min(K, r_lo + SK_KC);
    const int cg = threadIdx.x & 7, rg = threadIdx.x >> 3;
    const int col = c0 + cg * 8;
    const bool col_ok = col < N;

    // A slice: MR rows x SK_KC k as 16-byte chunks along k (chunks past K or
    // M read as zeros)
    constexpr int ACH = MR * SK_KC / 8, APER = (ACH + 255) / 256;
    const __amdgpu_buffer_rsrc_t ares = buf_rsrc(A, (uint32_t)((int64_t)M * K * 2));
    u32x4 av[APER];
#pragma unroll
    for (int u = 0; u < APER; ++u) {
        const int c = threadIdx.x + 256 * u, m = c / (SK_KC / 8), kk = (c % (SK_KC / 8)) * 8;
        const bool ok = c < ACH && m < M && r_lo + kk < r_hi;
        av[u] = buf_load16(ares, oob_or(ok, (uint32_t)(((int64_t)m * K + r_lo + kk) * 2)), 0);
    }
    asm volatile("" ::: "memory");
    const __amdgpu_buffer_rsrc_t bres = buf_rsrc(B, (uint32_t)((int64_t)K * N * 2));
    u32x4 w[SK_LD];
#pragma unroll
    for (int u = 0; u < SK_LD; ++u) {
        const int i = r_lo + rg + u * SK_RG;
        // nontemporal: B is read once (the MFMA kernel below measured slower with it)
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(bres, oob_or(col_ok && i < r_hi, (uint32_t)(((int64_t)i * N + col) * 2)), 0, 2);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < APER; ++u) asm volatile("" : "+v"(av[u]));
    // A into LDS pairs (K-tail chunks were zero-filled by the loads): the 8
    // k of a chunk share v and h and have consecutive rg
    f16* hvh = reinterpret_cast<f16*>(hv);
#pragma unroll
    for (int u = 0; u < APER; ++u) {
        const int c = threadIdx.x + 256 * u, m = c / (SK_KC / 8), kk = (c % (SK_KC / 8)) * 8;
        if (c < ACH) {
            const half8 h = as_half8(av[u]);
            const int hh = (kk >> 5) & 1, P0 = (kk & 31) + 32 * (kk >> 6);
#pragma unroll
            for (int e = 0; e < 8; ++e) hvh[((P0 + e) * MR + m) * 2 + hh] = h[e];
        }
    }
    __syncthreads();

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;
    // two B rows at a time: the column pairs (row k, row k + 32) go through
    // v_dot2_f32_f16 against A's pair (fp32 accumulation, no conversions)
#pragma unroll
    for (int v = 0; v < SK_LD / 2; ++v) {
        const uint32_t* hr = hv + (rg + 32 * v) * MR;  // zeros past K
        uint32_t a2[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) a2[m] = hr[m];
        const u32x4 w0 = w[2 * v], w1 = w[2 * v + 1];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t blo = __builtin_amdgcn_perm(w1[d], w0[d], 0x05040100u);  // column 2d
            const uint32_t bhi = __builtin_amdgcn_perm(w1[d], w0[d], 0x07060302u);  // column 2d + 1
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                acc[m][2 * d] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a2[m]),
                                                       __builtin_bit_cast(half2_t, blo), acc[m][2 * d], false);
                acc[m][2 * d + 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a2[m]),
                                                           __builtin_bit_cast(half2_t, bhi), acc[m][2 * d + 1], false);
            }
        }
    }

    // sum the row groups, 4 rows of A at a time
#pragma unroll
    for (int m0 = 0; m0 < MR; m0 += 4) {
#pragma unroll
        for (int mm = 0; mm < 4; ++mm)
            if (m0 + mm < MR)
#pragma unroll
                for (int e = 0; e < 8; ++e) red[(rg * 4 + mm) * SK_CB + cg * 8 + e] = acc[m0 + mm][e];
        __syncthreads();
        {
            const int mm = threadIdx.x / SK_CB, cc = threadIdx.x % SK_CB;
            const int m = m0 + mm, gc = c0 + cc;
            float v = 0.0f;
            for (int r = 0; r < SK_RG; ++r) v += red[(r * 4 + mm) * SK_CB + cc];
            if (m < M && m < MR && gc < N) {
                if (nks == 1) {
                    f16* dst = Cp + (int64_t)m * N + gc;
                    *dst = (f16)(p.acc ? v + (float)*dst : v);
                } else {
                    st_ag(part + (((int64_t)bz * nks + ks) * M + m) * N + gc, v);
                }
            }
        }
        __syncthreads();
    }
    if (nks > 1) gemv_finish(p, part, cnt, c0);
}

// Skinny GEMV on the MFMA (4 < M <= 16): the same workgroup slice and
// loads as gemv_sk, but the arithmetic is v_mfma_f32_16x16x32_f16 with A's
// 16 (zero-padded) rows as the A operand.  The B slice goes through LDS in
// two halves of 256 rows (rows of 64 halves, 16-byte chunk c of row r at
// slot c ^ 2 (r & 3)) and comes back as B operands via ds_read_b64_tr_b16;
// wave w owns columns c0 + 16 w .. +16 for the whole K range, so no
// cross-wave sum is needed.
constexpr int SKM_ALD = SK_KC + 8;  // A row stride in LDS (halves)

__global__ __launch_bounds__(256) void gemv_mf(GemmArgs p, float* __restrict__ part, unsigned* cnt) {
    __shared__ __attribute__((aligned(16))) f16 as_[16 * SKM_ALD];
    __shared__ __attribute__((aligned(16))) f16 bs[(SK_KC / 2) * SK_CB];
    const int M = p.M, N = p.N, K = p.K;
    const int bz = blockIdx.z, ks = blockIdx.y, nks = gridDim.y;
    const f16* A = p.A + (int64_t)bz * p.sA;
    const f16* B = p.B + (int64_t)bz * p.sB;
    f16* Cp = p.C + (int64_t)bz * p.sC;
    const int c0 = blockIdx.x * SK_CB, r_lo = ks * SK_KC, r_hi = min(K, r_lo + SK_KC);
    const int cg = threadIdx.x & 7, rg = threadIdx.x >> 3;
    const int col = c0 + cg * 8;
    const bool col_ok = col < N;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4, trow = l16 >> 2, tcol = (l16 & 3) * 4;

    // A slice: 16 rows (rows >= M read as zeros) x SK_KC k, 16-byte chunks
    constexpr int ACH = 16 * SK_KC / 8, APER = ACH / 256;
    const __amdgpu_buffer_rsrc_t ares = buf_rsrc(A, (uint32_t)((int64_t)M * K * 2));
    u32x4 av[APER];
#pragma unroll
    for (int u = 0; u < APER; ++u) {
        const int c = threadIdx.x + 256 * u, m = c / (SK_KC / 8), kk = (c % (SK_KC / 8)) * 8;
        const bool ok = m < M && r_lo + kk < r_hi;
        av[u] = buf_load16(ares, oob_or(ok, (uint32_t)(((int64_t)m * K + r_lo + kk) * 2)), 0);
    }
    asm volatile("" ::: "memory");
    const __amdgpu_buffer_rsrc_t bres = buf_rsrc(B, (uint32_t)((int64_t)K * N * 2));
    u32x4 w[SK_LD];
#pragma unroll
    for (int u = 0; u < SK_LD; ++u) {
        const int i = r_lo + rg + u * SK_RG;
        w[u] = buf_load16(bres, oob_or(col_ok && i < r_hi, (uint32_t)(((int64_t)i * N + col) * 2)), 0);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < APER; ++u) {
        asm volatile("" : "+v"(av[u]));
        const int c = threadIdx.x + 256 * u, m = c / (SK_KC / 8), kk = (c % (SK_KC / 8)) * 8;
        *reinterpret_cast<u32x4*>(as_ + m * SKM_ALD + kk) = av[u];
    }

    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    constexpr int HALF = SK_LD / 2;  // loads per thread per half (256 rows)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // B rows h*256 .. +256 of the slice into LDS
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            const int r = rg + u * SK_RG;
            *reinterpret_cast<u32x4*>(bs + r * SK_CB + ((cg ^ (2 * (r & 3))) << 3)) = w[h * HALF + u];
        }
        __syncthreads();
#pragma unroll
        for (int kq = 0; kq < SK_KC / 2 / 32; ++kq) {
            const half8 af = *reinterpret_cast<const half8*>(as_ + l16 * SKM_ALD + h * (SK_KC / 2) + kq * 32 + 8 * g);
            auto at = [&](int k) {
                const int c = wave * 16 + tcol;
                return bs + k * SK_CB + ((((c >> 3) ^ (2 * (k & 3))) << 3) | (c & 7));
            };
            const int k = kq * 32 + 8 * g + trow;
            const half8 bf = cat4(lds_read_tr(at(k)), lds_read_tr(at(k + 4)));
            acc = mfma16(af, bf, acc);
        }
        __syncthreads();
    }
    // D: column c0 + 16 wave + l16, rows 4 g + j
    const int gc = c0 + wave * 16 + l16;
    if (nks == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = 4 * g + j;
            if (m < M && gc < N) {
                f16* dst = Cp + (int64_t)m * N + gc;
                *dst = (f16)(p.acc ? acc[j] + (float)*dst : acc[j]);
            }
        }
        return;
    }
    // the partial goes out as 16-byte row pieces: through LDS (the B stage
    // is free after the last barrier), thread t stores row t / 16, columns
    // 4 (t % 16) .. +3, written through (sc1) like the agent-scope stores
    float* ps = reinterpret_cast<float*>(bs);  // [16][SK_CB]
#pragma unroll
    for (int j = 0; j < 4; ++j) ps[(4 * g + j) * SK_CB + wave * 16 + l16] = acc[j];
    __syncthreads();
    {
        const int m = threadIdx.x / (SK_CB / 4), q = (threadIdx.x % (SK_CB / 4)) * 4;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ps + m * SK_CB + q);
        const __amdgpu_buffer_rsrc_t pres =
            buf_rsrc(part + ((int64_t)bz * nks + ks) * M * N, (uint32_t)((int64_t)M * N * 4));
        __builtin_amdgcn_raw_buffer_store_b128(v, pres, oob_or(m < M && c0 + q < N, (uint32_t)(((int64_t)m * N + c0 + q) * 4)),
                                               0, 16 /* sc1 */);
    }
    gemv_finish_m16(p, part, cnt, c0);
}



template <int BM, int BN, bool TA, bool TB>
hipError_t launch_mfma(const GemmArgs& a, int batch, hipStream_t st) {
    const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
    dim3 grid((unsigned)(tm * tn), 1, batch);
    constexpr int NWV = (BM >= 256 && BN >= 256) ? 8 : 4;  // the large tile: two waves per SIMD
    if constexpr (BM == 64) {
        // at most one tile per CU and a long K: four K groups per workgroup
        // (16 waves), so that four shorter load/compute chains overlap
        if ((int64_t)tm * tn * batch <= device_cu_count() && a.K >= 16 * MB_K) {
            hipLaunchKernelGGL((gemm_mfma<BM, BN, TA, TB, NWV, 4>), grid, dim3(64 * NWV * 4), 0, st, a, tm, tn);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemm_mfma<BM, BN, TA, TB, NWV>), grid, dim3(64 * NWV), 0, st, a, tm, tn);
    return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_mfma_t(const GemmArgs& a, int batch, bool ta, bool tb, hipStream_t st) {
    if (!ta && !tb) return launch_mfma<BM, BN, false, false>(a, batch, st);
    if (!ta && tb) return launch_mfma<BM, BN, false, true>(a, batch, st);
    if (ta && !tb) return launch_mfma<BM, BN, true, false>(a, batch, st);
    return launch_mfma<BM, BN, true, true>(a, batch, st);
}

template <class Cfg, bool TA, bool TB>
hipError_t launch_tiled(const GemmArgs& a, int batch, hipStream_t st) {
    dim3 grid((a.N + Cfg::BN - 1) / Cfg::BN, (a.M + Cfg::BM - 1) / Cfg::BM, batch);
    hipLaunchKernelGGL((gemm_tiled<Cfg, TA, TB>), grid, dim3(Cfg::NT), 0, st, a);
    return hipGetLastError();
}

template <class Cfg>
hipError_t launch_tiled_t(const GemmArgs& a, int batch, bool ta, bool tb, hipStream_t st) {
    if (!ta && !tb) return launch_tiled<Cfg, false, false>(a, batch, st);
    if (!ta && tb) return launch_tiled<Cfg, false, true>(a, batch, st);
    if (ta && !tb) return launch_tiled<Cfg, true, false>(a, batch, st);
    return launch_tiled<Cfg, true, true>(a, batch, st);
}

using CfgL = TileCfg<256, 256, 64, 2, 2>;  // 4 waves of 128x128
using CfgM = TileCfg<128, 128, 64, 2, 2>;  // 4 waves of 64x64
using CfgS = TileCfg<64, 64, 64, 2, 2>;    // 4 waves of 32x32

// Library workspace for the split-K GEMV (grow-only): partials, and the
// per-column-block arrival counters in an allocation of their own (zeroed
// once; the last arrival of every launch leaves its counter at zero).
struct GemvWorkspace {
    float* part = nullptr;
    size_t part_elems = 0;
    unsigned* counters = nullptr;
    size_t n_counters = 0;
};
GemvWorkspace g_gemv_ws;

}  // namespace

void gemm_free_workspace() {
    if (g_gemv_ws.part) (void)hipFree(g_gemv_ws.part);
    if (g_gemv_ws.counters) (void)hipFree(g_gemv_ws.counters);
    g_gemv_ws = GemvWorkspace{};
}

static int gemv_workspace(size_t part_elems, size_t n_counters, hipStream_t st) {
    if (part_elems > g_gemv_ws.part_elems) {
        if (g_gemv_ws.part) EVK_HIP(hipFree(g_gemv_ws.part));
        g_gemv_ws.part = nullptr;
        g_gemv_ws.part_elems = 0;
        EVK_HIP(hipMalloc(&g_gemv_ws.part, part_elems * sizeof(float)));
        g_gemv_ws.part_elems = part_elems;
    }
    if (n_counters > g_gemv_ws.n_counters) {
        if (g_gemv_ws.counters) EVK_HIP(hipFree(g_gemv_ws.counters));
        g_gemv_ws.counters = nullptr;
        g_gemv_ws.n_counters = 0;
        EVK_HIP(hipMalloc(&g_gemv_ws.counters, n_counters * sizeof(unsigned)));
        EVK_HIP(hipMemsetAsync(g_gemv_ws.counters, 0, n_counters * sizeof(unsigned), st));
        g_gemv_ws.n_counters = n_counters;
    }
    return EVKHIP_OK;
}

// Picks a kernel for one evk::ai::matmul call.  Shapes were validated by the
// caller; `vec_ok` says every operand is 16-byte aligned with row lengths
// that are multiples of 8 halves.
// ---- static scratch of evkhip_matmul_noalloc ----
// Device memory of the library itself, for callers that cannot allocate:
// arrival counters, then fp32 split-K partials.  Each GPU holds its own copy
// at its own address (hipGetSymbolAddress, once per device); host code uses
// only that address, never the symbol itself.
constexpr size_t kScratchCounterBytes = 64u << 10;
constexpr size_t kScratchBytes = kScratchCounterBytes + EVKHIP_NOALLOC_PART_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static void* g_scratch_addr[kMaxDevices] = {};

int noalloc_scratch(GemvScratch* out) {
    int dev = 0;
    EVK_HIP(hipGetDevice(&dev));
    EVK_RETURN_IF(dev < 0 || dev >= kMaxDevices, EVKHIP_ERR_UNSUPPORTED, "noalloc scratch: device %d", dev);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        EVK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        EVK_RETURN_IF(!p, EVKHIP_ERR_HIP, "noalloc scratch: no device address");
        g_scratch_addr[dev] = p;
    }
    char* base = static_cast<char*>(g_scratch_addr[dev]);
    out->counters = reinterpret_cast<unsigned*>(base);
    out->n_counters = kScratchCounterBytes / sizeof(unsigned);
    out->part = reinterpret_cast<float*>(base + kScratchCounterBytes);
    out->part_elems = EVKHIP_NOALLOC_PART_BYTES / sizeof(float);
    return EVKHIP_OK;
}

int gemm_dispatch(const GemmArgs& a, int batch, bool ta, bool tb, bool vec_ok, hipStream_t st,
                  const GemvScratch* fixed) {
    if (a.M == 0 || a.N == 0) return EVKHIP_OK;
    hipError_t e;
    if (!vec_ok) {
        dim3 grid((unsigned)(((int64_t)a.M * a.N + 255) / 256), batch);
        hipLaunchKernelGGL(gemm_scalar, grid, dim3(256), 0, st, a, (int)ta, (int)tb);
        e = hipGetLastError();
        return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemm_scalar launch");
    }
    if (a.M <= 16 && !ta && !tb && a.K > 0 && (int64_t)a.K * a.N * 2 < INT32_MAX &&
        (int64_t)a.M * a.K * 2 < INT32_MAX) {
        const int ncb = (a.N + SK_CB - 1) / SK_CB;
        const int nks = (a.K + SK_KC - 1) / SK_KC;
        float* part = nullptr;
        unsigned* cnt = nullptr;
        if (nks > 1) {
            const size_t need_part = (size_t)batch * nks * a.M * a.N, need_cnt = (size_t)batch * ncb;
            if (fixed) {
                EVK_RETURN_IF(need_part > fixed->part_elems || need_cnt > fixed->n_counters,
                              EVKHIP_ERR_UNSUPPORTED,
                              "matmul_noalloc: the split-K pass needs %zu partial bytes and %zu counters; the "
                              "static scratch holds %zu and %zu",
                              need_part * sizeof(float), need_cnt, fixed->part_elems * sizeof(float),
                              fixed->n_counters);
                part = fixed->part;
                cnt = fixed->counters;
                // the counters start at zero (a fill kernel: no memset node
                // under graph capture)
                int rc = fill_launch(cnt, 0u, (int64_t)(need_cnt * 2), true, st);
                if (rc) return rc;
            } else {
                int rc = gemv_workspace(need_part, need_cnt, st);
                if (rc) return rc;
                part = g_gemv_ws.part;
                cnt = g_gemv_ws.counters;
            }
        }
        dim3 grid(ncb, nks, batch);
        if (a.M <= 1) hipLaunchKernelGGL(gemv_sk<1>, grid, dim3(256), 0, st, a, part, cnt);
        else if (a.M <= 2) hipLaunchKernelGGL(gemv_sk<2>, grid, dim3(256), 0, st, a, part, cnt);
        else if (a.M <= 4) hipLaunchKernelGGL(gemv_sk<4>, grid, dim3(256), 0, st, a, part, cnt);
        else hipLaunchKernelGGL(gemv_mf, grid, dim3(256), 0, st, a, part, cnt);
        e = hipGetLastError();
        return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemv launch");
    }
    const int64_t cus = device_cu_count();
    auto tiles = [&](int bm, int bn) {
        return (int64_t)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) * batch;
    };
    // the MFMA kernel addresses each operand through a buffer descriptor
    const bool fits = (int64_t)a.M * a.K * 2 < INT32_MAX && (int64_t)a.K * a.N * 2 < INT32_MAX &&
                      (int64_t)a.M * a.N < INT32_MAX;
    if (fits) {
        if (tiles(256, 256) >= cus) e = launch_mfma_t<256, 256>(a, batch, ta, tb, st);
        else if (tiles(128, 128) >= cus / 2) e = launch_mfma_t<128, 128>(a, batch, ta, tb, st);
        else e = launch_mfma_t<64, 64>(a, batch, ta, tb, st);
    } else if (tiles(256, 256) >= cus) {
        e = launch_tiled_t<CfgL>(a, batch, ta, tb, st);
    } else if (tiles(128, 128) >= cus / 2) {
        e = launch_tiled_t<CfgM>(a, batch, ta, tb, st);
    } else {
        e = launch_tiled_t<CfgS>(a, batch, ta, tb, st);
    }
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemm launch");
}

}  // namespace evkhip
