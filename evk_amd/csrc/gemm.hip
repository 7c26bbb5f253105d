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
// workgroups with a deterministic last-arriving-block reduction.
#include "kernels.h"

#include <algorithm>

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
// Workgroup: 4 waves; columns [n0, n0+512) (lane owns 8 columns); wave w
// handles rows k0 + w + 4t of the workgroup's K slice.  Partial sums of the
// 4 waves meet in LDS; the KS slices meet in `part` and the last-arriving
// workgroup of each column block adds them in slice order.
constexpr int GV_COLS = 512;
constexpr int GV_WAVES = 4;

template <int MR>
__global__ __launch_bounds__(256) void gemv_nn(GemmArgs p, int kslice, float* __restrict__ part,
                                               unsigned* __restrict__ counters) {
    __shared__ float red[GV_WAVES][4][GV_COLS];
    __shared__ float sa[MR][256];
    __shared__ unsigned s_last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nblk = blockIdx.x, split = blockIdx.y, bz = blockIdx.z;
    const int nsplit = gridDim.y;
    const int M = p.M, N = p.N, K = p.K;
    const f16* __restrict__ A = p.A + (int64_t)bz * p.sA;
    const f16* __restrict__ B = p.B + (int64_t)bz * p.sB;
    f16* __restrict__ Cp = p.C + (int64_t)bz * p.sC;
    const int n = nblk * GV_COLS + lane * 8;
    const int kbeg = split * kslice, kend = min(K, kbeg + kslice);

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[m][c] = 0.0f;

    for (int kc = kbeg; kc < kend; kc += 256) {
        __syncthreads();
        for (int t = threadIdx.x; t < MR * 256; t += 256) {
            int m = t / 256, kk = kc + (t % 256);
            sa[m][t % 256] = (m < M && kk < kend) ? (float)A[(int64_t)m * K + kk] : 0.0f;
        }
        __syncthreads();
        const int klim = min(256, kend - kc);
        if (n < N) {
            int kk = wave;
#pragma unroll 4
            for (; kk < klim; kk += GV_WAVES) {
                u32x4 w = *reinterpret_cast<const u32x4*>(B + (int64_t)(kc + kk) * N + n);
                half8 h = as_half8(w);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float av = sa[m][kk];
#pragma unroll
                    for (int c = 0; c < 8; ++c) acc[m][c] += av * (float)h[c];
                }
            }
        }
    }

    // reduce the 4 waves, 4 rows of M at a time
    const bool single = (nsplit == 1);
    for (int mb = 0; mb < MR; mb += 4) {
        __syncthreads();
#pragma unroll
        for (int mm = 0; mm < 4; ++mm)
            if (mb + mm < MR)
#pragma unroll
                for (int c = 0; c < 8; ++c) red[wave][mm][lane * 8 + c] = acc[mb + mm][c];
        __syncthreads();
        for (int t = threadIdx.x; t < 4 * GV_COLS; t += 256) {
            int mm = t / GV_COLS, col = t % GV_COLS;
            int m = mb + mm, gc = nblk * GV_COLS + col;
            if (m >= M || m >= MR || gc >= N) continue;
            float s = red[0][mm][col] + red[1][mm][col] + red[2][mm][col] + red[3][mm][col];
            if (single) {
                f16* dst = Cp + (int64_t)m * N + gc;
                if (p.acc) s += (float)*dst;
                *dst = (f16)s;
            } else {
                part[(((int64_t)bz * nsplit + split) * M + m) * N + gc] = s;
            }
        }
    }
    if (single) return;

    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned* cnt = counters + (int64_t)bz * gridDim.x + nblk;
        unsigned prev = atomicAdd(cnt, 1u);
        s_last = (prev == (unsigned)(nsplit - 1));
        if (s_last) *cnt = 0u;  // ready for the next launch
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int t = threadIdx.x; t < M * GV_COLS; t += 256) {
        int m = t / GV_COLS, gc = nblk * GV_COLS + (t % GV_COLS);
        if (gc >= N) continue;
        float s = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp)
            s += __hip_atomic_load(part + (((int64_t)bz * nsplit + sp) * M + m) * N + gc,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        f16* dst = Cp + (int64_t)m * N + gc;
        if (p.acc) s += (float)*dst;
        *dst = (f16)s;
    }
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

// Library workspace for the split-K GEMV (grow-only).
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

static int gemv_workspace(size_t part_elems, size_t n_counters) {
    if (part_elems > g_gemv_ws.part_elems) {
        if (g_gemv_ws.part) EVK_HIP(hipFree(g_gemv_ws.part));
        g_gemv_ws.part = nullptr;
        EVK_HIP(hipMalloc(&g_gemv_ws.part, part_elems * sizeof(float)));
        g_gemv_ws.part_elems = part_elems;
    }
    if (n_counters > g_gemv_ws.n_counters) {
        if (g_gemv_ws.counters) EVK_HIP(hipFree(g_gemv_ws.counters));
        g_gemv_ws.counters = nullptr;
        EVK_HIP(hipMalloc(&g_gemv_ws.counters, n_counters * sizeof(unsigned)));
        EVK_HIP(hipMemset(g_gemv_ws.counters, 0, n_counters * sizeof(unsigned)));
        g_gemv_ws.n_counters = n_counters;
    }
    return EVKHIP_OK;
}

// Picks a kernel for one evk::ai::matmul call.  Shapes were validated by the
// caller; `vec_ok` says every operand is 16-byte aligned with row lengths
// that are multiples of 8 halves.
int gemm_dispatch(const GemmArgs& a, int batch, bool ta, bool tb, bool vec_ok, hipStream_t st) {
    if (a.M == 0 || a.N == 0) return EVKHIP_OK;
    hipError_t e;
    if (!vec_ok) {
        dim3 grid((unsigned)(((int64_t)a.M * a.N + 255) / 256), batch);
        hipLaunchKernelGGL(gemm_scalar, grid, dim3(256), 0, st, a, (int)ta, (int)tb);
        e = hipGetLastError();
        return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemm_scalar launch");
    }
    if (a.M <= 16 && !ta && !tb && a.K > 0) {
        const int nblk = (a.N + GV_COLS - 1) / GV_COLS;
        const int cus = device_cu_count();
        // aim for ~2 workgroups per CU; K slices are multiples of 256 rows
        int want = std::max(1, (2 * cus + nblk * batch - 1) / (nblk * batch));
        int kslice = std::max(256, ((a.K + want - 1) / want + 255) / 256 * 256);
        int nsplit = (a.K + kslice - 1) / kslice;
        float* part = nullptr;
        unsigned* cnt = nullptr;
        if (nsplit > 1) {
            int rc = gemv_workspace((size_t)batch * nsplit * a.M * a.N, (size_t)batch * nblk);
            if (rc) return rc;
            part = g_gemv_ws.part;
            cnt = g_gemv_ws.counters;
        }
        dim3 grid(nblk, nsplit, batch);
        if (a.M <= 1) hipLaunchKernelGGL(gemv_nn<1>, grid, dim3(256), 0, st, a, kslice, part, cnt);
        else if (a.M <= 2) hipLaunchKernelGGL(gemv_nn<2>, grid, dim3(256), 0, st, a, kslice, part, cnt);
        else if (a.M <= 4) hipLaunchKernelGGL(gemv_nn<4>, grid, dim3(256), 0, st, a, kslice, part, cnt);
        else if (a.M <= 8) hipLaunchKernelGGL(gemv_nn<8>, grid, dim3(256), 0, st, a, kslice, part, cnt);
        else hipLaunchKernelGGL(gemv_nn<16>, grid, dim3(256), 0, st, a, kslice, part, cnt);
        e = hipGetLastError();
        return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemv launch");
    }
    const int64_t cus = device_cu_count();
    auto tiles = [&](int bm, int bn) {
        return (int64_t)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) * batch;
    };
    if (tiles(256, 256) >= cus) e = launch_tiled_t<CfgL>(a, batch, ta, tb, st);
    else if (tiles(128, 128) >= cus / 2) e = launch_tiled_t<CfgM>(a, batch, ta, tb, st);
    else e = launch_tiled_t<CfgS>(a, batch, ta, tb, st);
    return e == hipSuccess ? EVKHIP_OK : check_hip(e, "gemm launch");
}

}  // namespace evkhip
