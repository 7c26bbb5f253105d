// Internal interface between the C ABI (capi.hip) and the kernel files.
#pragma once

#include "common.h"

namespace evkhip {

// ---- gemm.hip ----
struct GemmArgs {
    const f16* A;
    const f16* B;
    f16* C;
    int M, N, K;
    int64_t sA, sB, sC;  // per-batch element strides (0 = broadcast)
    int acc;
};
// Caller-provided split-K scratch of the skinny (M <= 16) path: partials and
// arrival counters.  With it, gemm_dispatch allocates nothing.
struct GemvScratch {
    float* part;
    size_t part_elems;
    unsigned* counters;
    size_t n_counters;
};
int gemm_dispatch(const GemmArgs& a, int batch, bool ta, bool tb, bool vec_ok, hipStream_t st,
                  const GemvScratch* fixed = nullptr);
// The static per-device scratch of evkhip_matmul_noalloc, for the current
// device (its address is looked up once per device).
int noalloc_scratch(GemvScratch* out);
void gemm_free_workspace();

// ---- flash.hip ----
struct FlashArgs {
    const f16* q;
    const f16* k;
    const f16* v;
    const f16* o;
    const f16* dO;
    f16* out;          // O (forward) or dQ
    f16* dK;
    f16* dV;
    float* lse;        // public (B,H,N) fp32 or null
    float* lse2_rows;  // workspace (B, N*H): lse * log2(e) per query row
    float* d_rows;     // workspace (B, N*H): D_i = sum_j P_ij dP_ij
    int B, H, N;
    float scale_log2;  // scale * log2(e)
    float scale;
    int spin_limit;    // iterations of a bounded in-kernel wait before it gives up
};
// flash_wide.hip: MFMA forward / backward for the other multiples of 16 up
// to 256.  The backward takes the forward's O and LSE in a.o / a.lse (no
// workspace).
bool flash_wide_head(uint32_t dh);
hipError_t flash_forward_wide(const FlashArgs& a, int dh, bool causal, hipStream_t st);
hipError_t flash_backward_wide(const FlashArgs& a, int dh, bool causal, hipStream_t st);
// Head sizes with MFMA forward and backward kernels.
inline bool flash_mfma_head(uint32_t dh) { return dh == 32 || dh == 64 || dh == 128 || flash_wide_head(dh); }
// The wide-head kernels address one batch of Q (and dO, O) through 32-bit
// buffer offsets: they run only while that batch stays below 2 GiB.
inline bool flash_wide_fits(uint64_t N, uint64_t H, uint32_t dh) {
    return N * H * dh * 2u < (uint64_t)INT32_MAX;
}
int flash_forward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st);
int flash_backward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st);
void flash_free_workspace();

// ---- kv_step.hip ----
int kv_step_status(uint32_t* flags, bool clear);
void kv_step_free_workspace();

// ---- decode_persist.hip ----
int decode_status(uint32_t* flags, bool clear);
void decode_persist_free_workspace();
// Device status bits raised by the flash kernels (EVKHIP_STATUS_*): read after
// the work has completed; `clear` resets them.
int flash_status(uint32_t* flags, bool clear);
uint32_t flash_spin_limit();  // rounds of a bounded in-kernel wait (evkhip_debug_set_spin_limit)
// Spin limit of the bounded in-kernel waits (0 restores the default).
void flash_set_spin_limit(uint32_t n);

// ---- decode_ops.hip ----
// batch sequences: q, out (batch, heads*dh); sequence b's cache rows start at
// b * cache_bstride elements.
int sq_attention_launch(const f16* q, const f16* kc, const f16* vc, f16* out, int64_t row_stride, int heads,
                        int dh, int L, bool vec_ok, hipStream_t st, int batch = 1, int64_t cache_bstride = 0);
// Cache rows [pos0, pos0 + n) of each of `batch` caches (max_seq, D) take
// the rows of src (batch, n, D).
int kv_cache_write_launch(const f16* src, f16* cache, int batch, int n, int D, int max_seq, int pos0,
                          hipStream_t st);
int rms_norm_launch(const f16* in, f16* out, int64_t rows, int D, float eps, hipStream_t st);
int rope_launch(const f16* in, f16* out, int B, int S, int E, float base, int pos0, int hd, hipStream_t st);
int gelu_launch(const f16* in, f16* out, int64_t n, hipStream_t st);
int add_launch(const f16* a, const f16* b, f16* c, int64_t n, hipStream_t st);
int embed_launch(const f16* table, const uint16_t* idx, f16* out, int64_t n_idx, int dim, int vocab,
                 hipStream_t st);
int greedy_launch(const f16* logits, uint16_t* out, int B, int S, int V, int position, int token_base,
                  int token_count, hipStream_t st);
void decode_ops_free_workspace();

// ---- train_ops.hip (vec: the caller's pointers are 16-byte aligned) ----
int fill_launch(void* p, uint32_t pattern, int64_t n16, bool vec, hipStream_t st);
int scale_launch(f16* x, float s, int64_t n, bool vec, hipStream_t st);
int relu_launch(const f16* in, f16* out, int64_t n, bool vec, hipStream_t st);
int relu_bwd_launch(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec, hipStream_t st);
int gelu_bwd_launch(const f16* gout, const f16* in, f16* gin, int64_t n, bool vec, hipStream_t st);
int sgd_launch(f16* param, const f16* grad, float lr, int64_t n, bool vec, hipStream_t st);
int adam_launch(f16* param, const f16* grad, f16* m, f16* v, int64_t n, float lr, float beta1, float beta2,
                float c1inv, float c2inv, float eps, bool vec, hipStream_t st);
int softmax_launch(const f16* in, f16* out, float scale, int D, int64_t rows, bool vec, hipStream_t st);
int softmax_bwd_launch(const f16* probs, const f16* gout, f16* gin, float scale, int D, int64_t rows,
                       hipStream_t st);
int rms_norm_bwd_launch(const f16* in, const f16* gout, f16* gin, float eps, int D, int64_t rows, hipStream_t st);
int mse_loss_launch(const f16* pred, const f16* tgt, f16* grad, f16* result, int64_t n, hipStream_t st);
int cross_entropy_launch(const f16* logits, const uint16_t* tgt, f16* grad, f16* result, int64_t rows, int V,
                         bool vec, hipStream_t st);
int sum_batch_launch(const f16* in, f16* out, int batch, int64_t per_batch, hipStream_t st);
int causal_mask_launch(f16* scores, int64_t batch, int N, hipStream_t st);
int position_add_launch(const f16* in, const f16* pos, f16* out, int B, int64_t per_batch, hipStream_t st);
int position_add_bwd_launch(const f16* gout, f16* gin, f16* gpos, int B, int64_t per_batch, hipStream_t st);
int rope_bwd_launch(const f16* gout, f16* gin, int B, int S, int E, float base, hipStream_t st);
int embed_bwd_launch(const f16* gout, const uint16_t* idx, f16* gemb, int64_t n_idx, int dim, int vocab,
                     hipStream_t st);
void train_ops_free_workspace();

// ---- model.hip ----
void model_free_workspace();

}  // namespace evkhip
