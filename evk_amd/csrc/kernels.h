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
int gemm_dispatch(const GemmArgs& a, int batch, bool ta, bool tb, bool vec_ok, hipStream_t st);
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
};
int flash_forward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st);
int flash_backward(FlashArgs a, int dh, bool mfma, bool causal, hipStream_t st);
void flash_free_workspace();

// ---- decode_ops.hip ----
int sq_attention_launch(const f16* q, const f16* kc, const f16* vc, f16* out, int64_t row_stride, int heads,
                        int dh, int L, bool vec_ok, hipStream_t st);
int rms_norm_launch(const f16* in, f16* out, int64_t rows, int D, float eps, hipStream_t st);
int rope_launch(const f16* in, f16* out, int B, int S, int E, float base, int pos0, int hd, hipStream_t st);
int gelu_launch(const f16* in, f16* out, int64_t n, hipStream_t st);
int add_launch(const f16* a, const f16* b, f16* c, int64_t n, hipStream_t st);
int embed_launch(const f16* table, const uint16_t* idx, f16* out, int64_t n_idx, int dim, int vocab,
                 hipStream_t st);
int greedy_launch(const f16* logits, uint16_t* out, int B, int S, int V, int position, int token_base,
                  int token_count, hipStream_t st);
void decode_ops_free_workspace();

// ---- model.hip ----
void model_free_workspace();

}  // namespace evkhip
