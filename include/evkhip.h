/*
 * evkhip.h - C ABI of the MI355X (gfx950) kernel library behind evk::ai.
 *
 * This is the drop-in boundary: the evk::ai C++ API (include/evk_ai.h) keeps
 * the reference's signatures and calls these entry points instead of
 * recording Vulkan dispatches of the reference's SPIR-V compute shaders.
 *
 * Conventions
 *   - Every tensor is described by an evkhip_tensor: a device pointer plus the
 *     shape (row-major, contiguous).  Elements are IEEE binary16 unless the
 *     entry point says otherwise (token ids are raw uint16 in fp16 storage, as
 *     in the reference, evk_ai.h:560-566).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Entry points only
 *     enqueue work; ordering follows the stream, which reproduces the full
 *     barrier the reference records after every op (evk_ai.cpp:329 etc.).
 *   - Return value: EVKHIP_OK (0) or a negative EVKHIP_ERR_* code; the message
 *     of the last failure on the calling thread is evkhip_last_error().
 *   - Shape and argument validation happens on the host before any HIP call,
 *     so it can be exercised without a GPU.
 *   - Not thread-safe across concurrent calls that share library workspace
 *     (the reference is single-threaded with global state, evk_ai.cpp:4,63).
 */
#ifndef EVKHIP_H
#define EVKHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EVKHIP_MAX_DIMS 8

enum {
    EVKHIP_OK = 0,
    EVKHIP_ERR_INVALID_ARG = -1, /* null pointer, bad flag, inconsistent sizes */
    EVKHIP_ERR_SHAPE = -2,       /* shapes violate the op's contract            */
    EVKHIP_ERR_UNSUPPORTED = -3, /* valid request this build does not implement */
    EVKHIP_ERR_HIP = -4,         /* a HIP runtime call failed                   */
    EVKHIP_ERR_ALLOC = -5        /* workspace allocation failed                 */
};

typedef struct evkhip_tensor {
    void* data;                       /* device pointer                    */
    uint32_t rank;                    /* 1..EVKHIP_MAX_DIMS                */
    uint32_t dims[EVKHIP_MAX_DIMS];   /* dims[0] outermost                 */
} evkhip_tensor;

/* Library version string, e.g. "evkhip 0.1 gfx950". */
const char* evkhip_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* evkhip_last_error(void);

/* Replaces evk::ai::initialize (evk_ai.cpp:211-246): no pipelines to build;
 * records the current device.  Optional: every entry point works without it. */
int evkhip_init(void);

/* Replaces evk::ai::shutdown (evk_ai.cpp:248-252): frees library workspace
 * (the grow-only flash scratch, cf. evk_ai.cpp:135-157). */
int evkhip_shutdown(void);

/* Device status bits.  No counterpart in the reference, whose shaders hold
 * no in-kernel waits: a kernel of this library that waits for other waves
 * bounds the wait, and a wave that gives up (the result of that launch is
 * then unreliable) raises EVKHIP_STATUS_WAIT_TIMEOUT here instead of hanging.
 * Read after the work has completed (synchronise its stream first); `clear`
 * resets the bits. */
#define EVKHIP_STATUS_WAIT_TIMEOUT 1u
int evkhip_device_status(uint32_t* flags, int clear);

/* Test hook (no reference counterpart): iterations of the bounded in-kernel
 * waits before they give up; 0 restores the default (2^22).  Lets a test
 * force the timeout path from the host without any wave actually stalling. */
int evkhip_debug_set_spin_limit(uint32_t iterations);

/* evk::ai::matmul (evk_ai.h:495, evk_ai.cpp:254-330).
 * C[b] (+)= op(A[b]) . op(B[b]):  A (...,M,K) or (...,K,M) if transpose_a;
 * B (...,K,N) or (...,N,K) if transpose_b; C (...,M,N).  batch = max of the
 * operands' leading-dim products; an input with batch 1 broadcasts.  fp32
 * accumulation, fp16 output; acc_c adds the prior C.  tile_m/tile_n are the
 * reference's tile hints: accepted (and validated as multiples of 16 when
 * nonzero) but the kernel picks its own MFMA tiling, and M, N, K need not be
 * multiples of them. */
int evkhip_matmul(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c,
                  int transpose_a, int transpose_b, int acc_c,
                  uint32_t tile_m, uint32_t tile_n, void* stream);

/* evk::ai::matmul for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference.  Same arguments, results, errors and
 * kernels as evkhip_matmul, but it never allocates: the split-K partials and
 * arrival counters of the skinny (M <= 16) path live in a static per-device
 * array of EVKHIP_NOALLOC_PART_BYTES of partials (plus 64 KiB of counters),
 * held by each GPU the library runs on until the process ends.  A call whose
 * split-K pass needs more (batch * ceil(K/512) * M * N * 4 bytes) returns
 * EVKHIP_ERR_UNSUPPORTED before launching anything.  Every call on one GPU
 * shares that array and clears the counters it uses: calls that overlap on
 * one GPU (on different streams) race. */
#define EVKHIP_NOALLOC_PART_BYTES (8u << 20)
int evkhip_matmul_noalloc(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c,
                          int transpose_a, int transpose_b, int acc_c,
                          uint32_t tile_m, uint32_t tile_n, void* stream);

/* evk::ai::flash_attention (evk_ai.h:497-501, evk_ai.cpp:332-369).
 * MQA: Q,O (B,N,H*Dh); K,V (B,N,Dh); H = D/Dh; scale 1/sqrt(Dh).
 * Extensions (defaults reproduce the reference): causal != 0 masks keys
 * j > i; lse, if non-NULL, receives the fp32 log-sum-exp of every (b,h,i)
 * row, laid out (B,H,N).  Dh up to 256: multiples of 16 run MFMA kernels
 * (evkhip_flash_kernel_path), other sizes a scalar kernel. */
int evkhip_flash_attention(const evkhip_tensor* q, const evkhip_tensor* k,
                           const evkhip_tensor* v, const evkhip_tensor* o,
                           int causal, float* lse, void* stream);

/* Non-zero when the flash forward and backward run MFMA kernels for this
 * head size (no reference counterpart); other sizes take a scalar path. */
int evkhip_flash_has_mfma(uint32_t head_dim);

/* Which kernel family serves flash attention (forward and backward) at N
 * positions, `heads` query heads of head_dim (no reference counterpart; a
 * host-side query, no GPU work): MFMA kernels for 32, 64 and 128, the wide
 * MFMA kernels for the other multiples of 16 up to 256 while one batch of Q
 * stays below 2 GiB, the scalar kernels otherwise (pointers that are not
 * 16-byte aligned also take the scalar kernels). */
#define EVKHIP_FLASH_PATH_SCALAR 0
#define EVKHIP_FLASH_PATH_MFMA 1
#define EVKHIP_FLASH_PATH_WIDE 2
int evkhip_flash_kernel_path(uint32_t n, uint32_t heads, uint32_t head_dim);

/* evk::ai::flash_attention_bwd (evk_ai.h:503, evk_ai.cpp:371-473).
 * dQ (B,N,D); dK,dV (B,N,Dh) summed over the H heads sharing them.
 * heads != 0 must equal D/Dh.  With lse == NULL the row statistics and
 * D_i = sum_j P_ij dP_ij are recomputed from Q,K,V,dO and `o` is not read
 * (the reference never reads it either); with lse from the forward pass,
 * D_i = rowsum(dO_i * O_i) is taken from `o` and the recompute is skipped.
 * Uses library workspace (grow-only, freed by evkhip_shutdown). */
int evkhip_flash_attention_bwd(const evkhip_tensor* q, const evkhip_tensor* k,
                               const evkhip_tensor* v, const evkhip_tensor* o,
                               const evkhip_tensor* dO, const evkhip_tensor* dQ,
                               const evkhip_tensor* dK, const evkhip_tensor* dV,
                               uint32_t heads, int causal, const float* lse, void* stream);

/* Decode-step attention: the host entry that single_query_attention.comp
 * (lines 26-72) never had.  q (heads*dh) or (1,1,heads*dh); k_cache, v_cache
 * (...,max_len,heads*dh) row-major; attends over cache rows
 * [0,current_length).  heads == 1, dh <= 64, current_length <= 160 is the
 * shader's contract; this entry lifts those limits (split-K with a merge). */
int evkhip_single_query_attention(const evkhip_tensor* q, const evkhip_tensor* k_cache,
                                  const evkhip_tensor* v_cache, const evkhip_tensor* out,
                                  uint32_t current_length, uint32_t heads, void* stream);
/* Batched form of the same entry (B sequences decoded together, e.g. the
 * B = 16 of example/main_llm.cpp:622-654): caches (B, max_len, D) with B > 1,
 * q and out (B, D) or (B, 1, D); sequence b attends over rows
 * [0, current_length) of its own cache. */

/* KV-cache append (no reference counterpart; the reference recomputes the
 * whole sequence instead, main_llm.cpp:622-654): rows [pos0, pos0 + n) of
 * each sequence's cache take that sequence's rows of src.
 * src (B, n, D) or (n, D); cache (B, max_seq, D) or (max_seq, D). */
int evkhip_kv_cache_write(const evkhip_tensor* src, const evkhip_tensor* cache, uint32_t pos0, void* stream);

/* evk::ai::rms_norm (evk_ai.h:610, evk_ai.cpp:1045-1067, rms_norm.comp). */
int evkhip_rms_norm(const evkhip_tensor* in, const evkhip_tensor* out, float eps, void* stream);

/* evk::ai::rope (evk_ai.h:589-591, evk_ai.cpp:945-966, rope.comp).
 * Extensions (0 reproduces the reference): position t = position_offset +
 * sequence index; head_dim splits embed_dim into independently rotated heads
 * whose frequencies use head_dim (0 means embed_dim). */
int evkhip_rope(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t batch_size,
                uint32_t seq_len, uint32_t embed_dim, float rotary_base,
                uint32_t position_offset, uint32_t head_dim, void* stream);

/* evk::ai::gelu (evk_ai.h:540, evk_ai.cpp:679-699, gelu.comp). */
int evkhip_gelu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream);

/* evk::ai::add (evk_ai.h:521, evk_ai.cpp:568-591, add.comp). */
int evkhip_add(const evkhip_tensor* a, const evkhip_tensor* b, const evkhip_tensor* c,
               void* stream);

/* evk::ai::embed (evk_ai.h:558, evk_ai.cpp:782-806, embed.comp).
 * Indices are raw uint16 ids; ids >= vocab are clamped to vocab-1. */
int evkhip_embed(const evkhip_tensor* embeddings, const evkhip_tensor* indices,
                 const evkhip_tensor* out, void* stream);

/* evk::ai::greedy_sample (evk_ai.h:563-566, evk_ai.cpp:808-837,
 * greedy_sample.comp).  Same winner as the shader, including its tie order. */
int evkhip_greedy_sample(const evkhip_tensor* logits, const evkhip_tensor* out_tokens,
                         uint32_t position, uint16_t token_base, uint16_t token_count,
                         void* stream);

/* ---------------------------------------------------------------------------
 * Training ops: what the reference's Graph (evk_ai.h:616-1074) runs besides
 * matmul and flash attention.  Gradient outputs that the shader accumulates
 * into (grad_in += ...) are accumulated here too; every stored value is
 * rounded to fp16 as the shader rounds it.
 * ------------------------------------------------------------------------- */

/* Device fill by a kernel (so a captured HIP graph holds no memset node):
 * `bytes` (even) at `data` take the 32-bit little-endian `pattern` repeated;
 * a trailing 16-bit word takes its low half.  Backs evk::ai::zero
 * (evk_ai.cpp:139-147, which records vkCmdFillBuffer) and evk::Cmd::fill
 * (evk.h Cmd::fill, evk_vulkan.cpp vkCmdFillBuffer). */
int evkhip_fill(void* data, uint64_t bytes, uint32_t pattern, void* stream);

/* evk::ai::scale (evk_ai.h:599, evk_ai.cpp:992-1007, scale.comp): in place,
 * t = t * factor. */
int evkhip_scale(const evkhip_tensor* t, float factor, void* stream);

/* evk::ai::relu (evk_ai.h:533, evk_ai.cpp:636-656, relu.comp). */
int evkhip_relu(const evkhip_tensor* in, const evkhip_tensor* out, void* stream);

/* evk::ai::relu_backward (evk_ai.h:536, evk_ai.cpp:658-677, relu_bwd.comp):
 * grad_in += (in > 0 ? grad_out : 0). */
int evkhip_relu_backward(const evkhip_tensor* grad_out, const evkhip_tensor* in, const evkhip_tensor* grad_in,
                         void* stream);

/* evk::ai::gelu_backward (evk_ai.h:543, evk_ai.cpp:701-720, gelu_bwd.comp):
 * grad_in += grad_out * d gelu(in) / d in (tanh form). */
int evkhip_gelu_backward(const evkhip_tensor* grad_out, const evkhip_tensor* in, const evkhip_tensor* grad_in,
                         void* stream);

/* evk::ai::mse_loss (evk_ai.h:507, evk_ai.cpp:475-497, mse_loss.comp):
 * result[0] = mean((p - t)^2), pred_grad = 2 (p - t) / n. */
int evkhip_mse_loss(const evkhip_tensor* predicted, const evkhip_tensor* target, const evkhip_tensor* pred_grad,
                    const evkhip_tensor* result, void* stream);

/* evk::ai::sgd (evk_ai.h:510, evk_ai.cpp:499-519, sgd.comp):
 * param -= learning_rate * gradient. */
int evkhip_sgd(const evkhip_tensor* param, const evkhip_tensor* gradient, float learning_rate, void* stream);

/* evk::ai::adam (evk_ai.h:514-518, evk_ai.cpp:521-566, adam.comp): one step
 * with the caller's bias corrections 1/(1-beta1^t), 1/(1-beta2^t).  State
 * (same element count as param, fp16): m_state = m / rms and v_state =
 * log2(rms) + 41 (0 = rms 0), as the shader keeps them; zero-initialised
 * state is a fresh optimiser. */
int evkhip_adam(const evkhip_tensor* param, const evkhip_tensor* gradient, const evkhip_tensor* m_state,
                const evkhip_tensor* v_state, float learning_rate, float beta1, float beta2,
                float beta1_correction_inv, float beta2_correction_inv, float epsilon, void* stream);

/* evk::ai::softmax (evk_ai.h:525, evk_ai.cpp:593-613, softmax.comp): over
 * the last dimension of in * input_scale; entries <= -65504 are masked out
 * (probability 0). */
int evkhip_softmax(const evkhip_tensor* in, const evkhip_tensor* out, float input_scale, void* stream);

/* evk::ai::softmax_backward (evk_ai.h:529, evk_ai.cpp:615-634,
 * softmax_bwd.comp): grad_in += probs * (grad_out - dot(grad_out, probs)) * scale
 * per row of the last dimension. */
int evkhip_softmax_backward(const evkhip_tensor* probs, const evkhip_tensor* grad_out,
                            const evkhip_tensor* grad_in, float scale, void* stream);

/* evk::ai::rms_norm_backward (evk_ai.h:614, evk_ai.cpp:1072-1093,
 * rms_norm_bwd.comp): grad_in += (g - y dot(g, y) / D) / rms per row. */
int evkhip_rms_norm_backward(const evkhip_tensor* in, const evkhip_tensor* grad_out,
                             const evkhip_tensor* grad_in, float eps, void* stream);

/* evk::ai::cross_entropy_loss (evk_ai.h:552, evk_ai.cpp:722-780,
 * cross_entropy*.comp): logits (P,V), targets (P) raw uint16; target 0 or
 * >= V is ignored.  grad = (softmax - onehot) / n_valid (zero rows for
 * ignored targets); result[0] = mean loss over valid rows (0 if none).  The
 * per-row losses are summed in row order (deterministic). */
int evkhip_cross_entropy_loss(const evkhip_tensor* logits, const evkhip_tensor* targets,
                              const evkhip_tensor* grad, const evkhip_tensor* result, void* stream);

/* evk::ai::sum_batch (evk_ai.h:605, evk_ai.cpp:1027-1041, sum_batch.comp):
 * out[i] += sum_b in[b * size_per_batch + i]. */
int evkhip_sum_batch(const evkhip_tensor* in, const evkhip_tensor* out, uint32_t batch_count,
                     uint32_t size_per_batch, void* stream);

/* evk::ai::apply_causal_mask (evk_ai.h:577, evk_ai.cpp:862-882,
 * causal_mask.comp): scores (..., N, N), entries j > i set to -65504. */
int evkhip_apply_causal_mask(const evkhip_tensor* scores, void* stream);

/* evk::ai::position_add (evk_ai.h:580-581, evk_ai.cpp:885-905,
 * position_add.comp): out[b,t,:] = in[b,t,:] + pos_emb[t,:]. */
int evkhip_position_add(const evkhip_tensor* in, const evkhip_tensor* pos_emb, const evkhip_tensor* out,
                        uint32_t batch_size, uint32_t seq_len, uint32_t embed_dim, void* stream);

/* evk::ai::position_add_backward (evk_ai.h:584-585, evk_ai.cpp:907-943,
 * position_add_bwd.comp): grad_in += grad_out; grad_pos[t,:] += sum_b grad_out[b,t,:]. */
int evkhip_position_add_backward(const evkhip_tensor* grad_out, const evkhip_tensor* grad_in,
                                 const evkhip_tensor* grad_pos, uint32_t batch_size, uint32_t seq_len,
                                 uint32_t embed_dim, void* stream);

/* evk::ai::rope_backward (evk_ai.h:594-596, evk_ai.cpp:968-989, rope_bwd.comp):
 * grad_in += the transposed rotation of grad_out (positions from 0). */
int evkhip_rope_backward(const evkhip_tensor* grad_out, const evkhip_tensor* grad_in, uint32_t batch_size,
                         uint32_t seq_len, uint32_t embed_dim, float rotary_base, void* stream);

/* evk::ai::embed_backward (evk_ai.h:572, evk_ai.cpp:839-860, embed_bwd.comp):
 * grad_embeddings[idx[r]] += grad_out[r] for r in order (the shader's
 * sequence of fp16 roundings); ids >= vocab are skipped. */
int evkhip_embed_backward(const evkhip_tensor* grad_out, const evkhip_tensor* indices,
                          const evkhip_tensor* grad_embeddings, void* stream);

/* ---------------------------------------------------------------------------
 * KV-cached greedy decode (the caller the single-query path exists for; the
 * reference decodes by full recompute, example/main_llm.cpp:622-654).  The
 * model is the reference block (main_llm.cpp:528-546) in multi-head,
 * KV-cached form.  Weights: one fp16 blob laid out
 *   E (vocab,d); per layer Wqkv (d,3d) [q|k|v], Wo (d,d), W1 (d,hidden),
 *   W2 (hidden,d); Wout (d,vocab)
 * Cache: per layer K (max_seq,d) then V (max_seq,d).
 * ------------------------------------------------------------------------- */
typedef struct evkhip_model_cfg {
    uint32_t vocab, d, heads, dh, layers, hidden, max_seq;
    float eps, rope_base;
} evkhip_model_cfg;

/* Elements (fp16) of the weight blob / the KV cache for `cfg`. */
uint64_t evkhip_model_weight_elems(const evkhip_model_cfg* cfg);
uint64_t evkhip_model_cache_elems(const evkhip_model_cfg* cfg);

/* Prefill: runs prompt tokens[0..n_tokens) (device, uint16) at positions
 * pos0.. through the model, appending to the cache; then writes the last
 * position's logits (device, fp16 vocab) and its greedy id to next_id[0]
 * (device uint16).  Workspace is library-owned. */
int evkhip_model_prefill(const evkhip_model_cfg* cfg, const void* weights, void* cache,
                         const uint16_t* tokens, uint32_t n_tokens, uint32_t pos0,
                         uint16_t* next_id, void* logits, void* stream);

/* Greedy decode: token_io (device, uint16, n_steps+1 entries).  Step s feeds
 * token_io[s] at position pos0+s and writes its greedy id to token_io[s+1],
 * which the next step's embedding reads on the device (no host round trip).
 * logits (device, fp16 vocab) holds the last step's logits. */
int evkhip_model_decode(const evkhip_model_cfg* cfg, const void* weights, void* cache,
                        uint16_t* token_io, uint32_t n_steps, uint32_t pos0, void* logits,
                        void* stream);

/* Persistent decode (no counterpart in the reference: the reference decodes
 * by full recompute, example/main_llm.cpp:622-654).  evkhip_model_pack writes
 * the decode layout of a weight blob: E as is, every matrix transposed to
 * (out, in) (Wqkv^T (3d,d), Wo^T, W1^T (hidden,d), W2^T (d,hidden), Wout^T
 * (vocab,d)); evkhip_model_packed_elems elements, the same count.  Pack once
 * per weight set (and again after the weights change).
 * evkhip_model_decode_packed then has the meaning of evkhip_model_decode but
 * runs all n_steps in one persistent launch (one workgroup per CU, all
 * resident at once) whose stages hand their outputs over in device memory.  It needs d and hidden multiples of 8 (at most 8192
 * each), dh in {16,32,64,128}, max_seq <= 8192, heads * ceil(max_seq / 128)
 * <= 144 and no more than the workgroups it runs (one per CU), and
 * per-workgroup weight slices that fit in LDS (d=768, hidden=3072 do); other
 * shapes (or a GPU on which the launch cannot be resident at once) return
 * EVKHIP_ERR_UNSUPPORTED and evkhip_model_decode serves them.  Its in-kernel waits are bounded: one that
 * gives up raises EVKHIP_STATUS_WAIT_TIMEOUT (evkhip_device_status) and the
 * outputs of that call are then unreliable.  Calls that overlap on one GPU
 * race on the library's hand-over buffers. */
/* Fused KV-cached decode step of evk::ai::KVCacheDecoder (no reference
 * counterpart; the reference recomputes every position per sampled token,
 * example/main_llm.cpp:622-654, with the blocks of main_llm.cpp:528-546):
 * one launch runs, for each of `batch` sequences, one new position `pos`
 * through every layer (rms_norm; q, k, v = x.Wq, x.Wk, x.Wv; rope on q and k
 * with head size d at pos; the position's k, v written to row pos of the
 * caches; single-head causal attention over rows [0, pos]; x += attn.Wo;
 * x += gelu(rms_norm(x).W1).W2) and writes the logits rms_norm(x).Wout,
 * fp16 (batch, vocab).  Every op output is rounded to fp16 as the op-by-op
 * step rounds it.  Weights as the Graph stores them, (in, out) row-major:
 * w[l] = {Wq, Wk, Wv, Wo (d,d), W1 (d,hidden), W2 (hidden,d)}; emb (vocab,d),
 * w_out (d,vocab); k_cache[l], v_cache[l] (batch, max_seq, d); ids (batch)
 * raw uint16 token ids of position pos.  Needs d, hidden, vocab multiples of
 * 8 (d <= 2048, hidden <= 8192), max_seq <= 8192, at most
 * EVKHIP_KV_MAX_LAYERS layers and 16-byte aligned pointers, else
 * EVKHIP_ERR_UNSUPPORTED (the op-by-op step serves those shapes).  d = 256
 * with hidden a multiple of 256 up to 1024 (the reference caller's shape)
 * takes a kernel that streams the weights with loads always in flight,
 * on two workgroups a sequence that swap their halves of every product in
 * device memory when all 2 * batch of them fit on the GPU at once and the
 * stream is not being captured (else on one workgroup a sequence); other
 * shapes take a general one.  They sum in different orders.  The
 * two-workgroup waits are bounded: one that gives up raises
 * EVKHIP_STATUS_WAIT_TIMEOUT (evkhip_device_status) and the outputs of that
 * call are then unreliable.  Calls that overlap on one GPU race on its
 * hand-over buffers. */
#define EVKHIP_KV_MAX_LAYERS 24
typedef struct evkhip_kv_model {
    uint32_t batch, d, hidden, vocab, layers, max_seq;
    float eps, rope_base;
    const void* emb;
    const void* w_out;
    const void* w[EVKHIP_KV_MAX_LAYERS][6];
    void* k_cache[EVKHIP_KV_MAX_LAYERS];
    void* v_cache[EVKHIP_KV_MAX_LAYERS];
} evkhip_kv_model;
int evkhip_kv_decode_step(const evkhip_kv_model* m, const uint16_t* ids, uint32_t pos, void* logits,
                          void* stream);

/* Test hook of evkhip_model_decode_packed (no reference counterpart): sets
 * the hand-over epoch of this device's persistent decode `distance` tags
 * below the point where the tags wrap, so that the next launch that needs
 * more tags than that clears the mailboxes and restarts them from zero.
 * Synchronises the device; needs a persistent decode to have run on it. */
int evkhip_debug_decode_set_epoch(uint32_t distance);

/* Test hook of evkhip_kv_decode_step (no reference counterpart): puts the
 * launch counter that tags the two-workgroup step's hand-overs `distance`
 * launches below the point where it wraps, so that the launch that reaches
 * it clears the mailboxes and restarts the tags.  Synchronises the device;
 * needs a two-workgroup step to have run in this process. */
int evkhip_debug_kv_set_launch(uint32_t distance);
uint64_t evkhip_model_packed_elems(const evkhip_model_cfg* cfg);
int evkhip_model_pack(const evkhip_model_cfg* cfg, const void* weights, void* packed, void* stream);
int evkhip_model_decode_packed(const evkhip_model_cfg* cfg, const void* packed, void* cache,
                               uint16_t* token_io, uint32_t n_steps, uint32_t pos0, void* logits,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EVKHIP_H */
