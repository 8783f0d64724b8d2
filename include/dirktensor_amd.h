/*
 * dirktensor_amd — C ABI for the MI355X (gfx950) causal-attention path.
 *
 * Plain pointers, sizes and status codes only; no HIP, torch or C++ types in
 * the signatures (streams are passed as `void*` holding a hipStream_t, NULL
 * meaning the null stream). Every entry point validates its arguments before
 * it makes any HIP call and returns DT_OK (0) or a negative status; the message
 * for the last failure on the calling thread is available from dt_last_error().
 *
 * Tensor layout is the reference's: BTHD (batch, sequence, head, head_dim),
 * row-major and contiguous, head h occupying features [h*D, (h+1)*D) of a
 * d_model = H*D row (OlmoAttention.cpp:71; FlashAttention.cpp:87-88).
 *
 * Modes:
 *   DT_FP32_EXACT  fp32 inputs/outputs, fp32 MFMA (v_mfma_f32_32x32x2_f32),
 *                  fp32 accumulation; parity target 1e-4 of max|O|.
 *   DT_BF16        bf16 Q/K/V/O, bf16 MFMA (v_mfma_f32_32x32x16_bf16) with
 *                  fp32 accumulation and fp32 softmax; parity target 2e-2.
 *   m and l are always fp32.
 *
 * Memory:
 *   DT_MEM_DEVICE  all tensor pointers are device pointers; the call is
 *                  stream-ordered and returns without synchronising.
 *   DT_MEM_HOST    all tensor pointers are host pointers; the call copies in,
 *                  runs, copies out and synchronises (the reference's
 *                  synchronous value semantics).
 *   seq_lens is always a host pointer (B int32 values) or NULL.
 */
#ifndef DIRKTENSOR_AMD_H
#define DIRKTENSOR_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DT_OK 0
#define DT_ERR_INVALID_ARG (-1)
#define DT_ERR_UNSUPPORTED (-2)
#define DT_ERR_HIP (-3)
#define DT_ERR_BLAS (-4)
#define DT_ERR_NOT_IMPLEMENTED (-5)
#define DT_ERR_IO (-6)

#define DT_FP32_EXACT 0
#define DT_BF16 1

#define DT_MEM_DEVICE 0
#define DT_MEM_HOST 1

/* Model constants the kernels are built for (model_config.h:3-7). */
#define DT_HEAD_DIM 128
#define DT_MAX_SEQ_LEN 8192
#define DT_D_MODEL 2048
#define DT_N_HEADS 16
#define DT_ROPE_THETA 500000.0f /* OlmoAttention.cpp:16 */
#define DT_RMS_EPS 1e-6f        /* RMSNorm.h:10 */

typedef struct dt_ctx dt_ctx;
typedef struct dt_attn_layer dt_attn_layer;

/* Message describing the last failed call on this thread ("" if none). */
const char* dt_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int dt_version(void);

/*
 * Context: owns the device binding, the RoPE tables, the rocBLAS handle and the
 * host-memory staging buffers. Not thread-safe: use one per host thread.
 * Its workspaces (the hipBLASLt split-K buffer, the attention backward's row
 * statistics, the staging buffers) are shared by every call made with it, so
 * calls on one context must be ordered: issue them on one stream, or make a
 * stream wait (an event) for the previous call's stream before the next call.
 * Two calls on one context running at the same time on different streams race
 * on those workspaces. Use one context per stream for concurrent work.
 * No reference counterpart: the reference keeps this state in file-scope
 * statics (OlmoAttention.cpp:34-36) and in TBB's global pool.
 */
int dt_ctx_create(int device, dt_ctx** out);
int dt_ctx_destroy(dt_ctx* ctx);

/*
 * Context options (no reference counterpart).
 *   DT_OPT_QKV_FUSED  how dt_attn_layer_fwd (and the model forward) computes
 *                     the Q/K/V projection, the q/k RMSNorm and RoPE
 *                     (OlmoAttention.cpp:63-88):
 *                     DT_QKV_GEMM  one library GEMM, then a norm + RoPE kernel;
 *                     DT_QKV_FUSED one fused kernel (same results within the
 *                                  mode's tolerance);
 *                     DT_QKV_AUTO  (default) in DT_BF16 mode the fused kernel
 *                                  when its 128-row x one-head tiles fit one
 *                                  round on the GPU's CUs (B*T <= 640 at 16
 *                                  heads on MI355X), where it measured faster;
 *                                  the GEMM path above that and in
 *                                  DT_FP32_EXACT mode.
 *   DT_OPT_GEMM_TUNE  1 (default): the first bf16 GEMM of each new shape in
 *                     the process times hipBLASLt's heuristic candidates
 *                     (up to 16, into a scratch output; synchronises the
 *                     stream once; skipped while the stream is capturing a
 *                     graph) and keeps the first heuristic choice unless a
 *                     candidate whose repeated run is bit-identical is at
 *                     least 5 % faster (then the best-ranked candidate within
 *                     3 % of the fastest). The choice is shared by every
 *                     context of the process, so their bf16 GEMM results are
 *                     bit-identical; another process may time the candidates
 *                     differently and choose another algorithm, whose results
 *                     can differ in the last bits. 0: the first heuristic
 *                     choice, the same in every process.
 *   DT_OPT_BWD_DQ     how the attention backward (dt_flash_attn_bwd,
 *                     dt_attn_layer_bwd, the model backward) forms dQ
 *                     (FlashAttention.cpp:185-359), in both modes:
 *                     DT_BWD_DQ_RECOMPUTE  the dQ pass recomputes S and dP
 *                                          (no workspace);
 *                     DT_BWD_DQ_FROM_DS    the dK/dV pass stores dS in the
 *                                          mode's dtype (B*H*T*(T+128)/2
 *                                          values causal, B*H*T*T otherwise,
 *                                          a context buffer) and dQ = dS K
 *                                          reads it;
 *                     DT_BWD_DQ_AUTO       (default) the dS path where it
 *                                          measured faster (more than one
 *                                          128-row block per CU and pass)
 *                                          and its buffer needs at most
 *                                          2 GiB and a quarter of the free
 *                                          device memory; the recompute
 *                                          path otherwise or when the
 *                                          buffer cannot be had. The buffer
 *                                          is kept until dt_ctx_destroy.
 *                     Both give the same results within the mode's
 *                     tolerance; each is deterministic.
 *   DT_OPT_QKV_SPIN_LIMIT  polls (default 1048576, about a second) that a
 *                     workgroup of the fused QKV kernel spends waiting for the
 *                     other heads' row sums of squares before it gives up.
 *                     The kernel runs its H tiles of a row block in one round
 *                     (one workgroup per CU); a workgroup kept off its CU that
 *                     long (by another kernel holding CUs) makes the wait give
 *                     up: the q/k rows it normalises are then written as NaN
 *                     (the attention core turns such rows into its empty
 *                     rows, so the layer output is wrong) and the context's
 *                     status word is set, which dt_ctx_check
 *                     (and any synchronous DT_MEM_HOST layer or model forward)
 *                     reports as DT_ERR_HIP. 0 makes every wait give up at
 *                     once (for testing that report).
 *   DT_OPT_SIDE_STREAM 1 (default): the model backward (dt_model_bwd) runs
 *                     its weight gradients' GEMMs and norm-weight column sums
 *                     on a second stream of the context, beside the chain of
 *                     input gradients on the caller's stream, ordered by
 *                     events; the call's work on both streams is enqueued
 *                     behind what the caller's stream holds, and the caller's
 *                     stream waits for all of it before the call returns
 *                     (results are the same bits as on one stream). Skipped
 *                     while the caller's stream is capturing a graph. 0: one
 *                     stream. (dt_attn_layer_bwd always runs on the caller's
 *                     stream.)
 * Returns DT_ERR_INVALID_ARG for an unknown option or value.
 */
#define DT_OPT_QKV_FUSED 1
#define DT_OPT_GEMM_TUNE 2
#define DT_OPT_BWD_DQ 3
#define DT_OPT_QKV_SPIN_LIMIT 4
#define DT_OPT_SIDE_STREAM 5
#define DT_QKV_GEMM 0
#define DT_QKV_FUSED 1
#define DT_QKV_AUTO 2
#define DT_BWD_DQ_RECOMPUTE 0
#define DT_BWD_DQ_FROM_DS 1
#define DT_BWD_DQ_AUTO 2
int dt_ctx_set_option(dt_ctx* ctx, int option, int value);

/*
 * Waits for the context's device to finish its work, then reports a fused
 * QKV wait that gave up since the last check (DT_OPT_QKV_SPIN_LIMIT) as
 * DT_ERR_HIP and clears it; DT_OK otherwise. No reference counterpart (the
 * reference's CPU path has no such wait).
 */
int dt_ctx_check(dt_ctx* ctx);

/*
 * Builds the RoPE sin/cos tables on the host in fp64, casts them to fp32 and
 * uploads them (replaces compute_rope_buffers, OlmoAttention.cpp:18-36).
 * dt_ctx_create already calls it with (DT_ROPE_THETA, DT_MAX_SEQ_LEN).
 */
int dt_rope_table_init(dt_ctx* ctx, float theta, int max_seq_len);

/*
 * Causal flash attention forward (replaces flash_attention_forward,
 * FlashAttention.h:15-21 / FlashAttention.cpp:24-182).
 *   q, k, v, o : [B, T, H, D]   (fp32 in DT_FP32_EXACT, bf16 bits in DT_BF16)
 *   m, l       : [B, T, H] fp32: m = row max of the scaled scores, l = sum of
 *                exp(s - m) (FlashAttention.cpp:162-163); either may be NULL.
 *   scale      : score scale (the reference passes 1/sqrt(D), OlmoAttention.cpp:91)
 *   causal     : 1 = causal (key k > query q masked, FlashAttention.cpp:102);
 *                0 = full attention.
 *   seq_lens   : NULL, or B lengths in [1, T]: keys at t >= seq_lens[b] are
 *                masked and rows t >= seq_lens[b] are written as the
 *                reference's empty row (O = 0, m = -inf, l = 0,
 *                FlashAttention.cpp:165-174).
 * Requires D == 128, 1 <= T <= 8192, B >= 1, 1 <= H.
 */
int dt_flash_attn_fwd(dt_ctx* ctx, const void* q, const void* k, const void* v, void* o, float* m, float* l,
                      int B, int T, int H, int D, float scale, int causal, const int32_t* seq_lens, int dtype,
                      int mem, void* stream);

/*
 * Flash attention backward (replaces flash_attention_backward,
 * FlashAttention.h:33-43 / FlashAttention.cpp:185-359).
 *   d_o, o, q, k, v : [B, T, H, D] (fp32 in DT_FP32_EXACT, bf16 bits in DT_BF16):
 *                     the output gradient, the forward's output and its inputs.
 *   m, l            : the forward's [B, T, H] fp32 statistics (dt_flash_attn_fwd).
 *   d_q, d_k, d_v   : [B, T, H, D] results, in the same element type.
 * P = exp(scale q.k - m) / l and dS = P (dP - rowsum(O * dO)) scale, as the
 * reference; every gradient row is written by one workgroup (no atomics), so
 * the results are deterministic. Full sequences only (no seq_lens).
 * Requires D == 128, 1 <= T <= 8192. Uses a context workspace of 8*B*T*H bytes.
 */
int dt_flash_attn_bwd(dt_ctx* ctx, const void* d_o, const void* o, const float* m, const float* l, const void* q,
                      const void* k, const void* v, void* d_q, void* d_k, void* d_v, int B, int T, int H, int D,
                      float scale, int causal, int dtype, int mem, void* stream);

/*
 * dt_flash_attn_bwd without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory during the call (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same arguments as dt_flash_attn_bwd with mem = DT_MEM_DEVICE (device
 * pointers only, stream-ordered). It always takes the recompute path, so its
 * output is bit-identical to dt_flash_attn_bwd's on a context with
 * DT_OPT_BWD_DQ = DT_BWD_DQ_RECOMPUTE. With the default DT_BWD_DQ_AUTO,
 * dt_flash_attn_bwd takes the dS path above one 128-row block per CU and pass
 * (e.g. B*H = 16, T = 4096): dK and dV are then still bit-identical, and dQ
 * agrees within the mode's tolerance (a different summation order). The backward's row statistics go to a fixed device array of 8 MiB
 * per GPU, set up by dt_ctx_create and held until the process ends, so
 * B*T*H must be at most 1048576 (DT_ERR_UNSUPPORTED above that). Every call
 * on one GPU shares that array: calls that overlap in time on one GPU (on
 * different streams or host threads) race and must be ordered by the caller.
 */
int dt_flash_attn_bwd_noalloc(dt_ctx* ctx, const void* d_o, const void* o, const float* m, const float* l,
                              const void* q, const void* k, const void* v, void* d_q, void* d_k, void* d_v, int B,
                              int T, int H, int D, float scale, int causal, int dtype, void* stream);

/*
 * Fused q/k RMSNorm + RoPE (replaces RMSNorm::forward for q_norm/k_norm,
 * RMSNorm.cpp:15-22, plus apply_rope, OlmoAttention.cpp:111-146, as called at
 * OlmoAttention.cpp:70,76,87-88).
 *   q_in, k_in   : fp32 rows of the q and k projections, [B*T] rows of d_model
 *                  = H*D features, with row strides ld_in (elements).
 *   q_norm_w, k_norm_w : [d_model] fp32 norm weights.
 *   q_out, k_out : [B*T] rows with stride ld_out, in out_dtype (DT_FP32_EXACT
 *                  -> fp32, DT_BF16 -> bf16 bits); may alias q_in/k_in when
 *                  the element types match.
 *   q_rms, k_rms : [B*T] fp32 (the norms' saved rms), or NULL.
 * The norm spans all d_model features (not per head); position of row
 * b*T + t is t. Requires D == 128, T <= the RoPE table length.
 */
int dt_qk_norm_rope_fwd(dt_ctx* ctx, const float* q_in, const float* k_in, const float* q_norm_w,
                        const float* k_norm_w, void* q_out, void* k_out, float* q_rms, float* k_rms, int B, int T,
                        int H, int D, int ld_in, int ld_out, int out_dtype, int mem, void* stream);

/*
 * Attention layer (replaces class OlmoAttention, OlmoAttention.h:10-42).
 * dt_attn_layer_create copies the weights (fp32, [out][in] like torch Linear,
 * y = x W^T) to the device; with mem == DT_MEM_HOST they are host pointers.
 * dt_attn_layer_load reads the reference's per-layer .npy files
 * "{folder}/model.layers.{index}.self_attn.{q,k,v,o}_proj.weight.npy" and
 * "...{q,k}_norm.weight.npy" (the OlmoAttention(folder, index) constructor,
 * OlmoAttention.cpp:39-53).
 */
int dt_attn_layer_create(dt_ctx* ctx, const float* wq, const float* wk, const float* wv, const float* wo,
                         const float* q_norm_w, const float* k_norm_w, int d_model, int n_heads, int mem,
                         dt_attn_layer** out);
int dt_attn_layer_load(dt_ctx* ctx, const char* folder, unsigned index, dt_attn_layer** out);
int dt_attn_layer_destroy(dt_attn_layer* layer);

/*
 * OlmoAttention::forward (OlmoAttention.cpp:56-108): x [B, T, d_model] fp32 ->
 * out [B, T, d_model] fp32. dtype selects the attention-core mode and the
 * projection GEMM precision (DT_FP32_EXACT: fp32 GEMMs; DT_BF16: bf16 GEMM
 * inputs with fp32 accumulation). seq_lens as for dt_flash_attn_fwd.
 * save_for_backward = 1 keeps what the reference saves for backward
 * (OlmoAttention.h:28-38: the input, the pre-norm projections and rms, the
 * rotated q/k, v, the attention output and its m/l) in layer-owned device
 * buffers; it requires seq_lens == NULL. With 0 nothing is kept (prefill).
 */
int dt_attn_layer_fwd(dt_attn_layer* layer, const float* x, float* out, int B, int T, const int32_t* seq_lens,
                      int dtype, int mem, int save_for_backward, void* stream);

/*
 * OlmoAttention::backward (OlmoAttention.cpp:193-312): d_out [B, T, d_model]
 * fp32 -> d_x [B, T, d_model] fp32, for the last forward with
 * save_for_backward = 1 (same B and T; its dtype is used). Accumulates (+=)
 * the gradients of Wq, Wk, Wv, Wo and the two norm weights in the layer, as
 * the reference's param<2>::grad (beta = 1 at OlmoAttention.cpp:207-211,
 * 257-277; RMSNorm.cpp:31).
 */
int dt_attn_layer_bwd(dt_attn_layer* layer, const float* d_out, float* d_x, int B, int T, int mem, void* stream);

/* OlmoAttention::step (OlmoAttention.cpp:314-321): w -= lr * grad for all six parameters. */
int dt_attn_layer_step(dt_attn_layer* layer, float lr, void* stream);

/* OlmoAttention::zero_grad (OlmoAttention.cpp:323-330). */
int dt_attn_layer_zero_grad(dt_attn_layer* layer, void* stream);

/*
 * Copies of the layer's parameters / accumulated gradients ([d_model][d_model]
 * for the four projections, [d_model] for the norm weights; any pointer may be
 * NULL to skip it). No counterpart function in the reference, where they are
 * the param<2> members w and grad (param.h:5-15).
 */
int dt_attn_layer_get_weights(dt_attn_layer* layer, float* wq, float* wk, float* wv, float* wo, float* q_norm_w,
                              float* k_norm_w, int mem, void* stream);
int dt_attn_layer_get_grads(dt_attn_layer* layer, float* d_wq, float* d_wk, float* d_wv, float* d_wo,
                            float* d_q_norm_w, float* d_k_norm_w, int mem, void* stream);

/*
 * OLMo-2 model (replaces class OlmoModel, OlmoModel.h:14-34, with its OlmoBlock,
 * OlmoMlp, RMSNorm and OlmoLmHead members). Parameters are named by the
 * reference's .npy file stems without the extension: "model.embed_tokens.weight",
 * "model.layers.{i}.self_attn.{q,k,v,o}_proj.weight",
 * "model.layers.{i}.self_attn.{q,k}_norm.weight",
 * "model.layers.{i}.post_attention_layernorm.weight",
 * "model.layers.{i}.mlp.{gate,up,down}_proj.weight",
 * "model.layers.{i}.post_feedforward_layernorm.weight", "model.norm.weight",
 * "lm_head.weight" (shapes [out][in] as in the files).
 *
 * dt_model_create makes a zero-initialised model of the given sizes (d_model =
 * n_heads * 128); dt_model_set_param / dt_model_get_param copy one parameter
 * (or, with grad = 1, its accumulated gradient) in or out. dt_model_load is
 * the OlmoModel(folder) constructor (OlmoModel.cpp:12-23): it reads every
 * "{folder}/{name}.npy" for n_layers blocks (the reference's n_layers = 16,
 * model_config.h:7). The sizes come from the embedding ([vocab][d_model]) and
 * the first up_proj ([hidden][d_model]); every file's header (float32, C
 * order, complete data) and shape is checked before ctx is used or anything is
 * allocated, so a Git-LFS pointer, a wrong dtype or shape or a truncated file
 * is reported (DT_ERR_IO) without touching the device.
 */
typedef struct dt_model dt_model;
int dt_model_create(dt_ctx* ctx, int n_layers, int d_model, int n_heads, int hidden, int vocab, dt_model** out);
int dt_model_load(dt_ctx* ctx, const char* folder, int n_layers, dt_model** out);
int dt_model_destroy(dt_model* model);
int dt_model_set_param(dt_model* model, const char* name, const float* data, int64_t count, int mem);
int dt_model_get_param(dt_model* model, const char* name, float* out, int64_t count, int grad, int mem,
                       void* stream);

/*
 * OlmoModel::forward (OlmoModel.cpp:25-48): tokens [B, T] (a host array, like
 * seq_lens; every id in [0, vocab)) -> logits [B, T, vocab] fp32. dtype selects
 * the attention-core mode and the GEMM precision as for dt_attn_layer_fwd.
 * save_for_backward = 1 keeps each block's state for dt_model_bwd.
 */
int dt_model_fwd(dt_model* model, const int32_t* tokens, int B, int T, float* logits, int dtype, int mem,
                 int save_for_backward, void* stream);

/* OlmoModel::backward (OlmoModel.cpp:50-67) for the last saved forward: d_logits
 * [B, T, vocab] fp32; accumulates (+=) every parameter's gradient. */
int dt_model_bwd(dt_model* model, const float* d_logits, int mem, void* stream);

/* OlmoModel::step / zero_grad (OlmoModel.cpp:69-83): w -= lr * grad; grads = 0. */
int dt_model_step(dt_model* model, float lr, void* stream);
int dt_model_zero_grad(dt_model* model, void* stream);

/*
 * ce_loss (CrossEntropyLoss.cpp:8-43): the mean next-token cross entropy of
 * logits [B, T, V] against tokens[b][s+1] (a host array), skipping targets equal
 * to ignore_index; *loss is written to host memory. d_logits (nullable)
 * receives the gradient main.cpp:62-80 builds from it: (softmax - onehot) /
 * count at the positions with a target, 0 elsewhere. d_logits may be the same
 * buffer as logits (main.cpp turns probs into the gradient in place). When no
 * position has a target (T == 1, or every next token is ignore_index) the
 * reference divides 0 by 0 (CrossEntropyLoss.cpp:40, main.cpp:88): *loss and
 * every d_logits element are NaN here too.
 */
int dt_ce_loss(dt_ctx* ctx, const float* logits, const int32_t* tokens, int B, int T, int V, int ignore_index,
               float* loss, float* d_logits, int mem, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DIRKTENSOR_AMD_H */
