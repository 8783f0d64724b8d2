// Internal declarations shared by the HIP kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "dirktensor_amd.h"  // include/, on the include path

namespace dt {

// ---- error reporting (thread-local, read back through dt_last_error) ----
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define DT_HIP_TRY(expr)                                                                          \
    do {                                                                                          \
        hipError_t dt_e_ = (expr);                                                                \
        if (dt_e_ != hipSuccess)                                                                  \
            return ::dt::set_error(DT_ERR_HIP, "%s failed: %s (%s:%d)", #expr,                    \
                                   hipGetErrorString(dt_e_), __FILE__, __LINE__);                 \
    } while (0)

#define DT_TRY(expr)                  \
    do {                              \
        int dt_rc_ = (expr);          \
        if (dt_rc_ != DT_OK) return dt_rc_; \
    } while (0)

// ---- a growable device buffer owned by a context or layer ----
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    int ensure(size_t need);  // grows (hipFree + hipMalloc) when too small
    void release();
};

// Per-sequence lengths passed by value in kernel arguments (no device copy).
constexpr int kMaxRaggedBatch = 256;
struct SeqLens {
    int32_t len[kMaxRaggedBatch];
};

// Arguments of one attention-core launch. Row strides are in elements.
struct FlashArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* m;  // nullable
    float* l;  // nullable
    int B, T, H;
    int ldq, ldk, ldv, ldo;  // row (token) strides, elements
    float scale;
    int causal;
    int ragged;  // 1 when seq_lens are used
    // workspace of items split across workgroups (the context's; see flash_items.h): partial results and
    // one counter per split item, the counters zero between launches
    float* split_ws;
    int* split_cnt;
    int split_slots;  // capacity of the workspace in split items (0: none, nothing is split)
};

// one workgroup per CU of the current device, at most n_items (0x7fffffff: the CU count)
int persistent_grid(int64_t n_items, int* grid);
int launch_flash_fwd_f32(const FlashArgs& a, const SeqLens* lens, hipStream_t stream);
int launch_flash_fwd_bf16(const FlashArgs& a, const SeqLens* lens, hipStream_t stream);
// split items a launch of the bf16 forward would use (the workspace capacity it needs, in items)
int flash_fwd_split_items(const FlashArgs& a, const SeqLens* lens, int* n_items);

// Arguments of one attention-core backward (FlashAttention.cpp:185-359). Row strides in elements.
struct FlashBwdArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* d_o;
    const float* m;  // forward statistics, [B][T][H]
    const float* l;
    void* d_q;
    void* d_k;
    void* d_v;
    float* delta;  // workspace [B][H][T]: rowsum(O * dO)
    float* lse2;   // workspace [B][H][T]: m log2(e) + log2(l), +inf for an empty row
    int B, T, H;
    int ld_qkv;  // row stride of q, k and v
    int ld_o;    // row stride of o and d_o
    int ld_grad; // row stride of d_q, d_k and d_v
    float scale;
    int causal;
    // workspace for dS (flash_bwd_ds_bytes); when set, the dK/dV pass stores dS there and dQ is computed as
    // dS K from it instead of recomputing S and dP. NULL: the recompute path.
    void* ds_ws = nullptr;
};
int launch_flash_bwd_prep(const FlashBwdArgs& a, int bf16, hipStream_t stream);  // fills delta and lse2
// dS workspace of the backward's dS path: per (batch, head) and 128-key block kb, one block per 64-query
// tile the keys can see (tiles 2*kb .. under causality, all otherwise), the tiles of one key block
// consecutive. A block holds 128 keys x 64 queries of dS (16 KB in bf16, 32 KB in fp32).
struct BwdDsLayout {
    int nqt, nkb, causal;
    __host__ __device__ BwdDsLayout(int T, int causal_) : nqt((T + 63) / 64), nkb((T + 127) / 128), causal(causal_) {}
    __host__ __device__ int first_tile(int kb) const { return causal ? 2 * kb : 0; }
    __host__ __device__ int64_t block_offset(int kb) const {  // blocks before key block kb's, in one (batch, head)
        return (int64_t)kb * nqt - (causal ? (int64_t)kb * (kb - 1) : 0);
    }
    __host__ __device__ int64_t per_head() const { return block_offset(nkb); }
};
// bytes of the dS workspace of one backward call; elem_bytes 2 (bf16 mode) or 4 (fp32 exact mode)
inline size_t flash_bwd_ds_bytes(int B, int H, int T, int causal, int elem_bytes) {
    return (size_t)B * H * (size_t)BwdDsLayout(T, causal).per_head() * (size_t)(128 * 64 * elem_bytes);
}
int launch_flash_bwd_bf16(const FlashBwdArgs& a, hipStream_t stream);
int launch_flash_bwd_f32(const FlashBwdArgs& a, hipStream_t stream);

struct NormRopeArgs {
    const void* q_in;  // fp32, or bf16 when launched with in_bf16
    const void* k_in;
    const void* v_in;  // nullable: when set, V rows are converted into v_out
    const float* q_w;
    const float* k_w;
    void* q_out;
    void* k_out;
    void* v_out;
    float* q_rms;  // nullable
    float* k_rms;  // nullable
    const float* rope_cos;  // [rope_len][D/2]
    const float* rope_sin;  // [rope_len][D/2]
    int rows, T, H;
    int ld_in, ld_out;
    float eps;
};
int launch_qk_norm_rope(const NormRopeArgs& a, int out_bf16, hipStream_t stream, int in_bf16 = 0);

// Fused x [Wq;Wk;Wv]^T -> rope(norm(q)) | rope(norm(k)) | v (qkv_proj.hip). x, w, out and pre share one
// element type: bf16, or fp32 when launched with f32.
struct QkvArgs {
    const void* x;  // [rows][ldx]: the layer input rows (d_model = H*128 used)
    const void* w;  // [3*d_model][d_model]: Wq, Wk, Wv rows
    const float* q_w;  // q_norm / k_norm weights [d_model]
    const float* k_w;
    void* out;    // [rows][ld_out]: rotated, normalised q | k, then v
    void* pre;    // nullable: [rows][ld_pre], the pre-norm q | k (v columns untouched)
    float* rms;   // nullable: [2][rows], q then k
    const float* rope_cos;  // [>= T][64]
    const float* rope_sin;
    uint64_t* ss;      // workspace: per-row, per-head partial sums of squares, tagged with the epoch
    int64_t ss_bytes;  // its size (qkv_norm_rope_workspace)
    uint32_t epoch;    // nonzero, different from the previous launch's on the same workspace
    int rows, T, H;
    int ldx, ld_out, ld_pre;  // elements
    float eps;
    uint32_t* status = nullptr;  // set to kQkvWaitGaveUp when a wait for the other heads' sums gives up
    int spin_limit = 0;          // polls before such a wait gives up (0: every wait gives up at once)
};
// polls (coherent loads and s_sleep 1, about a second in all) before a wait of the fused kernel gives up
constexpr int kQkvSpinLimit = 1 << 20;
constexpr uint32_t kQkvWaitGaveUp = 1;
int qkv_norm_rope_workspace(int rows, int H, size_t* ss_bytes);
int launch_qkv_norm_rope(const QkvArgs& a, int f32, hipStream_t stream);
// the fused kernel's tiles for rows x (3 H heads) fit one round on this device's CUs
int qkv_fused_one_round(int rows, int H, bool* fits);

// Backward of the fused q/k RMSNorm + RoPE (OlmoAttention.cpp:234-244): dq/dk rows are rewritten in place
// from d(rope output) to d(pre-norm projection); the norm-weight gradients are accumulated (+=).
struct NormRopeBwdArgs {
    void* dq;  // [rows] rows of stride ld_d, fp32 or bf16 (in place)
    void* dk;
    const void* q_x;  // saved pre-norm projections, stride ld_x, in the dtype of dq / dk
    const void* k_x;
    const float* q_rms;  // saved rms, [rows]
    const float* k_rms;
    const float* q_w;
    const float* k_w;
    float* partial;  // workspace [2][norm_rope_bwd_blocks(rows)][H*128]
    const float* rope_cos;
    const float* rope_sin;
    int rows, T, H;
    int ld_d, ld_x;
};
int norm_rope_bwd_blocks(int rows);
// accumulate = false: the norm-weight gradients are overwritten (their buffers are logically zero)
int launch_qk_norm_rope_bwd(const NormRopeBwdArgs& a, int bf16, float* grad_q_w, float* grad_k_w, hipStream_t stream,
                            bool accumulate = true);
// out[c] += sum_b partial[b][c] (b = 0 .. nblk-1; out[c] = 0 + the sum when accumulate is false), deterministic
// order
// out[c] (+)= sum over the nblk partial rows of column c, in a fixed order; with out1, a second such sum over the
// nblk rows that follow, into out1, in the same launch
int launch_colsum(const float* partial, int nblk, int ncols, float* out, hipStream_t s, bool accumulate = true,
                  float* out1 = nullptr);
// w -= lr * g; w16 (nullable): the bf16 copy of w, refreshed in the same pass
int launch_sgd(float* w, const float* g, float lr, int64_t n, hipStream_t stream, uint16_t* w16 = nullptr);
// the same update of count short vectors (the norm weights) in one launch, one workgroup per vector
int launch_sgd_vecs(float* const* w, const float* const* g, const int* n, int count, float lr, hipStream_t stream);
int launch_fill_zero(float* p, int64_t n, hipStream_t stream);
int launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream);

// Row-major C[M][N] = op(A)[M][K] op(B)[K][N] + beta C: fp32 on rocBLAS, bf16 inputs with fp32 accumulation
// and output on hipBLASLt (rocBLAS when it has no algorithm for the shape); op = transpose when ta / tb is set.
int gemm_rm(dt_ctx* ctx, hipStream_t s, bool ta, bool tb, int M, int N, int K, const void* A, int lda,
            const void* B, int ldb, float beta, float* C, int ldc, bool bf16_in);
// the same with bf16 inputs and a bf16 output C (beta = 0; fp32 accumulation, one rounding at the end)
int gemm_rm_bf16(dt_ctx* ctx, hipStream_t s, bool ta, bool tb, int M, int N, int K, const void* A, int lda,
                 const void* B, int ldb, void* C, int ldc);
// .npy reader (v1-v3 headers, little-endian fp32, C order)
int read_npy_f32(const std::string& path, std::vector<float>& out, std::vector<size_t>& shape);
// the same checks (format, dtype, order, the data all present) and the shape, without reading the data
int read_npy_shape(const std::string& path, std::vector<size_t>& shape);
bool aligned16(const void* p);
// once per device, with it current (dt_ctx_create): looks up that device's address of the scratch array of
// dt_flash_attn_bwd_noalloc (noalloc.hip)
int noalloc_setup(int device);
int check_device_binding(dt_ctx* ctx);
// after the stream has been synchronised: DT_ERR_HIP (and clears the word) when a fused QKV wait gave up
int qkv_status_check(dt_ctx* ctx);

// The context's side stream: weight-gradient GEMMs run on it beside the backward's chain of input gradients,
// which never reads them. Created on first use (non-blocking, default priority; null when that fails or when s
// is being captured into a graph, and the caller then stays on s). GEMMs on it use their own BLAS handle and
// workspace.
hipStream_t side_stream(dt_ctx* ctx, hipStream_t s);
// Event slots of the context that order the two streams: a fork (side after main), and one per buffer the
// side stream's GEMMs read and the main stream later overwrites.
enum SideEvent { kEvFork = 0, kEvJoin, kEvDown, kEvGu, kEvO, kSideEvents };
// waiter waits for all that producer has enqueued so far (an event recorded in slot ev)
int stream_after(dt_ctx* ctx, hipStream_t waiter, hipStream_t producer, int ev);
// waiter waits for the last record of slot ev (a no-op if the slot was never recorded)
int stream_wait_slot(dt_ctx* ctx, hipStream_t waiter, int ev);
// records slot ev on producer
int stream_mark(dt_ctx* ctx, hipStream_t producer, int ev);

}  // namespace dt

// ---- opaque handles ----
struct dt_ctx {
    int device = 0;
    float* rope_cos = nullptr;  // device, [rope_len][64]
    float* rope_sin = nullptr;
    int rope_len = 0;
    float rope_theta = 0.0f;
    dt::DeviceBuffer stage[10];  // host-memory path staging
    dt::DeviceBuffer bwd_stats;  // attention-core backward: delta and lse2, 2 x [B][H][T] fp32
    void* blas = nullptr;        // rocblas_handle, created on first use
    void* lt = nullptr;          // hipBLASLt handle and per-shape plans (capi.hip), created on first use
    dt::DeviceBuffer lt_ws;      // hipBLASLt workspace (split-K partial sums)
    dt::DeviceBuffer fwd_split;  // attention forward: partial results of items split across workgroups
    dt::DeviceBuffer fwd_split_cnt;  // and their counters (zeroed when allocated; each launch leaves them zero)
    dt::DeviceBuffer qkv_ss;   // fused QKV projection: per-row, per-head sums of squares (zeroed when allocated)
    uint32_t qkv_epoch = 0;    // the tag of its last launch
    dt::DeviceBuffer qkv_status;  // its status word: nonzero once a wait gave up (zeroed when allocated and read)
    int qkv_spin = dt::kQkvSpinLimit;  // DT_OPT_QKV_SPIN_LIMIT
    int qkv_fused = DT_QKV_AUTO;  // DT_OPT_QKV_FUSED
    int gemm_tune = 1;            // DT_OPT_GEMM_TUNE
    int bwd_dq = DT_BWD_DQ_AUTO;  // DT_OPT_BWD_DQ
    dt::DeviceBuffer bwd_ds;      // bf16 attention backward: dS of one call (the dS path)
    void* side = nullptr;         // hipStream_t: the side stream (dt::side_stream)
    void* blas_side = nullptr;    // rocblas_handle for GEMMs on it
    dt::DeviceBuffer lt_ws_side;  // hipBLASLt workspace of GEMMs on it
    void* ev[dt::kSideEvents] = {};  // hipEvent_t slots (dt::SideEvent)
    int side_off = 0;             // DT_OPT_SIDE_STREAM = 0: everything on the caller's stream
};

// OlmoAttention on the device (OlmoAttention.h:10-42): weights, forward state kept for backward, gradients.
struct dt_attn_layer {
    dt_ctx* ctx = nullptr;
    int d_model = 0, n_heads = 0;
    float* w_qkv = nullptr;      // [3*d_model][d_model] fp32 (q rows, k rows, v rows)
    float* w_o = nullptr;        // [d_model][d_model]
    uint16_t* w_qkv16 = nullptr; // bf16 copies, made on first bf16 forward
    uint16_t* w_o16 = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    dt::DeviceBuffer qkv_pre, qkv16, attn, x16;  // qkv_pre: pre-norm Q|K|V, fp32 or bf16 by mode
    bool w16_stale = true;  // the bf16 copies lag the fp32 weights (before the first bf16 forward, after step)
    // zero_grad was called and the gradient buffers have not been cleared: they read as zero. The next backward
    // writes them instead of adding to them; anything else that reads them clears them first.
    bool grad_zero_pending = false;
    // forward state kept for backward (OlmoAttention.h:28-38) when save_for_backward is set
    dt::DeviceBuffer x32;   // the input rows (fp32)
    dt::DeviceBuffer att32; // fp32 mode: q_rope | k_rope | v, [rows][3*d_model]
    dt::DeviceBuffer rms;   // q and k rms, 2 x [rows]
    dt::DeviceBuffer stats; // attention m and l, 2 x [rows][H]
    int saved_B = 0, saved_T = 0, saved_dtype = -1;  // saved_T == 0: nothing saved
    // backward workspaces and the accumulated gradients (param<2>::grad, param.h:5-15)
    dt::DeviceBuffer d_attn32, d16, d_qkv, partial;
    float* g_qkv = nullptr;  // [3*d_model][d_model]
    float* g_o = nullptr;    // [d_model][d_model]
    float* g_qn = nullptr;   // [d_model]
    float* g_kn = nullptr;
};

// dt_attn_layer_fwd with one more input: x16_ready (bf16 mode, device memory) says that L->x16 already holds
// the B*T*d_model rows of x rounded to bf16 (the model's previous block writes them there with its last norm),
// so the layer does not round x itself
int attn_layer_fwd(dt_attn_layer* L, const float* x, float* out, int B, int T, const int32_t* seq_lens, int dtype,
                   int mem, int save_for_backward, void* stream, bool x16_ready);
// dt_attn_layer_bwd (device memory) with two more inputs: d_out16 (bf16 mode, nullable) holds d_out rounded to
// bf16 (the model's norm backward writes it beside d_out), so the layer does not round d_out itself; side (nullable)
// is the context's side stream for the weight-gradient GEMMs, which the caller joins back into its stream (slot
// kEvO is recorded on it after the last read of d_out and d_out16)
int attn_layer_bwd_dev(dt_attn_layer* L, const float* d_out, const uint16_t* d_out16, float* d_x, int B, int T,
                       void* stream, hipStream_t side);
// zero-initialised attention layer (weights set afterwards), and its gradient buffers (allocated zeroed)
// dt_attn_layer_step's updates of Wqkv and Wo (and their bf16 copies), without the two norm weights
int attn_layer_step_mats(dt_attn_layer* L, float lr, hipStream_t s);
int attn_layer_alloc(dt_ctx* ctx, int d_model, int n_heads, dt_attn_layer** out);
int attn_layer_ensure_grads(dt_attn_layer* L, hipStream_t s);  // all four buffers, or none on failure
bool attn_layer_grads_complete(const dt_attn_layer* L);
void attn_layer_free_grads(dt_attn_layer* L);
// clears the gradient buffers when a zero_grad is pending (they are then zero in memory as well)
int attn_layer_settle_grads(dt_attn_layer* L, hipStream_t s);

namespace dt {
// model kernels (model_kernels.hip)
int launch_embed_gather(const int32_t* tok, const float* E, float* x, int rows, int dm, hipStream_t s);
int launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t s);  // n % 4 == 0
int launch_rmsnorm_rows(const float* a, const float* w, const float* res, float* out, uint16_t* out16, float* y_save,
                        float* rms_save, int rows, int dm, float eps, hipStream_t s);
int launch_swiglu(const void* gu, void* act, int rows, int hid, int bf16, hipStream_t s);
int launch_ce_loss(const float* logits, const int32_t* target, float* term, float* grad, float* loss, int rows, int V,
                   int count, hipStream_t s);
int rmsnorm_bwd_blocks(int rows);
// dx16 (nullable): dx rounded to bf16 as well; dx may then be NULL (only the bf16 rows are written)
int launch_rmsnorm_bwd(const float* dy, const float* y, const float* rms, const float* w, const float* dx_add,
                       float* dx, float* partial, float* grad_w, int rows, int dm, hipStream_t s,
                       bool accumulate = true, uint16_t* dx16 = nullptr);
int launch_swiglu_bwd(const float* d_act, const void* gu, void* d_gu, int rows, int hid, int bf16, hipStream_t s);
int launch_embed_bwd(const float* dx, const int32_t* uniq, const int32_t* start, const int32_t* pos, int n_uniq,
                     float* g_embed, int dm, hipStream_t s);
// for each listed row r (rows on the device, each < the table's row count): w[r] -= lr * g[r], or, with
// zero_rows, g[r] = 0
int launch_embed_rows(float* w, float* g, const int32_t* rows, int n_rows, int dm, float lr, bool zero_rows,
                      hipStream_t s);
}  // namespace dt
