// Internal declarations shared by the HIP kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

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
};

int launch_flash_fwd_f32(const FlashArgs& a, const SeqLens* lens, hipStream_t stream);
int launch_flash_fwd_bf16(const FlashArgs& a, const SeqLens* lens, hipStream_t stream);

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
};
int launch_flash_bwd_prep(const FlashBwdArgs& a, int bf16, hipStream_t stream);  // fills delta and lse2
int launch_flash_bwd_bf16(const FlashBwdArgs& a, hipStream_t stream);
int launch_flash_bwd_f32(const FlashBwdArgs& a, hipStream_t stream);

struct NormRopeArgs {
    const float* q_in;
    const float* k_in;
    const float* v_in;  // nullable: when set, V rows are converted into v_out
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
int launch_qk_norm_rope(const NormRopeArgs& a, int out_bf16, hipStream_t stream);

// Backward of the fused q/k RMSNorm + RoPE (OlmoAttention.cpp:234-244): dq/dk rows are rewritten in place
// from d(rope output) to d(pre-norm projection); the norm-weight gradients are accumulated (+=).
struct NormRopeBwdArgs {
    void* dq;  // [rows] rows of stride ld_d, fp32 or bf16 (in place)
    void* dk;
    const float* q_x;  // saved pre-norm projections, stride ld_x
    const float* k_x;
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
int launch_qk_norm_rope_bwd(const NormRopeBwdArgs& a, int bf16, float* grad_q_w, float* grad_k_w, hipStream_t stream);
int launch_sgd(float* w, const float* g, float lr, int64_t n, hipStream_t stream);  // w -= lr * g
int launch_fill_zero(float* p, int64_t n, hipStream_t stream);
int launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream);

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
};
