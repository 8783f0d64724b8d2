// Attention-core backward that allocates nothing: dt_flash_attn_bwd_noalloc.
//
// dt_flash_attn_bwd keeps the backward's row statistics (delta = rowsum(O * dO) and lse2 =
// m log2 e + log2 l, 2 x [B][H][T] fp32) in a context buffer that grows with hipMalloc. Callers that
// cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc) use
// this variant instead: the statistics live in the file-scope device array `scratch` below, one copy per
// GPU, held until the process ends. The array's host-side name is not a device address, so its address
// on each device is taken once with hipGetSymbolAddress when a context is created on that device
// (noalloc_setup, called by dt_ctx_create with the device current) and only that pointer is used.
//
// Every call on one GPU shares that GPU's array, and it keeps the last call's contents: calls that overlap
// in time on one GPU (different streams, or different host threads) race on it. The prep kernel writes
// every delta/lse2 entry the two gradient kernels read (rows past T come from the bounded buffer loads as
// zeros, not from memory), so nothing needs clearing between calls.

#include <atomic>
#include <cmath>

#include "dt_internal.h"

namespace dt {
namespace {

constexpr int64_t kScratchRows = int64_t(1) << 20;      // B*T*H rows at most (e.g. B = 8, T = 8192, H = 16)
constexpr int64_t kScratchFloats = 2 * kScratchRows;    // delta and lse2: 8 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchFloats];

std::atomic<float*> g_scratch[kMaxDevices];  // per device: the address of `scratch` there

}  // namespace

int noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return set_error(DT_ERR_UNSUPPORTED, "device %d out of range", device);
    if (g_scratch[device].load(std::memory_order_acquire)) return DT_OK;
    int cur = -1;
    DT_HIP_TRY(hipGetDevice(&cur));
    if (cur != device) return set_error(DT_ERR_INVALID_ARG, "noalloc_setup: device %d is not current (%d)", device, cur);
    void* p = nullptr;
    DT_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(DT_ERR_HIP, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch[device].store(static_cast<float*>(p), std::memory_order_release);
    return DT_OK;
}

int64_t noalloc_max_rows() { return kScratchRows; }

}  // namespace dt

using namespace dt;

extern "C" int dt_flash_attn_bwd_noalloc(dt_ctx* ctx, const void* d_o, const void* o, const float* m, const float* l,
                                         const void* q, const void* k, const void* v, void* d_q, void* d_k, void* d_v,
                                         int B, int T, int H, int D, float scale, int causal, int dtype, void* stream) {
    clear_error();
    if (!d_o || !o || !m || !l || !q || !k || !v || !d_q || !d_k || !d_v)
        return set_error(DT_ERR_INVALID_ARG, "all tensor pointers must be non-NULL");
    if (D != DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "head_dim D=%d, kernels are built for D=%d", D, DT_HEAD_DIM);
    if (B < 1 || H < 1 || T < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d, H=%d must be >= 1", B, T, H);
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if (H > 65535 || B > 65535) return set_error(DT_ERR_UNSUPPORTED, "B=%d or H=%d exceeds grid limits", B, H);
    if ((int64_t)B * T * H > kScratchRows)
        return set_error(DT_ERR_UNSUPPORTED,
                         "B*T*H = %lld rows exceeds the no-alloc scratch limit of %lld rows (8 MiB of statistics); "
                         "use dt_flash_attn_bwd",
                         (long long)B * T * H, (long long)kScratchRows);
    if (dtype != DT_FP32_EXACT && dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (!(scale > 0.0f) || !std::isfinite(scale)) return set_error(DT_ERR_INVALID_ARG, "scale %g must be finite and > 0", scale);
    if (causal != 0 && causal != 1) return set_error(DT_ERR_INVALID_ARG, "causal must be 0 or 1");
    if (!aligned16(d_o) || !aligned16(o) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(d_q) ||
        !aligned16(d_k) || !aligned16(d_v))
        return set_error(DT_ERR_INVALID_ARG, "device tensors must be 16-byte aligned");
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return set_error(DT_ERR_UNSUPPORTED, "device out of range");
    float* stats = g_scratch[ctx->device].load(std::memory_order_acquire);
    if (!stats) return set_error(DT_ERR_INVALID_ARG, "the context's device has no no-alloc scratch address");
    DT_TRY(check_device_binding(ctx));

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int ld = H * D;
    const int64_t nst = (int64_t)B * T * H;
    const FlashBwdArgs ba{q, k, v, o, d_o, m, l, d_q, d_k, d_v, stats, stats + nst, B, T, H, ld, ld, ld, scale, causal};
    return dtype == DT_BF16 ? launch_flash_bwd_bf16(ba, s) : launch_flash_bwd_f32(ba, s);
}
