// C ABI of the attention path: argument validation, context, host-memory
// staging and the OlmoAttention layer orchestration (projections on rocBLAS,
// norm + RoPE and the attention core on this library's kernels).
//
// Every entry point validates all arguments before its first HIP call, so an
// invalid call returns a status without touching the device (the reference's
// shape checks are compiled-out asserts, CMakeLists.txt:68, and T > 8192 is
// undefined behaviour there, OlmoAttention.cpp:129).

#include "flash_items.h"

#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <array>
#include <map>
#include <mutex>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "dt_internal.h"

namespace dt {

static thread_local std::string t_err;

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

void clear_error() { t_err.clear(); }

int DeviceBuffer::ensure(size_t need) {
    if (need <= bytes) return DT_OK;
    if (ptr) {
        DT_HIP_TRY(hipFree(ptr));
        ptr = nullptr;
        bytes = 0;
    }
    size_t sz = (need + 255) & ~size_t(255);
    DT_HIP_TRY(hipMalloc(&ptr, sz));
    bytes = sz;
    return DT_OK;
}

void DeviceBuffer::release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_device_binding(dt_ctx* ctx) {
    DT_HIP_TRY(hipSetDevice(ctx->device));
    return DT_OK;
}

static int rope_upload(dt_ctx* ctx, float theta, int max_seq_len) {
    // compute_rope_buffers, OlmoAttention.cpp:18-31: fp64 inv_freq and angles, fp32 tables.
    const int half = DT_HEAD_DIM / 2;
    std::vector<float> cs((size_t)max_seq_len * half), sn((size_t)max_seq_len * half);
    std::vector<double> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0 / std::pow((double)theta, (double)(2 * i) / (double)DT_HEAD_DIM);
    for (int p = 0; p < max_seq_len; ++p)
        for (int i = 0; i < half; ++i) {
            const double ang = (double)p * inv[i];
            cs[(size_t)p * half + i] = (float)std::cos(ang);
            sn[(size_t)p * half + i] = (float)std::sin(ang);
        }
    if (ctx->rope_cos) DT_HIP_TRY(hipFree(ctx->rope_cos));
    if (ctx->rope_sin) DT_HIP_TRY(hipFree(ctx->rope_sin));
    ctx->rope_cos = ctx->rope_sin = nullptr;
    ctx->rope_len = 0;
    DT_HIP_TRY(hipMalloc(&ctx->rope_cos, cs.size() * sizeof(float)));
    DT_HIP_TRY(hipMalloc(&ctx->rope_sin, sn.size() * sizeof(float)));
    DT_HIP_TRY(hipMemcpy(ctx->rope_cos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
    DT_HIP_TRY(hipMemcpy(ctx->rope_sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice));
    ctx->rope_len = max_seq_len;
    ctx->rope_theta = theta;
    return DT_OK;
}

static int validate_seq_lens(const int32_t* seq_lens, int B, int T) {
    if (!seq_lens) return DT_OK;
    if (B > kMaxRaggedBatch)
        return set_error(DT_ERR_UNSUPPORTED, "seq_lens given with B=%d > %d", B, kMaxRaggedBatch);
    for (int b = 0; b < B; ++b)
        if (seq_lens[b] < 1 || seq_lens[b] > T)
            return set_error(DT_ERR_INVALID_ARG, "seq_lens[%d]=%d outside [1, T=%d]", b, seq_lens[b], T);
    return DT_OK;
}

static int run_flash(dt_ctx* ctx, const FlashArgs& fa_in, const int32_t* seq_lens, int dtype, hipStream_t s) {
    SeqLens sl;
    const SeqLens* lp = nullptr;
    if (seq_lens) {
        std::memcpy(sl.len, seq_lens, sizeof(int32_t) * fa_in.B);
        lp = &sl;
    }
    FlashArgs fa = fa_in;
    fa.split_ws = nullptr;
    fa.split_cnt = nullptr;
    fa.split_slots = 0;
    if (dtype != DT_BF16) return launch_flash_fwd_f32(fa, lp, s);
    // the workspace for items split across workgroups, grown to what this launch uses (counters start zero)
    int items = 0;
    DT_TRY(flash_fwd_split_items(fa, lp, &items));
    if (items > 0) {
        const size_t cnt_bytes = sizeof(int) * (size_t)items;
        if (ctx->fwd_split_cnt.bytes < cnt_bytes) {
            DT_TRY(ctx->fwd_split_cnt.ensure(cnt_bytes));
            DT_HIP_TRY(hipMemsetAsync(ctx->fwd_split_cnt.ptr, 0, ctx->fwd_split_cnt.bytes, s));
        }
        DT_TRY(ctx->fwd_split.ensure(sizeof(float) * (size_t)items * kMaxParts * kPartialFloats));
        fa.split_ws = static_cast<float*>(ctx->fwd_split.ptr);
        fa.split_cnt = static_cast<int*>(ctx->fwd_split_cnt.ptr);
        fa.split_slots = items;
    }
    return launch_flash_fwd_bf16(fa, lp, s);
}

// The fused projection + norm + RoPE launch with the context's workspace (zeroed when allocated, so no
// entry carries a live epoch) and the next epoch (never 0).
static int run_qkv_fused(dt_ctx* ctx, QkvArgs qa, int f32, hipStream_t s) {
    size_t ss_bytes = 0;
    DT_TRY(qkv_norm_rope_workspace(qa.rows, qa.H, &ss_bytes));
    if (ctx->qkv_ss.bytes < ss_bytes) {
        DT_TRY(ctx->qkv_ss.ensure(ss_bytes));
        DT_HIP_TRY(hipMemsetAsync(ctx->qkv_ss.ptr, 0, ctx->qkv_ss.bytes, s));
    }
    if (!ctx->qkv_status.ptr) {
        DT_TRY(ctx->qkv_status.ensure(256));
        DT_HIP_TRY(hipMemsetAsync(ctx->qkv_status.ptr, 0, ctx->qkv_status.bytes, s));
    }
    if (++ctx->qkv_epoch == 0) ctx->qkv_epoch = 1;
    qa.ss = static_cast<uint64_t*>(ctx->qkv_ss.ptr);
    qa.ss_bytes = (int64_t)ctx->qkv_ss.bytes;
    qa.status = static_cast<uint32_t*>(ctx->qkv_status.ptr);
    qa.epoch = ctx->qkv_epoch;
    qa.spin_limit = ctx->qkv_spin;
    return launch_qkv_norm_rope(qa, f32, s);
}

int qkv_status_check(dt_ctx* ctx) {
    if (!ctx->qkv_status.ptr) return DT_OK;
    uint32_t word = 0;
    DT_HIP_TRY(hipMemcpy(&word, ctx->qkv_status.ptr, sizeof(word), hipMemcpyDeviceToHost));
    if (word == 0) return DT_OK;
    DT_HIP_TRY(hipMemset(ctx->qkv_status.ptr, 0, sizeof(word)));
    return set_error(DT_ERR_HIP,
                     "fused QKV projection: a workgroup's wait for the other heads' row sums gave up (a workgroup "
                     "was kept off its CU); the q/k rows it normalises were written as NaN and the outputs built on them "
                     "are wrong");
}

// ---------------- rocBLAS helpers ----------------
static const char* blas_status_str(rocblas_status st) { return rocblas_status_to_string(st); }

// the rocBLAS handle of stream s: the side stream has its own, so that no handle-owned workspace is shared by
// GEMMs that run at the same time
static int ensure_blas(dt_ctx* ctx, hipStream_t s, rocblas_handle* out) {
    void*& slot = (ctx->side && s == static_cast<hipStream_t>(ctx->side)) ? ctx->blas_side : ctx->blas;
    if (!slot) {
        rocblas_handle h = nullptr;
        rocblas_status st = rocblas_create_handle(&h);
        if (st != rocblas_status_success)
            return set_error(DT_ERR_BLAS, "rocblas_create_handle: %s", blas_status_str(st));
        slot = h;
    }
    *out = static_cast<rocblas_handle>(slot);
    return rocblas_set_stream(*out, s) == rocblas_status_success ? DT_OK
                                                                  : set_error(DT_ERR_BLAS, "rocblas_set_stream failed");
}

// ---------------- the side stream ----------------
hipStream_t side_stream(dt_ctx* ctx, hipStream_t s) {
    if (ctx->side_off) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (cs != hipStreamCaptureStatusNone) return nullptr;
    if (!ctx->side) {
        hipStream_t st = nullptr;
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        for (int i = 0; i < kSideEvents; ++i) {
            hipEvent_t e = nullptr;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                for (int j = 0; j < i; ++j) (void)hipEventDestroy(static_cast<hipEvent_t>(ctx->ev[j]));
                for (int j = 0; j < i; ++j) ctx->ev[j] = nullptr;
                (void)hipStreamDestroy(st);
                return nullptr;
            }
            ctx->ev[i] = e;
        }
        ctx->side = st;
    }
    return static_cast<hipStream_t>(ctx->side);
}

int stream_mark(dt_ctx* ctx, hipStream_t producer, int ev) {
    DT_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ctx->ev[ev]), producer));
    return DT_OK;
}

int stream_wait_slot(dt_ctx* ctx, hipStream_t waiter, int ev) {
    DT_HIP_TRY(hipStreamWaitEvent(waiter, static_cast<hipEvent_t>(ctx->ev[ev]), 0));
    return DT_OK;
}

int stream_after(dt_ctx* ctx, hipStream_t waiter, hipStream_t producer, int ev) {
    DT_TRY(stream_mark(ctx, producer, ev));
    return stream_wait_slot(ctx, waiter, ev);
}

// bf16-input GEMMs go through hipBLASLt with its first heuristic choice (rocBLAS remains for fp32 inputs and
// for a shape hipBLASLt has no algorithm for). For the long-K products of the backward (the MLP's and the
// LM head's input gradients, d_h = d_gu W_gu with K = 16384 and d_y = d_logits W_lm with K = 100352, where
// M = N = 2048 gives a plain tiling only 64 output tiles) its choice splits K across workgroups and sums the
// parts in a workspace; it is bitwise repeatable run to run. Measured on the OLMo-2-1B shapes: forward
// 6.56 -> 6.42 ms, training step 31.5 -> 30.8 ms. A plan (descriptors and the chosen algorithm) is made
// once per shape and kept in the context.
namespace {
constexpr size_t kLtWorkspace = size_t(128) << 20;
constexpr int kLtCandidates = 16;  // heuristic candidates timed for a new shape
struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};
struct LtCache {
    hipblasLtHandle_t h = nullptr;
    std::map<std::array<int, 10>, LtPlan> plans;
};
// an order-independent 64-bit fingerprint of n words: sum of w_i * (odd multiplier of i), modulo 2^64 (integer
// additions commute, so the atomics leave the same value whatever order the blocks finish in)
__global__ void words_fingerprint_kernel(const uint32_t* p, int64_t n, unsigned long long* out) {
    unsigned long long acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        acc += (unsigned long long)p[i] * ((unsigned long long)i * 0x9E3779B97F4A7C15ull | 1ull);
    atomicAdd(out, acc);
}

// the split-K workspace of GEMMs on stream s (the side stream has its own: GEMMs on the two streams overlap)
DeviceBuffer& lt_workspace(dt_ctx* ctx, hipStream_t s) {
    return (ctx->side && s == static_cast<hipStream_t>(ctx->side)) ? ctx->lt_ws_side : ctx->lt_ws;
}

void lt_free(LtPlan& p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
}
}  // namespace

// One-time choice among hipBLASLt's heuristic candidates for a shape, returned as the candidate's rank in the
// heuristic list (0: its first choice). Each candidate runs once into a zeroed scratch output (beta 0, so an
// accumulating caller's C is not touched), again, then five times under events; a candidate whose second run does
// not reproduce the first bit for bit (a split-K reduction by atomics) is dropped. The first choice is kept unless
// another candidate is at least kTuneMargin faster; otherwise the lowest-ranked candidate within kTuneTie of the
// fastest wins, so that two timings of the same candidates rarely choose differently. Synchronises the stream.
constexpr float kTuneMargin = 0.05f;
constexpr float kTuneTie = 0.03f;
static int lt_tune(dt_ctx* ctx, hipStream_t s, hipblasLtHandle_t h, LtPlan& p,
                   const hipblasLtMatmulHeuristicResult_t* heur, int n, int M, int ldc, bool c_bf16, const void* A,
                   const void* B, int* rank) {
    *rank = 0;
    DeviceBuffer& ws = lt_workspace(ctx, s);
    DT_TRY(ws.ensure(kLtWorkspace));
    // whole 32-bit words covering the ldc * M output elements, the tail padded with zeros
    const size_t out_bytes = (size_t)ldc * M * (c_bf16 ? 2 : 4);
    const size_t words = (out_bytes + 3) / 4;
    void* scratch = nullptr;
    unsigned long long* fp = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&scratch, words * 4) != hipSuccess || hipMalloc(&fp, 2 * sizeof(unsigned long long)) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess ||
        hipMemsetAsync(scratch, 0, words * 4, s) != hipSuccess) {
        (void)hipGetLastError();  // no room to tune: keep the first heuristic choice
        if (scratch) (void)hipFree(scratch);
        if (fp) (void)hipFree(fp);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        return DT_OK;
    }
    const float one = 1.0f, zero = 0.0f;
    auto run = [&](const hipblasLtMatmulAlgo_t& algo) {
        return hipblasLtMatmul(h, p.desc, &one, B, p.la, A, p.lb, &zero, scratch, p.lc, scratch, p.lc, &algo,
                               ws.ptr, kLtWorkspace, s) == HIPBLAS_STATUS_SUCCESS;
    };
    const int64_t nw = (int64_t)words;
    const unsigned blocks = (unsigned)std::min<int64_t>((nw + 255) / 256, 4096);
    std::vector<float> ms_of(n, -1.0f);  // -1: failed or not reproducible
    for (int i = 0; i < n; ++i) {
        if (hipMemsetAsync(fp, 0, 2 * sizeof(unsigned long long), s) != hipSuccess) break;
        if (!run(heur[i].algo)) continue;
        hipLaunchKernelGGL(words_fingerprint_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint32_t*>(scratch),
                           nw, fp);
        bool ok = run(heur[i].algo);
        hipLaunchKernelGGL(words_fingerprint_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint32_t*>(scratch),
                           nw, fp + 1);
        ok = ok && hipEventRecord(e0, s) == hipSuccess;
        for (int r = 0; r < 5 && ok; ++r) ok = run(heur[i].algo);
        ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
        unsigned long long f[2] = {0, 1};
        ok = ok && hipMemcpy(f, fp, sizeof(f), hipMemcpyDeviceToHost) == hipSuccess;
        float ms = 0.0f;
        ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
        if (!ok) {
            (void)hipGetLastError();
            continue;
        }
        if (f[0] == f[1]) ms_of[i] = ms;  // else not reproducible run to run
    }
    (void)hipStreamSynchronize(s);
    (void)hipFree(scratch);
    (void)hipFree(fp);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    float best = -1.0f;
    for (int i = 0; i < n; ++i)
        if (ms_of[i] >= 0.0f && (best < 0.0f || ms_of[i] < best)) best = ms_of[i];
    if (best < 0.0f || (ms_of[0] >= 0.0f && best >= (1.0f - kTuneMargin) * ms_of[0])) return DT_OK;
    for (int i = 0; i < n; ++i)
        if (ms_of[i] >= 0.0f && ms_of[i] <= (1.0f + kTuneTie) * best) {
            *rank = i;
            break;
        }
    p.algo = heur[*rank].algo;
    return DT_OK;
}

// The rank chosen for a shape on a device, shared by every context of the process, so that all of them run the
// same algorithm for it and give the same bits (another process may time the candidates differently).
static std::mutex g_tune_mu;
static std::map<std::array<int, 11>, int> g_tune_rank;

// Row-major C[M][N] = op(A) op(B) + beta C with bf16 A, B and fp32 C (bf16 C when c_bf16) through hipBLASLt
// (the same column-major mapping as gemm_rm below). Returns 1 (no error set) when hipBLASLt offers no
// algorithm for the shape.
static int gemm_lt(dt_ctx* ctx, hipStream_t s, bool ta, bool tb, int M, int N, int K, const void* A, int lda,
                   const void* B, int ldb, float beta, void* C, int ldc, bool c_bf16 = false) {
    LtCache* lc = static_cast<LtCache*>(ctx->lt);
    if (!lc) {
        lc = new LtCache;
        if (hipblasLtCreate(&lc->h) != HIPBLAS_STATUS_SUCCESS) {
            delete lc;
            return set_error(DT_ERR_BLAS, "hipblasLtCreate failed");
        }
        ctx->lt = lc;
    }
    const std::array<int, 10> key{ta, tb, M, N, K, lda, ldb, ldc, beta == 0.0f, c_bf16};
    auto it = lc->plans.find(key);
    if (it == lc->plans.end()) {
        LtPlan p;
        const hipblasOperation_t opa = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;  // hipBLASLt's A is our B
        const hipblasOperation_t opb = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa)) ==
                      HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb)) ==
                      HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, tb ? K : N, tb ? N : K, ldb) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, ta ? M : K, ta ? K : M, lda) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&p.lc, c_bf16 ? HIP_R_16BF : HIP_R_32F, N, M, ldc) ==
                      HIPBLAS_STATUS_SUCCESS;
        int n = 0;
        hipblasLtMatmulHeuristicResult_t heur[kLtCandidates]{};
        if (ok) {
            hipblasLtMatmulPreference_t pref = nullptr;
            size_t wsz = kLtWorkspace;
            ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                       sizeof(wsz)) == HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulAlgoGetHeuristic(lc->h, p.desc, p.la, p.lb, p.lc, p.lc, pref,
                                                 ctx->gemm_tune ? kLtCandidates : 1, heur, &n) == HIPBLAS_STATUS_SUCCESS;
            if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        }
        if (!ok || n < 1) {
            lt_free(p);
            return 1;
        }
        p.algo = heur[0].algo;
        if (n > 1) {
            const std::array<int, 11> gkey{ctx->device, ta, tb, M, N, K, lda, ldb, ldc, beta == 0.0f, c_bf16};
            std::lock_guard<std::mutex> lock(g_tune_mu);
            auto g = g_tune_rank.find(gkey);
            if (g != g_tune_rank.end()) {
                if (g->second < n) p.algo = heur[g->second].algo;
            } else {
                // a capturing stream cannot take the tuning's allocations and synchronisations: keep the first
                // choice for this context and leave the shape to be tuned by a later uncaptured call
                hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
                if (hipStreamIsCapturing(s, &cs) != hipSuccess) (void)hipGetLastError();
                if (cs == hipStreamCaptureStatusNone) {
                    int rank = 0;
                    DT_TRY(lt_tune(ctx, s, lc->h, p, heur, n, M, ldc, c_bf16, A, B, &rank));
                    g_tune_rank.emplace(gkey, rank);
                }
            }
        }
        it = lc->plans.emplace(key, p).first;
    }
    DeviceBuffer& ws = lt_workspace(ctx, s);
    DT_TRY(ws.ensure(kLtWorkspace));
    const float one = 1.0f;
    const LtPlan& p = it->second;
    if (hipblasLtMatmul(lc->h, p.desc, &one, B, p.la, A, p.lb, &beta, C, p.lc, C, p.lc, &p.algo, ws.ptr,
                        kLtWorkspace, s) != HIPBLAS_STATUS_SUCCESS)
        return set_error(DT_ERR_BLAS, "hipBLASLt GEMM (%d x %d x %d%s) failed", M, N, K, c_bf16 ? ", bf16 out" : "");
    return DT_OK;
}

// Row-major C[M][N] = op(A)[M][K] op(B)[K][N] + beta C, op = transpose when the flag is set (A is then
// stored [K][M], B [N][K]). In rocBLAS's column-major terms a row-major X is X^T, so this is
// C^T = op(B)^T op(A)^T: B goes first, each transposed exactly when it is transposed here.
int gemm_rm(dt_ctx* ctx, hipStream_t s, bool ta, bool tb, int M, int N, int K, const void* A, int lda,
                   const void* B, int ldb, float beta, float* C, int ldc, bool bf16_in) {
    const float one = 1.0f;
    const rocblas_operation opb = tb ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation opa = ta ? rocblas_operation_transpose : rocblas_operation_none;
    if (bf16_in) {
        const int rc = gemm_lt(ctx, s, ta, tb, M, N, K, A, lda, B, ldb, beta, C, ldc);
        if (rc <= 0) return rc;  // done, or an error; 1: no hipBLASLt algorithm, rocBLAS below
    }
    rocblas_handle h = nullptr;
    DT_TRY(ensure_blas(ctx, s, &h));
    rocblas_status st;
    if (!bf16_in) {
        st = rocblas_sgemm(h, opb, opa, N, M, K, &one, static_cast<const float*>(B), ldb, static_cast<const float*>(A),
                           lda, &beta, C, ldc);
    } else {
        st = rocblas_gemm_ex(h, opb, opa, N, M, K, &one, B, rocblas_datatype_bf16_r, ldb, A, rocblas_datatype_bf16_r,
                             lda, &beta, C, rocblas_datatype_f32_r, ldc, C, rocblas_datatype_f32_r, ldc,
                             rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    }
    if (st != rocblas_status_success)
        return set_error(DT_ERR_BLAS, "rocBLAS GEMM (%d x %d x %d): %s", M, N, K, blas_status_str(st));
    return DT_OK;
}

int gemm_rm_bf16(dt_ctx* ctx, hipStream_t s, bool ta, bool tb, int M, int N, int K, const void* A, int lda,
                 const void* B, int ldb, void* C, int ldc) {
    const int rc = gemm_lt(ctx, s, ta, tb, M, N, K, A, lda, B, ldb, 0.0f, C, ldc, true);
    if (rc <= 0) return rc;  // done, or an error; 1: no hipBLASLt algorithm, rocBLAS below
    rocblas_handle h = nullptr;
    DT_TRY(ensure_blas(ctx, s, &h));
    const float one = 1.0f, zero = 0.0f;
    const rocblas_operation opb = tb ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation opa = ta ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_status st =
        rocblas_gemm_ex(h, opb, opa, N, M, K, &one, B, rocblas_datatype_bf16_r, ldb, A, rocblas_datatype_bf16_r, lda,
                        &zero, C, rocblas_datatype_bf16_r, ldc, C, rocblas_datatype_bf16_r, ldc, rocblas_datatype_f32_r,
                        rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success)
        return set_error(DT_ERR_BLAS, "rocBLAS GEMM (%d x %d x %d, bf16 out): %s", M, N, K, blas_status_str(st));
    return DT_OK;
}

// y = x W^T with W stored [N][K] like torch Linear (OlmoAttention.cpp:68,74,80,104)
static int gemm_xwt(dt_ctx* ctx, hipStream_t s, int M, int N, int K, const void* A, int lda, const void* W, int ldw,
                    float* C, int ldc, bool bf16_in) {
    return gemm_rm(ctx, s, false, true, M, N, K, A, lda, W, ldw, 0.0f, C, ldc, bf16_in);
}

// ---------------- .npy reader (v1/v2/v3, little-endian fp32, C order) ----------------
// Parses a .npy header (v1-v3): little-endian float32 in C order, the shape, and where the data starts; checks
// that the file holds all of the data. The file is left open at the data when f_out is given, else closed.
static int npy_header(const std::string& path, std::vector<size_t>& shape, FILE** f_out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return set_error(DT_ERR_IO, "cannot open %s", path.c_str());
    auto fail = [&](int rc) {
        std::fclose(f);
        return rc;
    };
    unsigned char magic[8];
    if (std::fread(magic, 1, 8, f) != 8 || std::memcmp(magic, "\x93NUMPY", 6) != 0)
        return fail(set_error(DT_ERR_IO, "%s is not a .npy file (a Git-LFS pointer?)", path.c_str()));
    uint32_t hlen = 0;
    long data_at = 0;
    if (magic[6] == 1) {
        unsigned char b[2];
        if (std::fread(b, 1, 2, f) != 2) return fail(set_error(DT_ERR_IO, "%s: truncated", path.c_str()));
        hlen = b[0] | (b[1] << 8);
        data_at = 10 + (long)hlen;
    } else {
        unsigned char b[4];
        if (std::fread(b, 1, 4, f) != 4) return fail(set_error(DT_ERR_IO, "%s: truncated", path.c_str()));
        hlen = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
        data_at = 12 + (long)hlen;
    }
    if (hlen > (1u << 20)) return fail(set_error(DT_ERR_IO, "%s: header of %u bytes", path.c_str(), hlen));
    std::string hdr(hlen, '\0');
    if (std::fread(&hdr[0], 1, hlen, f) != hlen) return fail(set_error(DT_ERR_IO, "%s: truncated", path.c_str()));
    if (hdr.find("'<f4'") == std::string::npos || hdr.find("'fortran_order': False") == std::string::npos)
        return fail(set_error(DT_ERR_IO, "%s: need little-endian float32 in C order, header %s", path.c_str(),
                              hdr.c_str()));
    size_t p = hdr.find("'shape': (");
    if (p == std::string::npos) return fail(set_error(DT_ERR_IO, "%s: no shape", path.c_str()));
    p += 10;
    shape.clear();
    size_t n = 1;
    while (p < hdr.size() && hdr[p] != ')') {
        while (p < hdr.size() && (hdr[p] == ' ' || hdr[p] == ',')) ++p;
        if (p < hdr.size() && hdr[p] == ')') break;
        size_t v = 0;
        bool any = false;
        while (p < hdr.size() && hdr[p] >= '0' && hdr[p] <= '9') {
            v = v * 10 + (hdr[p] - '0');
            ++p;
            any = true;
        }
        if (!any) return fail(set_error(DT_ERR_IO, "%s: bad shape", path.c_str()));
        shape.push_back(v);
        n *= v;
    }
    if (std::fseek(f, 0, SEEK_END) != 0) return fail(set_error(DT_ERR_IO, "%s: cannot seek", path.c_str()));
    const long size = std::ftell(f);
    if (size < 0 || (size_t)(size - data_at) < n * sizeof(float) || size < data_at)
        return fail(set_error(DT_ERR_IO, "%s: truncated data", path.c_str()));
    if (!f_out) {
        std::fclose(f);
        return DT_OK;
    }
    if (std::fseek(f, data_at, SEEK_SET) != 0) return fail(set_error(DT_ERR_IO, "%s: cannot seek", path.c_str()));
    *f_out = f;
    return DT_OK;
}

int read_npy_shape(const std::string& path, std::vector<size_t>& shape) { return npy_header(path, shape, nullptr); }

int read_npy_f32(const std::string& path, std::vector<float>& out, std::vector<size_t>& shape) {
    FILE* f = nullptr;
    DT_TRY(npy_header(path, shape, &f));
    size_t n = 1;
    for (size_t v : shape) n *= v;
    out.resize(n);
    const size_t got = std::fread(out.data(), sizeof(float), n, f);
    std::fclose(f);
    if (got != n) return set_error(DT_ERR_IO, "%s: truncated data", path.c_str());
    return DT_OK;
}

}  // namespace dt

// ---------------- layer ----------------

using namespace dt;

extern "C" {

const char* dt_last_error(void) { return t_err.c_str(); }

int dt_version(void) { return 3; }

int dt_ctx_create(int device, dt_ctx** out) {
    clear_error();
    if (!out) return set_error(DT_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (device < 0) return set_error(DT_ERR_INVALID_ARG, "device %d < 0", device);
    int count = 0;
    DT_HIP_TRY(hipGetDeviceCount(&count));
    if (device >= count) return set_error(DT_ERR_INVALID_ARG, "device %d >= device count %d", device, count);
    DT_HIP_TRY(hipSetDevice(device));
    DT_TRY(noalloc_setup(device));  // this device's address of the no-alloc entry point's scratch array
    dt_ctx* c = new dt_ctx();
    c->device = device;
    int rc = rope_upload(c, DT_ROPE_THETA, DT_MAX_SEQ_LEN);
    if (rc != DT_OK) {
        delete c;
        return rc;
    }
    *out = c;
    return DT_OK;
}

int dt_ctx_set_option(dt_ctx* ctx, int option, int value) {
    clear_error();
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    if (option == DT_OPT_QKV_FUSED) {
        if (value != DT_QKV_GEMM && value != DT_QKV_FUSED && value != DT_QKV_AUTO)
            return set_error(DT_ERR_INVALID_ARG, "DT_OPT_QKV_FUSED takes DT_QKV_GEMM, DT_QKV_FUSED or DT_QKV_AUTO, not %d",
                             value);
        ctx->qkv_fused = value;
        return DT_OK;
    }
    if (option == DT_OPT_GEMM_TUNE) {
        if (value != 0 && value != 1) return set_error(DT_ERR_INVALID_ARG, "DT_OPT_GEMM_TUNE takes 0 or 1, not %d", value);
        ctx->gemm_tune = value;
        return DT_OK;
    }
    if (option == DT_OPT_QKV_SPIN_LIMIT) {
        if (value < 0) return set_error(DT_ERR_INVALID_ARG, "DT_OPT_QKV_SPIN_LIMIT must be >= 0, not %d", value);
        ctx->qkv_spin = value;
        return DT_OK;
    }
    if (option == DT_OPT_SIDE_STREAM) {
        if (value != 0 && value != 1) return set_error(DT_ERR_INVALID_ARG, "DT_OPT_SIDE_STREAM takes 0 or 1, not %d", value);
        ctx->side_off = !value;
        return DT_OK;
    }
    if (option == DT_OPT_BWD_DQ) {
        if (value != DT_BWD_DQ_RECOMPUTE && value != DT_BWD_DQ_FROM_DS && value != DT_BWD_DQ_AUTO)
            return set_error(DT_ERR_INVALID_ARG,
                             "DT_OPT_BWD_DQ takes DT_BWD_DQ_RECOMPUTE, DT_BWD_DQ_FROM_DS or DT_BWD_DQ_AUTO, not %d", value);
        ctx->bwd_dq = value;
        return DT_OK;
    }
    return set_error(DT_ERR_INVALID_ARG, "unknown context option %d", option);
}

int dt_ctx_destroy(dt_ctx* ctx) {
    clear_error();
    if (!ctx) return DT_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->rope_cos) (void)hipFree(ctx->rope_cos);
    if (ctx->rope_sin) (void)hipFree(ctx->rope_sin);
    for (auto& b : ctx->stage) b.release();
    ctx->bwd_stats.release();
    ctx->bwd_ds.release();
    ctx->fwd_split.release();
    ctx->fwd_split_cnt.release();
    ctx->qkv_ss.release();
    ctx->qkv_status.release();
    if (ctx->side) (void)hipStreamSynchronize(static_cast<hipStream_t>(ctx->side));
    if (ctx->blas) rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas));
    if (ctx->blas_side) rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas_side));
    for (void* e : ctx->ev)
        if (e) (void)hipEventDestroy(static_cast<hipEvent_t>(e));
    if (ctx->side) (void)hipStreamDestroy(static_cast<hipStream_t>(ctx->side));
    if (ctx->lt) {
        LtCache* lc = static_cast<LtCache*>(ctx->lt);
        for (auto& kv : lc->plans) lt_free(kv.second);
        hipblasLtDestroy(lc->h);
        delete lc;
    }
    ctx->lt_ws.release();
    ctx->lt_ws_side.release();
    delete ctx;
    return DT_OK;
}

int dt_ctx_check(dt_ctx* ctx) {
    clear_error();
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));
    DT_HIP_TRY(hipDeviceSynchronize());
    return qkv_status_check(ctx);
}

int dt_rope_table_init(dt_ctx* ctx, float theta, int max_seq_len) {
    clear_error();
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    if (!(theta > 1.0f) || !std::isfinite(theta)) return set_error(DT_ERR_INVALID_ARG, "theta %g must be > 1", theta);
    if (max_seq_len < 1 || max_seq_len > (1 << 20))
        return set_error(DT_ERR_INVALID_ARG, "max_seq_len %d outside [1, 2^20]", max_seq_len);
    DT_TRY(check_device_binding(ctx));
    return rope_upload(ctx, theta, max_seq_len);
}

int dt_flash_attn_fwd(dt_ctx* ctx, const void* q, const void* k, const void* v, void* o, float* m, float* l, int B,
                      int T, int H, int D, float scale, int causal, const int32_t* seq_lens, int dtype, int mem,
                      void* stream) {
    clear_error();
    if (!q || !k || !v || !o) return set_error(DT_ERR_INVALID_ARG, "q, k, v and o must be non-NULL");
    if (D != DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "head_dim D=%d, kernels are built for D=%d", D, DT_HEAD_DIM);
    if (B < 1 || H < 1 || T < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d, H=%d must be >= 1", B, T, H);
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if (H > 65535 || B > 65535) return set_error(DT_ERR_UNSUPPORTED, "B=%d or H=%d exceeds grid limits", B, H);
    if (dtype != DT_FP32_EXACT && dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (!(scale > 0.0f) || !std::isfinite(scale)) return set_error(DT_ERR_INVALID_ARG, "scale %g must be finite and > 0", scale);
    if (causal != 0 && causal != 1) return set_error(DT_ERR_INVALID_ARG, "causal must be 0 or 1");
    if (mem == DT_MEM_DEVICE && (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)))
        return set_error(DT_ERR_INVALID_ARG, "device q/k/v/o must be 16-byte aligned");
    DT_TRY(validate_seq_lens(seq_lens, B, T));
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int ld = H * D;
    FlashArgs fa{q, k, v, o, m, l, B, T, H, ld, ld, ld, ld, scale, causal, seq_lens ? 1 : 0};
    if (mem == DT_MEM_DEVICE) return run_flash(ctx, fa, seq_lens, dtype, s);

    // host memory: stage through context buffers, synchronous like the reference
    const size_t esz = dtype == DT_BF16 ? 2 : 4;
    const size_t nel = (size_t)B * T * H * D;
    const size_t nst = (size_t)B * T * H;
    for (int i = 0; i < 4; ++i) DT_TRY(ctx->stage[i].ensure(nel * esz));
    DT_TRY(ctx->stage[4].ensure(nst * sizeof(float)));
    DT_TRY(ctx->stage[5].ensure(nst * sizeof(float)));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[0].ptr, q, nel * esz, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[1].ptr, k, nel * esz, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[2].ptr, v, nel * esz, hipMemcpyHostToDevice, s));
    FlashArgs fd = fa;
    fd.q = ctx->stage[0].ptr;
    fd.k = ctx->stage[1].ptr;
    fd.v = ctx->stage[2].ptr;
    fd.o = ctx->stage[3].ptr;
    fd.m = m ? static_cast<float*>(ctx->stage[4].ptr) : nullptr;
    fd.l = l ? static_cast<float*>(ctx->stage[5].ptr) : nullptr;
    DT_TRY(run_flash(ctx, fd, seq_lens, dtype, s));
    DT_HIP_TRY(hipMemcpyAsync(o, fd.o, nel * esz, hipMemcpyDeviceToHost, s));
    if (m) DT_HIP_TRY(hipMemcpyAsync(m, fd.m, nst * sizeof(float), hipMemcpyDeviceToHost, s));
    if (l) DT_HIP_TRY(hipMemcpyAsync(l, fd.l, nst * sizeof(float), hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

// The dS workspace of an attention backward when DT_OPT_BWD_DQ selects the dS path, else NULL. The
// automatic choice takes it where it measured faster (more than one 128-row block per CU and pass, e.g.
// B*H = 16 at T = 4096), with a buffer of at most kDsAutoCap bytes and a quarter of the device's free memory
// (the buffer is kept by the context; an unbounded one could starve the caller's own allocator), and takes the
// recompute path above that or when the buffer cannot be allocated.
constexpr size_t kDsAutoCap = size_t(2) << 30;
static int bwd_ds_workspace(dt_ctx* ctx, int B, int H, int T, int causal, int dtype, void** ws) {
    *ws = nullptr;
    if (ctx->bwd_dq == DT_BWD_DQ_RECOMPUTE) return DT_OK;
    const size_t bytes = flash_bwd_ds_bytes(B, H, T, causal, dtype == DT_BF16 ? 2 : 4);
    if (ctx->bwd_dq == DT_BWD_DQ_AUTO) {
        int cus = 0;
        DT_TRY(persistent_grid(0x7fffffff, &cus));
        const int64_t blocks = (int64_t)((T + 127) / 128) * B * H;
        if (blocks <= cus) return DT_OK;
        if (ctx->bwd_ds.bytes < bytes) {
            size_t free_b = 0, total_b = 0;
            if (bytes > kDsAutoCap || hipMemGetInfo(&free_b, &total_b) != hipSuccess || bytes > free_b / 4) {
                (void)hipGetLastError();
                return DT_OK;
            }
        }
        if (ctx->bwd_ds.ensure(bytes) != DT_OK) {  // out of memory: the recompute path needs no buffer
            (void)hipGetLastError();
            clear_error();
            return DT_OK;
        }
    } else {
        DT_TRY(ctx->bwd_ds.ensure(bytes));
    }
    *ws = ctx->bwd_ds.ptr;
    return DT_OK;
}

int dt_flash_attn_bwd(dt_ctx* ctx, const void* d_o, const void* o, const float* m, const float* l, const void* q,
                      const void* k, const void* v, void* d_q, void* d_k, void* d_v, int B, int T, int H, int D,
                      float scale, int causal, int dtype, int mem, void* stream) {
    clear_error();
    if (!d_o || !o || !m || !l || !q || !k || !v || !d_q || !d_k || !d_v)
        return set_error(DT_ERR_INVALID_ARG, "all tensor pointers must be non-NULL");
    if (D != DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "head_dim D=%d, kernels are built for D=%d", D, DT_HEAD_DIM);
    if (B < 1 || H < 1 || T < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d, H=%d must be >= 1", B, T, H);
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if (H > 65535 || B > 65535) return set_error(DT_ERR_UNSUPPORTED, "B=%d or H=%d exceeds grid limits", B, H);
    if (dtype != DT_FP32_EXACT && dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (!(scale > 0.0f) || !std::isfinite(scale)) return set_error(DT_ERR_INVALID_ARG, "scale %g must be finite and > 0", scale);
    if (causal != 0 && causal != 1) return set_error(DT_ERR_INVALID_ARG, "causal must be 0 or 1");
    if (mem == DT_MEM_DEVICE && (!aligned16(d_o) || !aligned16(o) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
                                 !aligned16(d_q) || !aligned16(d_k) || !aligned16(d_v)))
        return set_error(DT_ERR_INVALID_ARG, "device tensors must be 16-byte aligned");
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int ld = H * D;
    const size_t nst = (size_t)B * T * H;
    DT_TRY(ctx->bwd_stats.ensure(2 * nst * sizeof(float)));
    float* stats = static_cast<float*>(ctx->bwd_stats.ptr);
    FlashBwdArgs ba{q, k, v, o, d_o, m, l, d_q, d_k, d_v, stats, stats + nst, B, T, H, ld, ld, ld, scale, causal};
    DT_TRY(bwd_ds_workspace(ctx, B, H, T, causal, dtype, &ba.ds_ws));
    auto run = [&](const FlashBwdArgs& x) {
        return dtype == DT_BF16 ? launch_flash_bwd_bf16(x, s) : launch_flash_bwd_f32(x, s);
    };
    if (mem == DT_MEM_DEVICE) return run(ba);

    // host memory: stage through context buffers, synchronous like the reference
    const size_t esz = dtype == DT_BF16 ? 2 : 4;
    const size_t nel = (size_t)B * T * H * D;
    for (int i = 0; i < 8; ++i) DT_TRY(ctx->stage[i].ensure(nel * esz));
    DT_TRY(ctx->stage[8].ensure(nst * sizeof(float)));
    DT_TRY(ctx->stage[9].ensure(nst * sizeof(float)));
    const void* src[5] = {d_o, o, q, k, v};
    for (int i = 0; i < 5; ++i) DT_HIP_TRY(hipMemcpyAsync(ctx->stage[i].ptr, src[i], nel * esz, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[8].ptr, m, nst * sizeof(float), hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[9].ptr, l, nst * sizeof(float), hipMemcpyHostToDevice, s));
    FlashBwdArgs bd = ba;
    bd.d_o = ctx->stage[0].ptr;
    bd.o = ctx->stage[1].ptr;
    bd.q = ctx->stage[2].ptr;
    bd.k = ctx->stage[3].ptr;
    bd.v = ctx->stage[4].ptr;
    bd.d_q = ctx->stage[5].ptr;
    bd.d_k = ctx->stage[6].ptr;
    bd.d_v = ctx->stage[7].ptr;
    bd.m = static_cast<const float*>(ctx->stage[8].ptr);
    bd.l = static_cast<const float*>(ctx->stage[9].ptr);
    DT_TRY(run(bd));
    DT_HIP_TRY(hipMemcpyAsync(d_q, bd.d_q, nel * esz, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipMemcpyAsync(d_k, bd.d_k, nel * esz, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipMemcpyAsync(d_v, bd.d_v, nel * esz, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

int dt_qk_norm_rope_fwd(dt_ctx* ctx, const float* q_in, const float* k_in, const float* q_norm_w,
                        const float* k_norm_w, void* q_out, void* k_out, float* q_rms, float* k_rms, int B, int T,
                        int H, int D, int ld_in, int ld_out, int out_dtype, int mem, void* stream) {
    clear_error();
    if (!q_in || !k_in || !q_norm_w || !k_norm_w || !q_out || !k_out)
        return set_error(DT_ERR_INVALID_ARG, "q_in, k_in, norm weights, q_out and k_out must be non-NULL");
    if (D != DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "head_dim D=%d, kernels are built for D=%d", D, DT_HEAD_DIM);
    if (B < 1 || T < 1 || H < 1 || H > 256) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d, H=%d out of range", B, T, H);
    if ((int64_t)B * T > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "B*T too large");
    if (ld_in < H * D || ld_out < H * D || (ld_in & 3) || (ld_out & 3))
        return set_error(DT_ERR_INVALID_ARG, "row strides ld_in=%d / ld_out=%d must be >= H*D=%d and multiples of 4",
                         ld_in, ld_out, H * D);
    if (out_dtype != DT_FP32_EXACT && out_dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", out_dtype);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (mem == DT_MEM_DEVICE && (!aligned16(q_in) || !aligned16(k_in) || !aligned16(q_out) || !aligned16(k_out) ||
                                 !aligned16(q_norm_w) || !aligned16(k_norm_w)))
        return set_error(DT_ERR_INVALID_ARG, "device pointers must be 16-byte aligned");
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    if (T > ctx->rope_len) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds the RoPE table length %d", T, ctx->rope_len);
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int rows = B * T;
    NormRopeArgs na{q_in, k_in, nullptr, q_norm_w, k_norm_w, q_out, k_out, nullptr, q_rms, k_rms,
                    ctx->rope_cos, ctx->rope_sin, rows, T, H, ld_in, ld_out, DT_RMS_EPS};
    if (mem == DT_MEM_DEVICE) return launch_qk_norm_rope(na, out_dtype == DT_BF16, s);

    const size_t esz = out_dtype == DT_BF16 ? 2 : 4;
    const size_t in_bytes = (size_t)rows * ld_in * 4, out_bytes = (size_t)rows * ld_out * esz;
    const size_t w_bytes = (size_t)H * D * 4;
    DT_TRY(ctx->stage[0].ensure(in_bytes));
    DT_TRY(ctx->stage[1].ensure(in_bytes));
    DT_TRY(ctx->stage[2].ensure(out_bytes));
    DT_TRY(ctx->stage[3].ensure(out_bytes));
    DT_TRY(ctx->stage[4].ensure(2 * w_bytes));
    DT_TRY(ctx->stage[5].ensure(2 * (size_t)rows * 4));
    char* wbuf = static_cast<char*>(ctx->stage[4].ptr);
    float* rbuf = static_cast<float*>(ctx->stage[5].ptr);
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[0].ptr, q_in, in_bytes, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(ctx->stage[1].ptr, k_in, in_bytes, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(wbuf, q_norm_w, w_bytes, hipMemcpyHostToDevice, s));
    DT_HIP_TRY(hipMemcpyAsync(wbuf + w_bytes, k_norm_w, w_bytes, hipMemcpyHostToDevice, s));
    NormRopeArgs nd = na;
    nd.q_in = static_cast<const float*>(ctx->stage[0].ptr);
    nd.k_in = static_cast<const float*>(ctx->stage[1].ptr);
    nd.q_w = reinterpret_cast<const float*>(wbuf);
    nd.k_w = reinterpret_cast<const float*>(wbuf + w_bytes);
    nd.q_out = ctx->stage[2].ptr;
    nd.k_out = ctx->stage[3].ptr;
    nd.q_rms = q_rms ? rbuf : nullptr;
    nd.k_rms = k_rms ? rbuf + rows : nullptr;
    DT_TRY(launch_qk_norm_rope(nd, out_dtype == DT_BF16, s));
    DT_HIP_TRY(hipMemcpyAsync(q_out, nd.q_out, out_bytes, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipMemcpyAsync(k_out, nd.k_out, out_bytes, hipMemcpyDeviceToHost, s));
    if (q_rms) DT_HIP_TRY(hipMemcpyAsync(q_rms, rbuf, rows * 4, hipMemcpyDeviceToHost, s));
    if (k_rms) DT_HIP_TRY(hipMemcpyAsync(k_rms, rbuf + rows, rows * 4, hipMemcpyDeviceToHost, s));
    DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

}  // extern "C"

int attn_layer_alloc(dt_ctx* ctx, int d_model, int n_heads, dt_attn_layer** out) {
    dt_attn_layer* L = new dt_attn_layer();
    L->ctx = ctx;
    L->d_model = d_model;
    L->n_heads = n_heads;
    const size_t wsz = (size_t)d_model * d_model * sizeof(float);
    hipError_t e = hipMalloc(&L->w_qkv, 3 * wsz);
    if (e == hipSuccess) e = hipMalloc(&L->w_o, wsz);
    if (e == hipSuccess) e = hipMalloc(&L->q_norm, d_model * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&L->k_norm, d_model * sizeof(float));
    if (e == hipSuccess) e = hipMemset(L->w_qkv, 0, 3 * wsz);
    if (e == hipSuccess) e = hipMemset(L->w_o, 0, wsz);
    if (e == hipSuccess) e = hipMemset(L->q_norm, 0, d_model * sizeof(float));
    if (e == hipSuccess) e = hipMemset(L->k_norm, 0, d_model * sizeof(float));
    if (e != hipSuccess) {
        dt_attn_layer_destroy(L);
        return set_error(DT_ERR_HIP, "layer allocation: %s", hipGetErrorString(e));
    }
    *out = L;
    return DT_OK;
}

extern "C" {

int dt_attn_layer_create(dt_ctx* ctx, const float* wq, const float* wk, const float* wv, const float* wo,
                         const float* q_norm_w, const float* k_norm_w, int d_model, int n_heads, int mem,
                         dt_attn_layer** out) {
    clear_error();
    if (!out) return set_error(DT_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!wq || !wk || !wv || !wo || !q_norm_w || !k_norm_w) return set_error(DT_ERR_INVALID_ARG, "weights must be non-NULL");
    if (n_heads < 1 || n_heads > 256 || d_model != n_heads * DT_HEAD_DIM)
        return set_error(DT_ERR_UNSUPPORTED, "d_model=%d must equal n_heads (%d) * %d", d_model, n_heads, DT_HEAD_DIM);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    DT_TRY(check_device_binding(ctx));
    dt_attn_layer* L = nullptr;
    DT_TRY(attn_layer_alloc(ctx, d_model, n_heads, &L));
    const size_t wsz = (size_t)d_model * d_model * sizeof(float);
    const hipMemcpyKind kind = mem == DT_MEM_HOST ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    hipError_t e = hipMemcpy(L->w_qkv, wq, wsz, kind);
    if (e == hipSuccess) e = hipMemcpy(reinterpret_cast<char*>(L->w_qkv) + wsz, wk, wsz, kind);
    if (e == hipSuccess) e = hipMemcpy(reinterpret_cast<char*>(L->w_qkv) + 2 * wsz, wv, wsz, kind);
    if (e == hipSuccess) e = hipMemcpy(L->w_o, wo, wsz, kind);
    if (e == hipSuccess) e = hipMemcpy(L->q_norm, q_norm_w, d_model * sizeof(float), kind);
    if (e == hipSuccess) e = hipMemcpy(L->k_norm, k_norm_w, d_model * sizeof(float), kind);
    if (e != hipSuccess) {
        dt_attn_layer_destroy(L);
        return set_error(DT_ERR_HIP, "layer weight upload: %s", hipGetErrorString(e));
    }
    *out = L;
    return DT_OK;
}

int dt_attn_layer_load(dt_ctx* ctx, const char* folder, unsigned index, dt_attn_layer** out) {
    clear_error();
    if (!out) return set_error(DT_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!folder) return set_error(DT_ERR_INVALID_ARG, "folder is NULL");
    // file names of the OlmoAttention(folder, index) constructor, OlmoAttention.cpp:39-53
    const char* names[6] = {"q_proj.weight", "k_proj.weight", "v_proj.weight",
                            "o_proj.weight", "q_norm.weight", "k_norm.weight"};
    std::vector<float> w[6];
    size_t d = 0;
    for (int i = 0; i < 6; ++i) {
        std::string path = std::string(folder) + "/model.layers." + std::to_string(index) + ".self_attn." + names[i] + ".npy";
        std::vector<size_t> shape;
        DT_TRY(read_npy_f32(path, w[i], shape));
        if (i == 0) {
            if (shape.size() != 2 || shape[0] != shape[1]) return set_error(DT_ERR_IO, "%s: expected a square matrix", path.c_str());
            d = shape[0];
        }
        const bool ok = i < 4 ? (shape.size() == 2 && shape[0] == d && shape[1] == d) : (shape.size() == 1 && shape[0] == d);
        if (!ok) return set_error(DT_ERR_IO, "%s: unexpected shape", path.c_str());
    }
    if (d % DT_HEAD_DIM) return set_error(DT_ERR_UNSUPPORTED, "d_model=%zu is not a multiple of %d", d, DT_HEAD_DIM);
    if (!ctx) return set_error(DT_ERR_INVALID_ARG, "ctx is NULL");
    return dt_attn_layer_create(ctx, w[0].data(), w[1].data(), w[2].data(), w[3].data(), w[4].data(), w[5].data(),
                                (int)d, (int)(d / DT_HEAD_DIM), DT_MEM_HOST, out);
}

int dt_attn_layer_destroy(dt_attn_layer* L) {
    clear_error();
    if (!L) return DT_OK;
    if (L->ctx) (void)hipSetDevice(L->ctx->device);
    if (L->w_qkv) (void)hipFree(L->w_qkv);
    if (L->w_o) (void)hipFree(L->w_o);
    if (L->w_qkv16) (void)hipFree(L->w_qkv16);
    if (L->w_o16) (void)hipFree(L->w_o16);
    if (L->q_norm) (void)hipFree(L->q_norm);
    if (L->k_norm) (void)hipFree(L->k_norm);
    if (L->g_qkv) (void)hipFree(L->g_qkv);
    if (L->g_o) (void)hipFree(L->g_o);
    if (L->g_qn) (void)hipFree(L->g_qn);
    if (L->g_kn) (void)hipFree(L->g_kn);
    for (dt::DeviceBuffer* b : {&L->qkv_pre, &L->qkv16, &L->attn, &L->x16, &L->x32, &L->att32, &L->rms, &L->stats,
                                &L->d_attn32, &L->d16, &L->d_qkv, &L->partial})
        b->release();
    delete L;
    return DT_OK;
}

int dt_attn_layer_fwd(dt_attn_layer* L, const float* x, float* out, int B, int T, const int32_t* seq_lens,
                      int dtype, int mem, int save_for_backward, void* stream) {
    return attn_layer_fwd(L, x, out, B, T, seq_lens, dtype, mem, save_for_backward, stream, false);
}

}  // extern "C"

int attn_layer_fwd(dt_attn_layer* L, const float* x, float* out, int B, int T, const int32_t* seq_lens, int dtype,
                   int mem, int save_for_backward, void* stream, bool x16_ready) {
    clear_error();
    if (x16_ready && (dtype != DT_BF16 || mem != DT_MEM_DEVICE))
        return set_error(DT_ERR_INVALID_ARG, "a bf16 copy of x is taken in bf16 mode with device memory only");
    if (!x || !out) return set_error(DT_ERR_INVALID_ARG, "x and out must be non-NULL");
    if (B < 1 || T < 1) return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d must be >= 1", B, T);
    if (T > DT_MAX_SEQ_LEN) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds max_seq_len %d", T, DT_MAX_SEQ_LEN);
    if ((int64_t)B * T > 0x7fffffff / 8) return set_error(DT_ERR_UNSUPPORTED, "B*T too large");
    if (dtype != DT_FP32_EXACT && dtype != DT_BF16) return set_error(DT_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (save_for_backward != 0 && save_for_backward != 1)
        return set_error(DT_ERR_INVALID_ARG, "save_for_backward must be 0 or 1");
    if (save_for_backward && seq_lens)
        return set_error(DT_ERR_UNSUPPORTED, "save_for_backward with seq_lens: the backward covers full sequences only");
    if (mem == DT_MEM_DEVICE && (!aligned16(x) || !aligned16(out)))
        return set_error(DT_ERR_INVALID_ARG, "device x/out must be 16-byte aligned");
    DT_TRY(validate_seq_lens(seq_lens, B, T));
    if (!L) return set_error(DT_ERR_INVALID_ARG, "layer is NULL");
    dt_ctx* ctx = L->ctx;
    if (T > ctx->rope_len) return set_error(DT_ERR_INVALID_ARG, "T=%d exceeds the RoPE table length %d", T, ctx->rope_len);
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);

    const int dm = L->d_model, H = L->n_heads, rows = B * T;
    const size_t act = (size_t)rows * dm;
    const float* xd = x;
    float* od = out;
    L->saved_T = 0;  // a failed or inference forward leaves nothing to differentiate
    if (save_for_backward && dtype != DT_BF16) {
        // the reference keeps its own copy of the input (m_act_input_2d, OlmoAttention.cpp:64); in bf16 mode that
        // copy is the bf16 x the projections read (x16 below), the only form of x the backward reads there
        DT_TRY(L->x32.ensure(act * 4));
        DT_HIP_TRY(hipMemcpyAsync(L->x32.ptr, x, act * 4, mem == DT_MEM_HOST ? hipMemcpyHostToDevice
                                                                              : hipMemcpyDeviceToDevice, s));
        xd = static_cast<const float*>(L->x32.ptr);
    } else if (mem == DT_MEM_HOST) {
        DT_TRY(ctx->stage[0].ensure(act * 4));
        DT_HIP_TRY(hipMemcpyAsync(ctx->stage[0].ptr, x, act * 4, hipMemcpyHostToDevice, s));
        xd = static_cast<const float*>(ctx->stage[0].ptr);
    }
    if (save_for_backward) {
        DT_TRY(L->rms.ensure((size_t)2 * rows * 4));
        DT_TRY(L->stats.ensure((size_t)2 * rows * H * 4));
    }
    if (mem == DT_MEM_HOST) {
        DT_TRY(ctx->stage[1].ensure(act * 4));
        od = static_cast<float*>(ctx->stage[1].ptr);
    }
    bool fused = ctx->qkv_fused == DT_QKV_FUSED && H % 4 == 0;  // (the fused kernel needs H % 4 == 0)
    // auto: the fused kernel in bf16 mode where its tiles fit one round (measured faster there); fp32 exact mode
    // keeps rocBLAS sgemm + the norm kernel (T = 512: 226 against 235 us per layer)
    if (ctx->qkv_fused == DT_QKV_AUTO && dtype == DT_BF16) DT_TRY(qkv_fused_one_round(rows, H, &fused));
    float* rms = save_for_backward ? static_cast<float*>(L->rms.ptr) : nullptr;
    float* st_m = save_for_backward ? static_cast<float*>(L->stats.ptr) : nullptr;
    float* st_l = save_for_backward ? st_m + (size_t)rows * H : nullptr;
    const float scale = 1.0f / std::sqrt((float)DT_HEAD_DIM);  // OlmoAttention.cpp:91

    if (dtype == DT_FP32_EXACT) {
        DT_TRY(L->qkv_pre.ensure(act * 3 * 4));
        float* qkv = static_cast<float*>(L->qkv_pre.ptr);
        DT_TRY(L->attn.ensure(act * 4));
        float* attn = static_cast<float*>(L->attn.ptr);
        // the attention input: in place of the projections, or in att32 when the pre-norm projections must
        // survive for the norms' backward
        float* att = qkv;
        if (save_for_backward) {
            DT_TRY(L->att32.ensure(act * 3 * 4));
            att = static_cast<float*>(L->att32.ptr);
        }
        if (fused) {
            // x [Wq;Wk;Wv]^T, q/k norm and RoPE in one kernel (OlmoAttention.cpp:63-88)
            QkvArgs qa{xd, L->w_qkv, L->q_norm, L->k_norm, att, save_for_backward ? qkv : nullptr, rms,
                       ctx->rope_cos, ctx->rope_sin, nullptr, 0, 0, rows, T, H, dm, 3 * dm, 3 * dm, DT_RMS_EPS};
            DT_TRY(run_qkv_fused(ctx, qa, 1, s));
        } else {
            // Q|K|V = x [Wq;Wk;Wv]^T in one N = 3*d_model GEMM (OlmoAttention.cpp:68,74,80)
            DT_TRY(gemm_xwt(ctx, s, rows, 3 * dm, dm, xd, dm, L->w_qkv, dm, qkv, 3 * dm, false));
            // q/k norm + RoPE (OlmoAttention.cpp:70,76,87-88), with V copied beside them into att32
            NormRopeArgs na{qkv, qkv + dm, save_for_backward ? qkv + 2 * dm : nullptr, L->q_norm, L->k_norm, att,
                            att + dm, att + 2 * dm, rms, rms ? rms + rows : nullptr, ctx->rope_cos, ctx->rope_sin,
                            rows, T, H, 3 * dm, 3 * dm, DT_RMS_EPS};
            DT_TRY(launch_qk_norm_rope(na, 0, s));
        }
        FlashArgs fa{att, att + dm, att + 2 * dm, attn, st_m, st_l, B, T, H, 3 * dm, 3 * dm, 3 * dm, dm,
                     scale, 1, seq_lens ? 1 : 0};
        DT_TRY(run_flash(ctx, fa, seq_lens, DT_FP32_EXACT, s));  // OlmoAttention.cpp:94
        DT_TRY(gemm_xwt(ctx, s, rows, dm, dm, attn, dm, L->w_o, dm, od, dm, false));  // :104
    } else {
        if (!L->w_qkv16 || !L->w_o16) {  // (a failed allocation leaves the pair incomplete: retried here)
            if (!L->w_qkv16) DT_HIP_TRY(hipMalloc(&L->w_qkv16, (size_t)3 * dm * dm * 2));
            if (!L->w_o16) DT_HIP_TRY(hipMalloc(&L->w_o16, (size_t)dm * dm * 2));
            L->w16_stale = true;
        }
        if (L->w16_stale) {
            DT_TRY(launch_f32_to_bf16(L->w_qkv, L->w_qkv16, (int64_t)3 * dm * dm, s));
            DT_TRY(launch_f32_to_bf16(L->w_o, L->w_o16, (int64_t)dm * dm, s));
            L->w16_stale = false;
        }
        DT_TRY(L->x16.ensure(act * 2));
        DT_TRY(L->qkv_pre.ensure(act * 3 * 2));
        DT_TRY(L->qkv16.ensure(act * 3 * 2));
        DT_TRY(L->attn.ensure(act * 2));
        uint16_t* x16 = static_cast<uint16_t*>(L->x16.ptr);
        uint16_t* pre16 = static_cast<uint16_t*>(L->qkv_pre.ptr);
        uint16_t* qkv16 = static_cast<uint16_t*>(L->qkv16.ptr);
        uint16_t* attn16 = static_cast<uint16_t*>(L->attn.ptr);
        if (!x16_ready) DT_TRY(launch_f32_to_bf16(xd, x16, (int64_t)act, s));
        if (fused) {
            // x [Wq;Wk;Wv]^T, q/k norm and RoPE in one kernel (OlmoAttention.cpp:63-88); the pre-norm q|k rows
            // (bf16) only when the norms' backward will read them
            QkvArgs qa{x16, L->w_qkv16, L->q_norm, L->k_norm, qkv16, save_for_backward ? pre16 : nullptr, rms,
                       ctx->rope_cos, ctx->rope_sin, nullptr, 0, 0, rows, T, H, dm, 3 * dm, 3 * dm, DT_RMS_EPS};
            DT_TRY(run_qkv_fused(ctx, qa, 0, s));
        } else {
            // the projections leave the GEMM as bf16 (fp32 accumulation, one rounding): the norm kernel reads
            // half the bytes, and the norms' backward reads the same bf16 rows
            DT_TRY(gemm_rm_bf16(ctx, s, false, true, rows, 3 * dm, dm, x16, dm, L->w_qkv16, dm, pre16, 3 * dm));
            NormRopeArgs na{pre16, pre16 + dm, pre16 + 2 * dm, L->q_norm, L->k_norm, qkv16, qkv16 + dm,
                            qkv16 + 2 * dm, rms, rms ? rms + rows : nullptr, ctx->rope_cos, ctx->rope_sin, rows, T, H,
                            3 * dm, 3 * dm, DT_RMS_EPS};
            DT_TRY(launch_qk_norm_rope(na, 1, s, 1));
        }
        FlashArgs fa{qkv16, qkv16 + dm, qkv16 + 2 * dm, attn16, st_m, st_l, B, T, H, 3 * dm, 3 * dm, 3 * dm,
                     dm, scale, 1, seq_lens ? 1 : 0};
        DT_TRY(run_flash(ctx, fa, seq_lens, DT_BF16, s));
        DT_TRY(gemm_xwt(ctx, s, rows, dm, dm, attn16, dm, L->w_o16, dm, od, dm, true));
    }
    if (mem == DT_MEM_HOST) {
        DT_HIP_TRY(hipMemcpyAsync(out, od, act * 4, hipMemcpyDeviceToHost, s));
        DT_HIP_TRY(hipStreamSynchronize(s));
        DT_TRY(qkv_status_check(ctx));
    }
    if (save_for_backward) {
        L->saved_B = B;
        L->saved_T = T;
        L->saved_dtype = dtype;
    }
    return DT_OK;
}

int attn_layer_settle_grads(dt_attn_layer* L, hipStream_t s) {
    if (!L->grad_zero_pending || !L->g_qkv) return DT_OK;
    const int64_t dm = L->d_model;
    DT_TRY(launch_fill_zero(L->g_qkv, 3 * dm * dm, s));
    DT_TRY(launch_fill_zero(L->g_o, dm * dm, s));
    DT_TRY(launch_fill_zero(L->g_qn, dm, s));
    DT_TRY(launch_fill_zero(L->g_kn, dm, s));
    L->grad_zero_pending = false;
    return DT_OK;
}

bool attn_layer_grads_complete(const dt_attn_layer* L) { return L->g_qkv && L->g_o && L->g_qn && L->g_kn; }

void attn_layer_free_grads(dt_attn_layer* L) {
    for (float** p : {&L->g_qkv, &L->g_o, &L->g_qn, &L->g_kn})
        if (*p) {
            (void)hipFree(*p);
            *p = nullptr;
        }
}

// The four gradient buffers exist together or not at all: a failed allocation frees what was allocated, so
// no later call sees g_qkv set with another slot null.
int attn_layer_ensure_grads(dt_attn_layer* L, hipStream_t s) {
    if (attn_layer_grads_complete(L)) return DT_OK;
    attn_layer_free_grads(L);
    const size_t dm = L->d_model;
    auto alloc_all = [&]() -> int {
        DT_HIP_TRY(hipMalloc(&L->g_qkv, 3 * dm * dm * 4));
        DT_HIP_TRY(hipMalloc(&L->g_o, dm * dm * 4));
        DT_HIP_TRY(hipMalloc(&L->g_qn, dm * 4));
        DT_HIP_TRY(hipMalloc(&L->g_kn, dm * 4));
        DT_TRY(launch_fill_zero(L->g_qkv, (int64_t)(3 * dm * dm), s));
        DT_TRY(launch_fill_zero(L->g_o, (int64_t)(dm * dm), s));
        DT_TRY(launch_fill_zero(L->g_qn, (int64_t)dm, s));
        DT_TRY(launch_fill_zero(L->g_kn, (int64_t)dm, s));
        return DT_OK;
    };
    const int rc = alloc_all();
    if (rc != DT_OK) attn_layer_free_grads(L);
    return rc;
}


// `writing` is set once the first gradient buffer is about to be written
// side: the stream the weight gradients' last steps run on (null: s): the GEMMs of dWo and dWqkv and the column
// sums of the q/k norm weights' partial rows. Each starts after the main stream has formed its input (slot
// kEvFork); slot kEvO marks the end of dWo's GEMM, the last reader of d_out on it. The caller joins it back.
static int attn_layer_bwd(dt_attn_layer* L, const float* d_out, const uint16_t* d_out16, float* d_x, int B, int T,
                          int mem, void* stream, hipStream_t side, bool& writing) {
    clear_error();
    if (!d_out || !d_x) return set_error(DT_ERR_INVALID_ARG, "d_out and d_x must be non-NULL");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    if (mem == DT_MEM_DEVICE && (!aligned16(d_out) || !aligned16(d_x)))
        return set_error(DT_ERR_INVALID_ARG, "device d_out/d_x must be 16-byte aligned");
    if (!L) return set_error(DT_ERR_INVALID_ARG, "layer is NULL");
    if (L->saved_T == 0)
        return set_error(DT_ERR_INVALID_ARG, "no saved forward: call dt_attn_layer_fwd with save_for_backward = 1 first");
    if (B != L->saved_B || T != L->saved_T)
        return set_error(DT_ERR_INVALID_ARG, "B=%d, T=%d differ from the saved forward's B=%d, T=%d", B, T, L->saved_B,
                         L->saved_T);
    dt_ctx* ctx = L->ctx;
    DT_TRY(check_device_binding(ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf = L->saved_dtype == DT_BF16;
    const int dm = L->d_model, H = L->n_heads, rows = B * T;
    const size_t act = (size_t)rows * dm;
    const size_t esz = bf ? 2 : 4;
    DT_TRY(attn_layer_ensure_grads(L, s));
    // after zero_grad the gradients are written, not added to (beta = 0: the buffers still hold old values)
    const bool fresh = L->grad_zero_pending;
    const float gb = fresh ? 0.0f : 1.0f;

    const float* gd = d_out;
    float* dxd = d_x;
    if (mem == DT_MEM_HOST) {
        DT_TRY(ctx->stage[0].ensure(act * 4));
        DT_TRY(ctx->stage[1].ensure(act * 4));
        DT_HIP_TRY(hipMemcpyAsync(ctx->stage[0].ptr, d_out, act * 4, hipMemcpyHostToDevice, s));
        gd = static_cast<const float*>(ctx->stage[0].ptr);
        dxd = static_cast<float*>(ctx->stage[1].ptr);
    }
    DT_TRY(L->d_attn32.ensure(act * 4));
    DT_TRY(L->d_qkv.ensure(act * 3 * esz));
    const int nblk = norm_rope_bwd_blocks(rows);
    DT_TRY(L->partial.ensure((size_t)2 * nblk * dm * 4));
    DT_TRY(ctx->bwd_stats.ensure((size_t)2 * rows * H * 4));
    float* d_attn = static_cast<float*>(L->d_attn32.ptr);
    void* dqkv = L->d_qkv.ptr;
    float* bstats = static_cast<float*>(ctx->bwd_stats.ptr);
    const float* st_m = static_cast<const float*>(L->stats.ptr);
    const float* st_l = st_m + (size_t)rows * H;
    const float* rms = static_cast<const float*>(L->rms.ptr);
    const char* pre = static_cast<const char*>(L->qkv_pre.ptr);  // pre-norm Q|K|V, in the mode's dtype
    const float scale = 1.0f / std::sqrt((float)DT_HEAD_DIM);

    // step 1 (OlmoAttention.cpp:198-217): dWo += d_out^T attn; d_attn = d_out Wo
    const void *g_in = gd, *wo = L->w_o, *attn = L->attn.ptr;
    if (bf) {
        DT_TRY(L->d16.ensure(act * 2));
        if (d_out16 && mem == DT_MEM_DEVICE) {
            g_in = d_out16;
        } else {
            DT_TRY(launch_f32_to_bf16(gd, static_cast<uint16_t*>(L->d16.ptr), (int64_t)act, s));
            g_in = L->d16.ptr;
        }
        wo = L->w_o16;
    }
    writing = true;
    if (side) DT_TRY(stream_after(ctx, side, s, kEvFork));
    DT_TRY(gemm_rm(ctx, side ? side : s, true, false, dm, dm, rows, g_in, dm, attn, dm, gb, L->g_o, dm, bf));
    if (side) DT_TRY(stream_mark(ctx, side, kEvO));
    const void* d_o = d_attn;
    if (bf) {  // d_attn leaves the GEMM as bf16 (fp32 accumulation, one rounding): the attention backward is its
               // only reader (in the first half of d_attn32's bytes)
        uint16_t* d_attn16 = reinterpret_cast<uint16_t*>(d_attn);
        DT_TRY(gemm_rm_bf16(ctx, s, false, false, rows, dm, dm, g_in, dm, wo, dm, d_attn16, dm));
        d_o = d_attn16;
    } else {
        DT_TRY(gemm_rm(ctx, s, false, false, rows, dm, dm, g_in, dm, wo, dm, 0.0f, d_attn, dm, false));
    }
    // step 2 (:219-232): the attention core's backward from the saved m and l
    const char* att = static_cast<const char*>(bf ? L->qkv16.ptr : L->att32.ptr);
    char* dq = static_cast<char*>(dqkv);
    FlashBwdArgs ba{att, att + dm * esz, att + 2 * dm * esz, attn, d_o, st_m, st_l, dq, dq + dm * esz,
                    dq + 2 * dm * esz, bstats, bstats + (size_t)rows * H, B, T, H, 3 * dm, dm, 3 * dm, scale, 1};
    DT_TRY(bwd_ds_workspace(ctx, B, H, T, 1, bf ? DT_BF16 : DT_FP32_EXACT, &ba.ds_ws));
    DT_TRY(bf ? launch_flash_bwd_bf16(ba, s) : launch_flash_bwd_f32(ba, s));
    // steps 3-4 (:234-244): RoPE backward and the q/k norms' backward, in place on dq | dk
    NormRopeBwdArgs nb{dq, dq + dm * esz, pre, pre + dm * esz, rms, rms + rows, L->q_norm, L->k_norm,
                       static_cast<float*>(L->partial.ptr), ctx->rope_cos, ctx->rope_sin, rows, T, H, 3 * dm, 3 * dm};
    DT_TRY(launch_qk_norm_rope_bwd(nb, bf, side ? nullptr : L->g_qn, side ? nullptr : L->g_kn, s, !fresh));
    if (side) {
        DT_TRY(stream_after(ctx, side, s, kEvFork));
        DT_TRY(launch_colsum(nb.partial, nblk, dm, L->g_qn, side, !fresh, L->g_kn));
    }
    // step 5 (:246-309): [dWq;dWk;dWv] += [dq|dk|dv]^T x and d_x = [dq|dk|dv] [Wq;Wk;Wv]
    const void* xin = bf ? L->x16.ptr : L->x32.ptr;
    const void* wqkv = bf ? static_cast<const void*>(L->w_qkv16) : static_cast<const void*>(L->w_qkv);
    DT_TRY(gemm_rm(ctx, side ? side : s, true, false, 3 * dm, dm, rows, dqkv, 3 * dm, xin, dm, gb, L->g_qkv, dm, bf));
    L->grad_zero_pending = false;  // every gradient buffer has been written
    DT_TRY(gemm_rm(ctx, s, false, false, rows, dm, 3 * dm, dqkv, 3 * dm, wqkv, dm, 0.0f, dxd, dm, bf));
    if (mem == DT_MEM_HOST) {
        if (side) DT_TRY(stream_after(ctx, s, side, kEvJoin));
        DT_HIP_TRY(hipMemcpyAsync(d_x, dxd, act * 4, hipMemcpyDeviceToHost, s));
        DT_HIP_TRY(hipStreamSynchronize(s));
    }
    return DT_OK;
}

int attn_layer_step_mats(dt_attn_layer* L, float lr, hipStream_t s) {
    DT_TRY(attn_layer_ensure_grads(L, s));
    DT_TRY(attn_layer_settle_grads(L, s));
    const int64_t dm = L->d_model;
    // the bf16 copies (once the bf16 mode has made them) are rewritten from the updated weights in the
    // same pass, so they are current afterwards
    const bool copies = L->w_qkv16 && L->w_o16;
    DT_TRY(launch_sgd(L->w_qkv, L->g_qkv, lr, 3 * dm * dm, s, copies ? L->w_qkv16 : nullptr));  // OlmoAttention.cpp:315-317
    DT_TRY(launch_sgd(L->w_o, L->g_o, lr, dm * dm, s, copies ? L->w_o16 : nullptr));            // :318
    L->w16_stale = !copies;
    return DT_OK;
}

int attn_layer_bwd_dev(dt_attn_layer* L, const float* d_out, const uint16_t* d_out16, float* d_x, int B, int T,
                       void* stream, hipStream_t side) {
    bool writing = false;
    const int rc = attn_layer_bwd(L, d_out, d_out16, d_x, B, T, DT_MEM_DEVICE, stream, side, writing);
    if (rc != DT_OK && writing && L->grad_zero_pending) {
        if (side) (void)stream_after(L->ctx, static_cast<hipStream_t>(stream), side, kEvJoin);
        (void)attn_layer_settle_grads(L, static_cast<hipStream_t>(stream));
    }
    return rc;
}

extern "C" {

int dt_attn_layer_bwd(dt_attn_layer* L, const float* d_out, float* d_x, int B, int T, int mem, void* stream) {
    // one stream: a lone layer has no later work for its weight-gradient GEMMs to run beside (on the side stream
    // they measured slower, T = 512 and 2048); the model backward gives them the next block's
    bool writing = false;
    const int rc = attn_layer_bwd(L, d_out, nullptr, d_x, B, T, mem, stream, nullptr, writing);
    // a backward that failed after zero_grad, once it had begun writing gradients, may have written some of them:
    // clear them all, so that they read as the zero_grad left them (the error stays the one reported)
    if (rc != DT_OK && writing && L->grad_zero_pending) (void)attn_layer_settle_grads(L, static_cast<hipStream_t>(stream));
    return rc;
}

int dt_attn_layer_step(dt_attn_layer* L, float lr, void* stream) {
    clear_error();
    if (!L) return set_error(DT_ERR_INVALID_ARG, "layer is NULL");
    if (!std::isfinite(lr)) return set_error(DT_ERR_INVALID_ARG, "lr must be finite");
    DT_TRY(check_device_binding(L->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    DT_TRY(attn_layer_step_mats(L, lr, s));
    // :319-320, RMSNorm.cpp:38-40: both norm weights in one launch
    float* w[2] = {L->q_norm, L->k_norm};
    const float* g[2] = {L->g_qn, L->g_kn};
    const int n[2] = {L->d_model, L->d_model};
    return launch_sgd_vecs(w, g, n, 2, lr, s);
}

int dt_attn_layer_zero_grad(dt_attn_layer* L, void* stream) {
    clear_error();
    if (!L) return set_error(DT_ERR_INVALID_ARG, "layer is NULL");
    DT_TRY(check_device_binding(L->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!L->g_qkv) return attn_layer_ensure_grads(L, s);  // allocated zeroed
    // OlmoAttention.cpp:323-330, deferred: the next backward overwrites the gradients instead of adding to them,
    // which saves writing zeros over every buffer and the GEMMs' reads of them; step and the parameter
    // copies clear the buffers first when no backward came in between
    L->grad_zero_pending = true;
    return DT_OK;
}

// copies the six parameter arrays (grads == 0) or their gradients (grads == 1) out of the layer
static int copy_params(dt_attn_layer* L, int grads, float* wq, float* wk, float* wv, float* wo, float* qn, float* kn,
                       int mem, void* stream) {
    clear_error();
    if (!L) return set_error(DT_ERR_INVALID_ARG, "layer is NULL");
    if (mem != DT_MEM_DEVICE && mem != DT_MEM_HOST) return set_error(DT_ERR_INVALID_ARG, "unknown mem %d", mem);
    DT_TRY(check_device_binding(L->ctx));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (grads) {
        DT_TRY(attn_layer_ensure_grads(L, s));
        DT_TRY(attn_layer_settle_grads(L, s));
    }
    const size_t dm = L->d_model, w2 = dm * dm * 4;
    const float* src_qkv = grads ? L->g_qkv : L->w_qkv;
    const float* srcs[6] = {src_qkv, src_qkv + dm * dm, src_qkv + 2 * dm * dm, grads ? L->g_o : L->w_o,
                            grads ? L->g_qn : L->q_norm, grads ? L->g_kn : L->k_norm};
    float* dsts[6] = {wq, wk, wv, wo, qn, kn};
    const size_t bytes[6] = {w2, w2, w2, w2, dm * 4, dm * 4};
    const hipMemcpyKind kind = mem == DT_MEM_HOST ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    for (int i = 0; i < 6; ++i)
        if (dsts[i]) DT_HIP_TRY(hipMemcpyAsync(dsts[i], srcs[i], bytes[i], kind, s));
    if (mem == DT_MEM_HOST) DT_HIP_TRY(hipStreamSynchronize(s));
    return DT_OK;
}

int dt_attn_layer_get_weights(dt_attn_layer* L, float* wq, float* wk, float* wv, float* wo, float* q_norm_w,
                              float* k_norm_w, int mem, void* stream) {
    return copy_params(L, 0, wq, wk, wv, wo, q_norm_w, k_norm_w, mem, stream);
}

int dt_attn_layer_get_grads(dt_attn_layer* L, float* d_wq, float* d_wk, float* d_wv, float* d_wo, float* d_q_norm_w,
                            float* d_k_norm_w, int mem, void* stream) {
    return copy_params(L, 1, d_wq, d_wk, d_wv, d_wo, d_q_norm_w, d_k_norm_w, mem, stream);
}

}  // extern "C"
