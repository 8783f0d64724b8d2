// Backward of the fused q/k RMSNorm + RoPE, and the layer's parameter updates, for gfx950.
//
// qk_norm_rope_bwd replaces, for the q and k branches of
// OlmoAttention::backward (OlmoAttention.cpp:234-244), apply_rope_backward
// (OlmoAttention.cpp:149-190) followed by RMSNorm::backward (RMSNorm.cpp:24-36):
//   g_n[d]    =  g[d] cos[t,d] + g[d+64] sin[t,d]        (transpose of the rotation)
//   g_n[d+64] = -g[d] sin[t,d] + g[d+64] cos[t,d]
//   n = x / rms (the forward's normalised row), c = mean over the row of g_n * n * w
//   dx = (w * g_n - n * c) / rms,   dw += sum over rows of g_n * n
// with x the saved pre-norm projection and rms the forward's saved rms. The
// reference recomputes n as y / w from the saved output y (RMSNorm.cpp:29);
// x / rms is the same quantity without the division by w.
// The gradient g arrives in the attention-core dtype (fp32 or bf16) inside the
// [rows][3*d_model] dq|dk|dv buffer and dx is written back in place; the saved
// x is in the same dtype (the bf16 layer path keeps its pre-norm projections as
// the bf16 output of the QKV GEMM).
//
// dw is reduced deterministically: a workgroup handles a fixed number of rows
// (norm_rope_bwd_rows: up to kMaxRows, fewer for short inputs, so that the
// grid still has two workgroups per CU) and writes one partial row of column
// sums; launch_colsum adds the partials, in a fixed order, into the gradient
// (the reference's `+=`, RMSNorm.cpp:31).
//
// One workgroup of 256 threads per row block of q (blockIdx.y == 0) or k (== 1);
// thread t owns dims [4*(t%16), +4) and [4*(t%16)+64, +4) of heads t/16,
// t/16 + 16, ..., so both halves of each rotate-half pair sit in one thread.
// HBM bound: per row it reads g, x (twice, the second time mostly from L2)
// and writes dx.

#include <algorithm>

#include "dt_internal.h"

namespace dt {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

constexpr int kMaxRows = 16;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

template <bool kBF16>
__device__ __forceinline__ float4 load4(const void* base, int64_t idx) {
    if constexpr (kBF16) {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
        return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
    } else {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    }
}
template <bool kBF16>
__device__ __forceinline__ void store4(void* base, int64_t idx, float4 v) {
    if constexpr (kBF16) {
        uint2 w;
        w.x = pack_bf16x2(v.x, v.y);
        w.y = pack_bf16x2(v.z, v.w);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx) = w;
    } else {
        *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = v;
    }
}

// g_n for one rotate-half pair block: (a, b) = rows d and d+64 of g
__device__ __forceinline__ void rope_back(const float4& a, const float4& b, const float4& c, const float4& s, float (&n0)[4],
                                          float (&n1)[4]) {
    const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
    const float cv[4] = {c.x, c.y, c.z, c.w}, sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        n0[e] = av[e] * cv[e] + bv[e] * sv[e];
        n1[e] = -av[e] * sv[e] + bv[e] * cv[e];
    }
}

template <bool kBF16>
__global__ __launch_bounds__(256) void qk_norm_rope_bwd_kernel(NormRopeBwdArgs a, int rpb) {
    __shared__ float red[kMaxRows][4];
    const int which = blockIdx.y;
    const int r0 = blockIdx.x * rpb;
    const int tid = threadIdx.x;
    const int head = tid >> 4;
    const int d0 = 4 * (tid & 15);
    const int C = a.H * 128;
    const int nr = min(rpb, a.rows - r0);

    void* g = which == 0 ? a.dq : a.dk;
    const void* x = which == 0 ? a.q_x : a.k_x;
    const float* rms = which == 0 ? a.q_rms : a.k_rms;
    const float* w = which == 0 ? a.q_w : a.k_w;

    // pass 1: per row, s = sum over the row of g_n * n * w
    for (int i = 0; i < nr; ++i) {
        const int row = r0 + i;
        const int t = row % a.T;
        const float inv = 1.0f / rms[row];
        const float4 c4 = *reinterpret_cast<const float4*>(a.rope_cos + (int64_t)t * 64 + d0);
        const float4 s4 = *reinterpret_cast<const float4*>(a.rope_sin + (int64_t)t * 64 + d0);
        float acc = 0.0f;
        for (int hx = head; hx < a.H; hx += 16) {
            const int64_t gi = (int64_t)row * a.ld_d + hx * 128 + d0;
            const int64_t xi = (int64_t)row * a.ld_x + hx * 128 + d0;
            float n0[4], n1[4];
            rope_back(load4<kBF16>(g, gi), load4<kBF16>(g, gi + 64), c4, s4, n0, n1);
            const float4 x0 = load4<kBF16>(x, xi);
            const float4 x1 = load4<kBF16>(x, xi + 64);
            const float4 w0 = *reinterpret_cast<const float4*>(w + hx * 128 + d0);
            const float4 w1 = *reinterpret_cast<const float4*>(w + hx * 128 + d0 + 64);
            acc += n0[0] * (x0.x * inv) * w0.x + n0[1] * (x0.y * inv) * w0.y + n0[2] * (x0.z * inv) * w0.z +
                   n0[3] * (x0.w * inv) * w0.w + n1[0] * (x1.x * inv) * w1.x + n1[1] * (x1.y * inv) * w1.y +
                   n1[2] * (x1.z * inv) * w1.z + n1[3] * (x1.w * inv) * w1.w;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
        if ((tid & 63) == 0) red[i][tid >> 6] = acc;
    }
    __syncthreads();

    // pass 2: dx in place, and this workgroup's column sums of g_n * n
    float* part = a.partial + ((int64_t)which * gridDim.x + blockIdx.x) * C;
    for (int hx = head; hx < a.H; hx += 16) {
        float p0[4] = {0.f, 0.f, 0.f, 0.f}, p1[4] = {0.f, 0.f, 0.f, 0.f};
        const float4 w0 = *reinterpret_cast<const float4*>(w + hx * 128 + d0);
        const float4 w1 = *reinterpret_cast<const float4*>(w + hx * 128 + d0 + 64);
        const float wv0[4] = {w0.x, w0.y, w0.z, w0.w}, wv1[4] = {w1.x, w1.y, w1.z, w1.w};
        for (int i = 0; i < nr; ++i) {
            const int row = r0 + i;
            const int t = row % a.T;
            const float inv = 1.0f / rms[row];
            const float cm = (red[i][0] + red[i][1] + red[i][2] + red[i][3]) / (float)C;
            const float4 c4 = *reinterpret_cast<const float4*>(a.rope_cos + (int64_t)t * 64 + d0);
            const float4 s4 = *reinterpret_cast<const float4*>(a.rope_sin + (int64_t)t * 64 + d0);
            const int64_t gi = (int64_t)row * a.ld_d + hx * 128 + d0;
            const int64_t xi = (int64_t)row * a.ld_x + hx * 128 + d0;
            float n0[4], n1[4];
            rope_back(load4<kBF16>(g, gi), load4<kBF16>(g, gi + 64), c4, s4, n0, n1);
            const float4 x0 = load4<kBF16>(x, xi);
            const float4 x1 = load4<kBF16>(x, xi + 64);
            const float xv0[4] = {x0.x * inv, x0.y * inv, x0.z * inv, x0.w * inv};
            const float xv1[4] = {x1.x * inv, x1.y * inv, x1.z * inv, x1.w * inv};
            float o0[4], o1[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o0[e] = (wv0[e] * n0[e] - xv0[e] * cm) * inv;
                o1[e] = (wv1[e] * n1[e] - xv1[e] * cm) * inv;
                p0[e] += n0[e] * xv0[e];
                p1[e] += n1[e] * xv1[e];
            }
            store4<kBF16>(g, gi, make_float4(o0[0], o0[1], o0[2], o0[3]));
            store4<kBF16>(g, gi + 64, make_float4(o1[0], o1[1], o1[2], o1[3]));
        }
        *reinterpret_cast<float4*>(part + hx * 128 + d0) = make_float4(p0[0], p0[1], p0[2], p0[3]);
        *reinterpret_cast<float4*>(part + hx * 128 + d0 + 64) = make_float4(p1[0], p1[1], p1[2], p1[3]);
    }
}

// grad_q[j] += sum_b partial[0][b][j], grad_k[j] += sum_b partial[1][b][j], in block order

// w -= lr * g (OlmoAttention.cpp:314-321, RMSNorm.cpp:38-40), rounded as written: the product, then the
// difference (no fused multiply-add), so the update is reproducible on the host
__global__ __launch_bounds__(256) void sgd_kernel(float* w, const float* g, float lr, int64_t n) {
#pragma clang fp contract(off)
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float step = lr * g[i];
        w[i] = w[i] - step;
    }
}

// The same update four elements per thread and step (w, g 16-byte aligned, n4 = n / 4 groups), with the
// updated weights also written as bf16 (round to nearest even, as f32_to_bf16) into w16 when it is not
// NULL: the copy the bf16 GEMMs read is refreshed in the same pass instead of by a second read of w.
__global__ __launch_bounds__(256) void sgd4_kernel(float4* w, const float4* g, float lr, int64_t n4, uint2* w16) {
#pragma clang fp contract(off)
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float4 gv = g[i];
        float4 wv = w[i];
        wv.x = wv.x - lr * gv.x;
        wv.y = wv.y - lr * gv.y;
        wv.z = wv.z - lr * gv.z;
        wv.w = wv.w - lr * gv.w;
        w[i] = wv;
        if (w16) w16[i] = make_uint2(pack_bf16x2(wv.x, wv.y), pack_bf16x2(wv.z, wv.w));
    }
}

// sgd_kernel's update over several short vectors, workgroup b taking vector b
constexpr int kMaxSgdVecs = 96;
struct SgdVecs {
    float* w[kMaxSgdVecs];
    const float* g[kMaxSgdVecs];
    int n[kMaxSgdVecs];
};
__global__ __launch_bounds__(256) void sgd_vecs_kernel(SgdVecs v, float lr) {
#pragma clang fp contract(off)
    float* w = v.w[blockIdx.x];
    const float* g = v.g[blockIdx.x];
    const int n = v.n[blockIdx.x];
    for (int i = threadIdx.x; i < n; i += 256) {
        const float step = lr * g[i];
        w[i] = w[i] - step;
    }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.0f;
}

unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

}  // namespace

// rows per workgroup: kMaxRows, or the power of two that still gives the q and k grids 512 workgroups
// together (two per CU); a function of the row count only, so the summation order is fixed per shape
static int norm_rope_bwd_rows(int rows) {
    int r = 1;
    while (2 * r <= kMaxRows && 2 * r * 256 <= rows) r *= 2;
    return r;
}
int norm_rope_bwd_blocks(int rows) {
    const int r = norm_rope_bwd_rows(rows);
    return (rows + r - 1) / r;
}

int launch_qk_norm_rope_bwd(const NormRopeBwdArgs& a, int bf16, float* grad_q_w, float* grad_k_w,
                            hipStream_t stream, bool accumulate) {
    const int nblk = norm_rope_bwd_blocks(a.rows);
    const int rpb = norm_rope_bwd_rows(a.rows);
    dim3 grid(nblk, 2);
    if (bf16) hipLaunchKernelGGL(qk_norm_rope_bwd_kernel<true>, grid, dim3(256), 0, stream, a, rpb);
    else hipLaunchKernelGGL(qk_norm_rope_bwd_kernel<false>, grid, dim3(256), 0, stream, a, rpb);
    DT_HIP_TRY(hipGetLastError());
    if (!grad_q_w && !grad_k_w) return DT_OK;  // the caller sums the partial rows itself
    const int C = a.H * 128;  // partial: [q, k][nblk][C]
    return launch_colsum(a.partial, nblk, C, grad_q_w, stream, accumulate, grad_k_w);
}

int launch_sgd(float* w, const float* g, float lr, int64_t n, hipStream_t stream, uint16_t* w16) {
    const bool vec = n % 4 == 0 && ((uintptr_t)w | (uintptr_t)g | (uintptr_t)w16) % 16 == 0;
    if (vec) {
        hipLaunchKernelGGL(sgd4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, stream, reinterpret_cast<float4*>(w),
                           reinterpret_cast<const float4*>(g), lr, n / 4, reinterpret_cast<uint2*>(w16));
    } else {
        hipLaunchKernelGGL(sgd_kernel, dim3(grid_for(n)), dim3(256), 0, stream, w, g, lr, n);
        DT_HIP_TRY(hipGetLastError());
        if (w16) return launch_f32_to_bf16(w, w16, n, stream);
    }
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_sgd_vecs(float* const* w, const float* const* g, const int* n, int count, float lr, hipStream_t stream) {
    for (int b0 = 0; b0 < count; b0 += kMaxSgdVecs) {
        SgdVecs v{};
        const int c = std::min(count - b0, kMaxSgdVecs);
        for (int i = 0; i < c; ++i) {
            v.w[i] = w[b0 + i];
            v.g[i] = g[b0 + i];
            v.n[i] = n[b0 + i];
        }
        hipLaunchKernelGGL(sgd_vecs_kernel, dim3(c), dim3(256), 0, stream, v, lr);
        DT_HIP_TRY(hipGetLastError());
    }
    return DT_OK;
}

int launch_fill_zero(float* p, int64_t n, hipStream_t stream) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n)), dim3(256), 0, stream, p, n);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
