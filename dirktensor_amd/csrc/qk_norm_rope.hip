// Fused q/k RMSNorm + RoPE for gfx950.
//
// Replaces, for one token row, RMSNorm::forward on the q and k projections
// (RMSNorm.cpp:15-22, called at OlmoAttention.cpp:70,76; the norm spans all
// d_model = H*D features, not one head) followed by apply_rope
// (OlmoAttention.cpp:111-146, rotate-half pairs (d, d+64), position = t).
//
// One workgroup of 256 threads handles one row of q (blockIdx.y == 0), of k
// (== 1) or, when v_in is set, converts one row of v (== 2). Thread t
// owns dims [4*(t%16), +4) and [4*(t%16)+64, +4) of head t/16, so both halves
// of each rotate-half pair sit in the same thread. HBM-bound: per row it reads
// d_model inputs (fp32, or in the bf16 layer path the bf16 output of the QKV
// GEMM) and writes d_model outputs (fp32 or bf16); the sin/cos tables are
// [rope_len][64] fp32 (the reference's [rope_len][128] tables repeat the same
// angles in both halves, OlmoAttention.cpp:24, so one half is exact).
//
// Rounding follows the reference's expression order: rms = sqrt(ss / C + eps),
// y = (x / rms) * w, out[d] = y[d] cos - y[d+64] sin, out[d+64] = y[d+64] cos + y[d] sin.

#include "dt_internal.h"

namespace dt {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

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

// kIn16: inputs are bf16; kBF16: outputs are bf16
template <bool kIn16, bool kBF16>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeArgs a) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const int which = blockIdx.y;
    const int tid = threadIdx.x;
    const int head = tid >> 4;
    const int d0 = 4 * (tid & 15);
    const int C = a.H * 128;

    if (which == 2) {  // v: plain conversion of the row
        for (int i = 4 * tid; i < C; i += 4 * 256)
            store4<kBF16>(a.v_out, (int64_t)row * a.ld_out + i, load4<kIn16>(a.v_in, (int64_t)row * a.ld_in + i));
        return;
    }

    const void* src = which == 0 ? a.q_in : a.k_in;
    const int64_t rb = (int64_t)row * a.ld_in;
    const float* w = which == 0 ? a.q_w : a.k_w;
    void* dst = which == 0 ? a.q_out : a.k_out;
    float* rms_out = which == 0 ? a.q_rms : a.k_rms;
    const int t = row % a.T;

    const bool active = head < a.H;
    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
    if (active) {
        x0 = load4<kIn16>(src, rb + head * 128 + d0);
        x1 = load4<kIn16>(src, rb + head * 128 + d0 + 64);
    }
    float ss = x0.x * x0.x + x0.y * x0.y + x0.z * x0.z + x0.w * x0.w + x1.x * x1.x + x1.y * x1.y + x1.z * x1.z +
               x1.w * x1.w;
    // handle rows wider than one workgroup pass (H > 16)
    for (int hx = head + 16; hx < a.H; hx += 16) {
        const float4 y0 = load4<kIn16>(src, rb + hx * 128 + d0);
        const float4 y1 = load4<kIn16>(src, rb + hx * 128 + d0 + 64);
        ss += y0.x * y0.x + y0.y * y0.y + y0.z * y0.z + y0.w * y0.w + y1.x * y1.x + y1.y * y1.y + y1.z * y1.z +
              y1.w * y1.w;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float rms = sqrtf(ss / (float)C + a.eps);
    if (rms_out && tid == 0) rms_out[row] = rms;

    const float* cs = a.rope_cos + (int64_t)t * 64 + d0;
    const float* sn = a.rope_sin + (int64_t)t * 64 + d0;
    const float4 c4 = *reinterpret_cast<const float4*>(cs);
    const float4 s4 = *reinterpret_cast<const float4*>(sn);
    for (int hx = head; hx < a.H; hx += 16) {
        float4 u0 = x0, u1 = x1;
        if (hx != head) {
            u0 = load4<kIn16>(src, rb + hx * 128 + d0);
            u1 = load4<kIn16>(src, rb + hx * 128 + d0 + 64);
        }
        const float4 w0 = *reinterpret_cast<const float4*>(&w[hx * 128 + d0]);
        const float4 w1 = *reinterpret_cast<const float4*>(&w[hx * 128 + d0 + 64]);
        const float y0[4] = {(u0.x / rms) * w0.x, (u0.y / rms) * w0.y, (u0.z / rms) * w0.z, (u0.w / rms) * w0.w};
        const float y1[4] = {(u1.x / rms) * w1.x, (u1.y / rms) * w1.y, (u1.z / rms) * w1.z, (u1.w / rms) * w1.w};
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
        float r0[4], r1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r0[e] = y0[e] * cv[e] - y1[e] * sv[e];
            r1[e] = y1[e] * cv[e] + y0[e] * sv[e];
        }
        const int64_t ob = (int64_t)row * a.ld_out + hx * 128 + d0;
        store4<kBF16>(dst, ob, make_float4(r0[0], r0[1], r0[2], r0[3]));
        store4<kBF16>(dst, ob + 64, make_float4(r1[0], r1[1], r1[2], r1[3]));
    }
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* in, uint16_t* out, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float4 v = reinterpret_cast<const float4*>(in)[i];
        uint2 w;
        w.x = pack_bf16x2(v.x, v.y);
        w.y = pack_bf16x2(v.z, v.w);
        reinterpret_cast<uint2*>(out)[i] = w;
    }
}

}  // namespace

int launch_qk_norm_rope(const NormRopeArgs& a, int out_bf16, hipStream_t stream, int in_bf16) {
    dim3 grid(a.rows, a.v_in ? 3 : 2);
    if (in_bf16 && !out_bf16) return set_error(DT_ERR_INVALID_ARG, "qk_norm_rope: bf16 input needs bf16 output");
    if (in_bf16) hipLaunchKernelGGL((qk_norm_rope_kernel<true, true>), grid, dim3(256), 0, stream, a);
    else if (out_bf16) hipLaunchKernelGGL((qk_norm_rope_kernel<false, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((qk_norm_rope_kernel<false, false>), grid, dim3(256), 0, stream, a);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream) {
    const int64_t n4 = n / 4;  // callers pass multiples of 4
    int64_t blocks = (n4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, in, out, n4);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
