// Row statistics for the attention-core backward, both modes.
//
// flash_attention_backward (FlashAttention.cpp:185-359) needs, per query row,
// D = O . dO (:232-238) and the forward's m and l to rebuild
// P = exp(s - m) / l (:260-275). This kernel computes them once per row, in
// the form the backward kernels consume:
//   delta[b][h][t] = sum_d O[b,t,h,d] * dO[b,t,h,d]            (fp32)
//   lse2[b][h][t]  = m[b,t,h] * log2(e) + log2(l[b,t,h])        (fp32)
// so that P = exp2(s_raw * scale * log2(e) - lse2) with s_raw = q . k. A row
// with l == 0 (the reference's empty row, FlashAttention.cpp:165-174) gets
// lse2 = +inf and so P = 0. The [b][h][t] layout makes the 64 rows of one
// tile a contiguous 256-byte run for the backward kernels' LDS DMA.
//
// HBM bound: 2 * 128 elements read and 8 bytes written per row.

#include "dt_internal.h"

namespace dt {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// 16 lanes per row, 8 elements per lane; 16 rows per 256-thread block
template <bool kBf16>
__global__ __launch_bounds__(256) void flash_bwd_prep_kernel(FlashBwdArgs a, int64_t n_rows) {
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // = (b*T + t)*H + h
    const int part = threadIdx.x & 15;
    float acc = 0.0f;
    if (row < n_rows) {
        const int64_t bt = row / a.H;
        const int h = (int)(row - bt * a.H);
        const int64_t off = bt * a.ld_o + (int64_t)h * 128 + 8 * part;
        if (kBf16) {
            const uint4 o = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.o) + off);
            const uint4 g = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.d_o) + off);
            const uint32_t ow[4] = {o.x, o.y, o.z, o.w}, gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) acc += bf16_lo(ow[e]) * bf16_lo(gw[e]) + bf16_hi(ow[e]) * bf16_hi(gw[e]);
        } else {
            const float4* op = reinterpret_cast<const float4*>(static_cast<const float*>(a.o) + off);
            const float4* gp = reinterpret_cast<const float4*>(static_cast<const float*>(a.d_o) + off);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 o = op[j], g = gp[j];
                acc += o.x * g.x + o.y * g.y + o.z * g.z + o.w * g.w;
            }
        }
    }
#pragma unroll
    for (int s = 8; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 16);
    if (row < n_rows && part == 0) {
        const int64_t bt = row / a.H;
        const int h = (int)(row - bt * a.H);
        const int64_t b = bt / a.T;
        const int t = (int)(bt - b * a.T);
        const int64_t dst = (b * a.H + h) * a.T + t;
        const float l = a.l[row];
        a.delta[dst] = acc;
        a.lse2[dst] = l > 0.0f ? a.m[row] * kLog2e + __log2f(l) : __builtin_huge_valf();
    }
}

}  // namespace

int launch_flash_bwd_prep(const FlashBwdArgs& a, int bf16, hipStream_t stream) {
    const int64_t n_rows = (int64_t)a.B * a.T * a.H;
    const int64_t blocks = (n_rows + 15) / 16;
    if (blocks > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many rows");
    if (bf16)
        hipLaunchKernelGGL(flash_bwd_prep_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a, n_rows);
    else
        hipLaunchKernelGGL(flash_bwd_prep_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a, n_rows);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
