// Causal flash attention backward, fp32 exact mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_backward (FlashAttention.cpp:185-359) with fp32
// tensors and fp32 MFMA (v_mfma_f32_32x32x2_f32) products.
//
// Same decomposition as the bf16 mode: flash_bwd_dkdv_f32 owns 128 keys of one
// (batch, head) per workgroup (32 per wave, K and V rows in registers) and
// streams 64-query tiles of Q, dO, lse2 and delta; flash_bwd_dq_f32 owns 128
// queries (Q and dO rows in registers) and streams 64-key tiles of K and V.
// Each gradient row has a single owner, so no atomics; S and dP are computed
// in both kernels. Block j and block n-1-j of a head share a workgroup.
//
// v_mfma_f32_32x32x2_f32 takes one A value per lane (row l%32, k = l/32) and
// one B value (column l%32, k = l/32). For the products over the head
// dimension, k step s of lane half hh is dim 64*hh + s, so a lane's register
// operand is half of one row (64 floats) and its LDS operand is read four
// steps at a time as a float4. For the products over queries (dK/dV) or keys
// (dQ), the B operand is an accumulator element: step (blk, i) pairs k = hh
// with row 32*blk + 8*(i/4) + 4*hh + i%4, the accumulator layout, and the A
// operand is one float of that row read from LDS.
//
// Tiles are staged through registers: the next tile's global loads are issued
// before the current tile's products and written to LDS after them (two
// barriers per tile). LDS rows are padded to 132 floats.

#include "dt_internal.h"

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kTile = 64;
constexpr int kLd = 132;  // LDS row stride (floats)
constexpr int kBlk = 128;
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ floatx16 mfma(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 zero16() {
    floatx16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

// A 64 x 128 fp32 tile in flight: thread tid holds rows tid/32 + 8*j (j < 8), floats 4*(tid%32) .. +3
struct TileRegs {
    float4 v[8];
};
__device__ __forceinline__ void tile_load(TileRegs& R, const float* base, int r0, int T, int ld, int tid) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = r0 + (tid >> 5) + 8 * j;
        R.v[j] = r < T ? *reinterpret_cast<const float4*>(base + (int64_t)r * ld + 4 * (tid & 31))
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}
__device__ __forceinline__ void tile_store(float* lds, const TileRegs& R, int tid) {
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<float4*>(lds + ((tid >> 5) + 8 * j) * kLd + 4 * (tid & 31)) = R.v[j];
}
// one row half from global memory: f[s] = X[row][64*hh + s], zeros when row >= T
__device__ __forceinline__ void load_half_row(float (&f)[64], const float* base, int row, int T, int ld, int hh) {
    if (row < T) {
        const float4* p = reinterpret_cast<const float4*>(base + (int64_t)row * ld + 64 * hh);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float4 x = p[j];
            f[4 * j] = x.x;
            f[4 * j + 1] = x.y;
            f[4 * j + 2] = x.z;
            f[4 * j + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < 64; ++s) f[s] = 0.0f;
    }
}
// C[32 rows of block blk] += X[rows][64*hh + s] * f[s] over s: the product over the head dimension with
// the LDS tile's rows as M and a register row half as the B operand
__device__ __forceinline__ floatx16 dot_rows(const float* tile, int blk, int ln, int hh, const float (&f)[64]) {
    floatx16 acc = zero16();
    const float* row = tile + (32 * blk + ln) * kLd + 64 * hh;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float4 x = *reinterpret_cast<const float4*>(row + 4 * j);
        acc = mfma(x.x, f[4 * j], acc);
        acc = mfma(x.y, f[4 * j + 1], acc);
        acc = mfma(x.z, f[4 * j + 2], acc);
        acc = mfma(x.w, f[4 * j + 3], acc);
    }
    return acc;
}
// acc[db] += sum over the 64 tile rows of tile[row][32*db + ln] * w[blk][i], row = 32*blk + 8*(i/4) + 4*hh + i%4
__device__ __forceinline__ void acc_cols(floatx16 (&acc)[4], const float* tile, int ln, int hh, const floatx16 (&w)[2]) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float* row = tile + (32 * blk + 8 * (i / 4) + 4 * hh + (i % 4)) * kLd + ln;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = mfma(row[32 * db], w[blk][i], acc[db]);
        }
}
// accumulator X^T (4 blocks of 32 dims x 32 rows, lane = row) * mul -> row `row` of [T][ld] at base
__device__ __forceinline__ void store_rows(float* base, int row, int ld, int hh, const floatx16 (&x)[4], float mul) {
    float* p = base + (int64_t)row * ld;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4*>(p + 32 * db + 8 * g + 4 * hh) =
                make_float4(x[db][4 * g] * mul, x[db][4 * g + 1] * mul, x[db][4 * g + 2] * mul, x[db][4 * g + 3] * mul);
}

// ------------------------------------------------------------------------------------------------ dK, dV
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dkdv_f32_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(16))) float Qs[kTile * kLd];
    __shared__ __attribute__((aligned(16))) float Gs[kTile * kLd];
    __shared__ __attribute__((aligned(16))) float Ls[kTile];
    __shared__ __attribute__((aligned(16))) float Ds[kTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int nkb = (T + kBlk - 1) / kBlk;
    const int npair = (nkb + 1) / 2;
    const int pair = blockIdx.x % npair;
    const int bh = blockIdx.x / npair;
    const int b = bh / a.H, h = bh % a.H;

    const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Gg = static_cast<const float*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    const float* lse2g = a.lse2 + (int64_t)bh * T;
    const float* deltag = a.delta + (int64_t)bh * T;
    float* dKg = static_cast<float*>(a.d_k) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;
    float* dVg = static_cast<float*>(a.d_v) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    for (int half = 0; half < 2; ++half) {
        const int kb = half ? nkb - 1 - pair : pair;
        if (half && kb == pair) break;
        const int kw = kb * kBlk + 32 * wave;
        const int key = kw + ln;

        float kf[64], vf[64];
        load_half_row(kf, Kg, key, T, a.ld_qkv, hh);
        load_half_row(vf, Vg, key, T, a.ld_qkv, hh);
        floatx16 dv[4], dk[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            dv[db] = zero16();
            dk[db] = zero16();
        }

        const int q_begin = a.causal ? kb * kBlk : 0;
        const int n_steps = (T - q_begin + kTile - 1) / kTile;
        TileRegs rq, rg;
        float rl = 0.0f, rd = 0.0f;
        auto fetch = [&](int q0) {
            tile_load(rq, Qg, q0, T, a.ld_qkv, tid);
            tile_load(rg, Gg, q0, T, a.ld_o, tid);
            if (tid < kTile) {
                rl = q0 + tid < T ? lse2g[q0 + tid] : 0.0f;
                rd = q0 + tid < T ? deltag[q0 + tid] : 0.0f;
            }
        };
        auto commit = [&]() {
            tile_store(Qs, rq, tid);
            tile_store(Gs, rg, tid);
            if (tid < kTile) {
                Ls[tid] = rl;
                Ds[tid] = rd;
            }
        };
        fetch(q_begin);
        __syncthreads();  // the previous block's last tile is no longer read
        commit();
        __syncthreads();
        for (int it = 0; it < n_steps; ++it) {
            const int q0 = q_begin + it * kTile;
            if (it + 1 < n_steps) fetch(q0 + kTile);
            if (!(a.causal && q0 + kTile - 1 < kw)) {
                const bool need_mask = a.causal && q0 < kw + 31;
                floatx16 sc[2], dp[2];
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    sc[qb] = dot_rows(Qs, qb, ln, hh, kf);  // S = Q K^T (raw)
                    dp[qb] = dot_rows(Gs, qb, ln, hh, vf);  // dP = dO V^T
                }
                floatx16 p[2], ds[2];
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int qi = 32 * qb + 8 * (i / 4) + 4 * hh + (i % 4);
                        float pv = __builtin_amdgcn_exp2f(sc[qb][i] * c - Ls[qi]);
                        if (need_mask && key > q0 + qi) pv = 0.0f;
                        p[qb][i] = pv;
                        ds[qb][i] = pv * (dp[qb][i] - Ds[qi]);
                    }
                acc_cols(dv, Gs, ln, hh, p);   // dV^T += dO^T P
                acc_cols(dk, Qs, ln, hh, ds);  // dK^T += Q^T dS
            }
            if (it + 1 < n_steps) {
                __syncthreads();
                commit();
                __syncthreads();
            }
        }
        if (key < T) {
            store_rows(dKg, key, a.ld_grad, hh, dk, a.scale);  // dS carries the reference's scale (:293)
            store_rows(dVg, key, a.ld_grad, hh, dv, 1.0f);
        }
    }
}

// ------------------------------------------------------------------------------------------------ dQ
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dq_f32_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(16))) float Ks[kTile * kLd];
    __shared__ __attribute__((aligned(16))) float Vs[kTile * kLd];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int nqb = (T + kBlk - 1) / kBlk;
    const int npair = (nqb + 1) / 2;
    const int pair = blockIdx.x % npair;
    const int bh = blockIdx.x / npair;
    const int b = bh / a.H, h = bh % a.H;

    const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Gg = static_cast<const float*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    float* dQg = static_cast<float*>(a.d_q) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    for (int half = 0; half < 2; ++half) {
        const int qb = half ? nqb - 1 - pair : pair;
        if (half && qb == pair) break;
        const int qw = qb * kBlk + 32 * wave;
        const int q = qw + ln;

        float qf[64], gf[64];
        load_half_row(qf, Qg, q, T, a.ld_qkv, hh);
        load_half_row(gf, Gg, q, T, a.ld_o, hh);
        const float lse2 = q < T ? a.lse2[(int64_t)bh * T + q] : 0.0f;
        const float delta = q < T ? a.delta[(int64_t)bh * T + q] : 0.0f;
        const int lim = a.causal ? min(q, T - 1) : T - 1;
        floatx16 dq[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) dq[db] = zero16();

        const int k_end = a.causal ? min(qb * kBlk + kBlk, T) : T;
        const int n_steps = (k_end + kTile - 1) / kTile;
        TileRegs rk, rv;
        tile_load(rk, Kg, 0, T, a.ld_qkv, tid);
        tile_load(rv, Vg, 0, T, a.ld_qkv, tid);
        __syncthreads();
        tile_store(Ks, rk, tid);
        tile_store(Vs, rv, tid);
        __syncthreads();
        for (int it = 0; it < n_steps; ++it) {
            const int k0 = it * kTile;
            if (it + 1 < n_steps) {
                tile_load(rk, Kg, k0 + kTile, T, a.ld_qkv, tid);
                tile_load(rv, Vg, k0 + kTile, T, a.ld_qkv, tid);
            }
            if (!(a.causal && k0 > qw + 31)) {
                const bool need_mask = (a.causal && k0 + kTile - 1 > qw) || k0 + kTile > T;
                floatx16 sc[2], dp[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    sc[kb] = dot_rows(Ks, kb, ln, hh, qf);  // S^T = K Q^T (raw)
                    dp[kb] = dot_rows(Vs, kb, ln, hh, gf);  // dP^T = V dO^T
                }
                floatx16 ds[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        float pv = __builtin_amdgcn_exp2f(sc[kb][i] * c - lse2);
                        if (need_mask && k0 + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4) > lim) pv = 0.0f;
                        ds[kb][i] = pv * (dp[kb][i] - delta);
                    }
                acc_cols(dq, Ks, ln, hh, ds);  // dQ^T += K^T dS^T
            }
            if (it + 1 < n_steps) {
                __syncthreads();
                tile_store(Ks, rk, tid);
                tile_store(Vs, rv, tid);
                __syncthreads();
            }
        }
        if (q < T) store_rows(dQg, q, a.ld_grad, hh, dq, a.scale);
    }
}

}  // namespace

int launch_flash_bwd_f32(const FlashBwdArgs& a, hipStream_t stream) {
    DT_TRY(launch_flash_bwd_prep(a, 0, stream));
    const int64_t npair = ((a.T + kBlk - 1) / kBlk + 1) / 2;
    const int64_t grid = npair * a.B * a.H;
    if (grid > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many workgroups");
    hipLaunchKernelGGL(flash_bwd_dkdv_f32_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, a);
    DT_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(flash_bwd_dq_f32_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, a);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
