// Causal flash attention forward, fp32 exact mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_forward (FlashAttention.cpp:24-182). The reference
// runs 256x256 tiles with two cblas_sgemm calls per tile and a scalar softmax;
// here one workgroup owns 128 queries of one (batch, head) and streams 64-key
// tiles of K and V through LDS.
//
// Work split: 4 waves x 32 queries. Each wave computes S^T = K Q^T for its 32
// queries with v_mfma_f32_32x32x2_f32, so that in the accumulator layout one
// lane holds one query (lane % 32) and 16 keys; the row max / row sum of the
// online softmax are then a per-lane reduction plus one exchange with lane ^ 32.
// The probabilities stay in the accumulator registers and feed the PV product
// O^T += V^T P^T directly as the B operand (the MFMA's k index is only a
// summation label, so V rows are read in the accumulator's key order).
//
// Numerics follow the reference: S = scale * Q K^T (FlashAttention.cpp:83-91),
// keys with k_pos > q_pos masked (:102), m = row max of the scaled scores,
// l = sum exp(s - m) (:159-163), output O / l, and a row with l == 0 written as
// zeros (:165-174). The online rescale uses the running max directly
// (FA-2 form) instead of the reference's tile-local max with alpha/beta
// factors (:134-156); both equal sum_k exp(s_k - m_final) up to rounding.
// exp is evaluated as exp2 with log2(e) folded into the scale.

#include "dt_internal.h"

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;   // head_dim (model_config.h:3)
constexpr int kBM = 128;  // queries per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kLdK = 132; // LDS row stride (floats): 16 rows at one column hit 16 distinct 4-bank groups
constexpr int kLdV = 132;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

__global__ __launch_bounds__(256, 2) void flash_fwd_f32_kernel(FlashArgs a, SeqLens lens) {
    __shared__ __attribute__((aligned(16))) float Ks[kBN * kLdK];
    __shared__ __attribute__((aligned(16))) float Vs[kBN * kLdV];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ln = lane & 31;  // query within the wave's 32 (MFMA n index)
    const int hh = lane >> 5;  // lane half (MFMA k index)
    const int qt = gridDim.x - 1 - blockIdx.x;  // longest (latest) query tiles first
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int T = a.T;
    const int L = a.ragged ? lens.len[b] : T;  // valid keys / rows of this sequence
    const int q0 = qt * kBM;
    const int qw0 = q0 + wave * 32;  // first query of this wave
    const int qrow = qw0 + ln;

    const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ldq + (int64_t)h * kD;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ldk + (int64_t)h * kD;
    const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ldv + (int64_t)h * kD;
    float* Og = static_cast<float*>(a.o) + (int64_t)b * T * a.ldo + (int64_t)h * kD;
    const int64_t stat_base = ((int64_t)b * T) * a.H + h;  // m/l index of row t: stat_base + t*H

    if (q0 >= L) {
        // Every row of this tile is padding: the reference's empty row (l == 0).
        if (qrow < T) {
            float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int j = 0; j < 16; ++j) *reinterpret_cast<float4*>(&Og[(int64_t)qrow * a.ldo + 64 * hh + 4 * j]) = z;
            if (hh == 0) {
                if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = kNegInf;
                if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = 0.0f;
            }
        }
        return;
    }

    // Q fragment in registers: q[4*j + e] = Q[qrow][8*j + 4*hh + e] (B operand of S^T = K Q^T).
    float q[64];
    if (qrow < T) {
        const float* qp = Qg + (int64_t)qrow * a.ldq + 4 * hh;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float4 v = *reinterpret_cast<const float4*>(qp + 8 * j);
            q[4 * j + 0] = v.x; q[4 * j + 1] = v.y; q[4 * j + 2] = v.z; q[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 64; ++j) q[j] = 0.0f;
    }

    // O^T accumulators: o[bb][i] holds O[q][d] with d = 4*m + bb, m = 8*(i/4) + 4*hh + (i%4).
    floatx16 o[4];
#pragma unroll
    for (int bb = 0; bb < 4; ++bb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[bb][i] = 0.0f;

    float m_run = kNegInf;  // running max of the raw (unscaled) scores
    float l_run = 0.0f;
    const float c = a.scale * kLog2e;

    const int k_end = a.causal ? min(q0 + kBM, L) : L;
    const int n_tiles = (k_end + kBN - 1) / kBN;

    for (int kt = 0; kt < n_tiles; ++kt) {
        const int k0 = kt * kBN;
        __syncthreads();  // previous tile fully consumed
        // cooperative load of the K and V tiles (rows beyond L are zero-filled)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = (tid >> 5) + 8 * i;
            const int key = k0 + r;
            const int col = 4 * (tid & 31);
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (key < L) {
                kv = *reinterpret_cast<const float4*>(&Kg[(int64_t)key * a.ldk + col]);
                vv = *reinterpret_cast<const float4*>(&Vg[(int64_t)key * a.ldv + col]);
            }
            *reinterpret_cast<float4*>(&Ks[r * kLdK + col]) = kv;
            *reinterpret_cast<float4*>(&Vs[r * kLdV + col]) = vv;
        }
        __syncthreads();

        if (a.causal && k0 > qw0 + 31) continue;  // every key of this tile is after every query of this wave

        // S^T for two 32-key blocks: st[kb][i] = S[qrow][key], key = k0 + 32*kb + 8*(i/4) + 4*hh + (i%4)
        floatx16 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) st[kb][i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const float4 kv = *reinterpret_cast<const float4*>(&Ks[(32 * kb + ln) * kLdK + 8 * j + 4 * hh]);
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, q[4 * j + 0], st[kb], 0, 0, 0);
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, q[4 * j + 1], st[kb], 0, 0, 0);
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, q[4 * j + 2], st[kb], 0, 0, 0);
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, q[4 * j + 3], st[kb], 0, 0, 0);
            }
        }

        // mask (diagonal / ragged tail only) and tile max
        const bool need_mask = (a.causal && k0 + kBN - 1 > qw0) || (k0 + kBN > L);
        float tmax = kNegInf;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (need_mask) {
                    const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                    if ((a.causal && key > qrow) || key >= L) st[kb][i] = kNegInf;
                }
                tmax = fmaxf(tmax, st[kb][i]);
            }
        tmax = fmaxf(tmax, xor32(tmax));
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = (m_new == kNegInf) ? 0.0f : m_new;
        const float mc = m_use * c;
        const float alpha = exp2f((m_run - m_use) * c);  // 0 when m_run == -inf
        float psum = 0.0f;
        {
            // s*c and m*c rounded separately (no fma contraction), so the row's maximum
            // contributes exactly exp2(0) = 1, as exp(s - m) does in the reference.
#pragma clang fp contract(off)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = __builtin_amdgcn_exp2f(st[kb][i] * c - mc);
                    st[kb][i] = p;
                    psum += p;
                }
        }
        psum += xor32(psum);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[bb][i] *= alpha;

        // O^T += V^T P^T: MFMA step (kb, s) takes key k0 + 32*kb + 8*(s/4) + 4*hh + (s%4) from lane half hh.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int key = 32 * kb + 8 * (s / 4) + 4 * hh + (s % 4);
                const float4 vv = *reinterpret_cast<const float4*>(&Vs[key * kLdV + 4 * ln]);
                const float p = st[kb][s];
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, p, o[0], 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, p, o[1], 0, 0, 0);
                o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, p, o[2], 0, 0, 0);
                o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, p, o[3], 0, 0, 0);
            }
    }

    // finalize (FlashAttention.cpp:159-175)
    if (qrow < T) {
        const bool valid = qrow < L && l_run > 0.0f;
        float* op = Og + (int64_t)qrow * a.ldo;
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float4 v;
                if (valid) {
                    v.x = o[0][4 * I + r] / l_run; v.y = o[1][4 * I + r] / l_run;
                    v.z = o[2][4 * I + r] / l_run; v.w = o[3][4 * I + r] / l_run;
                } else {
                    v = make_float4(0.f, 0.f, 0.f, 0.f);
                }
                *reinterpret_cast<float4*>(&op[32 * I + 16 * hh + 4 * r]) = v;
            }
        if (hh == 0) {
            if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? m_run * a.scale : kNegInf;
            if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l_run : 0.0f;
        }
    }
}

}  // namespace

int launch_flash_fwd_f32(const FlashArgs& a, const SeqLens* lens, hipStream_t stream) {
    SeqLens sl;
    if (a.ragged) sl = *lens;
    else sl.len[0] = a.T;
    dim3 grid((a.T + kBM - 1) / kBM, a.H, a.B);
    hipLaunchKernelGGL(flash_fwd_f32_kernel, grid, dim3(256), 0, stream, a, sl);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
