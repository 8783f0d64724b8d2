// Causal flash attention forward, bf16 MFMA mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_forward (FlashAttention.cpp:24-182) with bf16
// Q/K/V/O, fp32 accumulation and an fp32 online softmax.
//
// Work split: one workgroup = 4 waves x 32 queries of one (batch, head); K and
// V stream through LDS in 64-key tiles, prefetched into registers one tile
// ahead. Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS, B = the wave's Q fragment held in registers), so in
// the accumulator one lane owns one query and 16 keys; row max and row sum are
// a per-lane reduction plus one exchange with lane ^ 32. P is converted to
// bf16 in place and used as the B operand of O^T += V^T P^T. The A operand
// (V^T) comes from the gfx950 transposing LDS read ds_read_b64_tr_b16: a
// 16-lane group reads a 4-key x 16-dim block and each lane receives one dim
// column of 4 keys, which is exactly the MFMA's 8-key k slice taken as two
// 4-key runs in the accumulator's key order.
//
// Semantics as in the fp32 kernel: scaled scores, causal predicate k > q
// masked (FlashAttention.cpp:102), m = max of the scaled scores, l = sum
// exp(s - m), rows with l == 0 written as zeros (FlashAttention.cpp:165-174).

#include "dt_internal.h"

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

constexpr int kD = 128;
constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kLdK = 136;  // bf16 elements per K row in LDS (272 B)
constexpr int kLdV = 160;  // bf16 elements per V row in LDS (320 B)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ shortx4 lds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(p));
}

__global__ __launch_bounds__(256, 2) void flash_fwd_bf16_kernel(FlashArgs a, SeqLens lens) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * kLdK];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[kBN * kLdV];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int qt = gridDim.x - 1 - blockIdx.x;  // longest query tiles first
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int T = a.T;
    const int L = a.ragged ? lens.len[b] : T;
    const int q0 = qt * kBM;
    const int qw0 = q0 + wave * 32;
    const int qrow = qw0 + ln;

    const uint16_t* Qg = static_cast<const uint16_t*>(a.q) + (int64_t)b * T * a.ldq + (int64_t)h * kD;
    const uint16_t* Kg = static_cast<const uint16_t*>(a.k) + (int64_t)b * T * a.ldk + (int64_t)h * kD;
    const uint16_t* Vg = static_cast<const uint16_t*>(a.v) + (int64_t)b * T * a.ldv + (int64_t)h * kD;
    uint16_t* Og = static_cast<uint16_t*>(a.o) + (int64_t)b * T * a.ldo + (int64_t)h * kD;
    const int64_t stat_base = ((int64_t)b * T) * a.H + h;

    if (q0 >= L) {
        if (qrow < T) {
            const uint4 z = make_uint4(0, 0, 0, 0);
            for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4*>(&Og[(int64_t)qrow * a.ldo + 64 * hh + 8 * j]) = z;
            if (hh == 0) {
                if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = kNegInf;
                if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = 0.0f;
            }
        }
        return;
    }

    // Q fragment: qf[c] = Q[qrow][16*c + 8*hh .. +8] (B operand of S^T = K Q^T).
    bf16x8 qf[8];
    if (qrow < T) {
        const uint16_t* qp = Qg + (int64_t)qrow * a.ldq + 8 * hh;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) qf[cc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + 16 * cc));
    } else {
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) qf[cc] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
    }

    // O^T accumulators: o[db][i] = O[qrow][32*db + 8*(i/4) + 4*hh + (i%4)]
    floatx16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;

    float m_run = kNegInf;
    float l_run = 0.0f;
    const float c = a.scale * kLog2e;

    const int k_end = a.causal ? min(q0 + kBM, L) : L;
    const int n_tiles = (k_end + kBN - 1) / kBN;

    // cooperative tile load: thread covers rows (tid/16) + 16*i, 16-byte chunk tid%16
    const int ld_row = tid >> 4;
    const int ld_col = 8 * (tid & 15);
    uint4 pk_k[4], pk_v[4];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = k0 + ld_row + 16 * i;
            if (key < L) {
                pk_k[i] = *reinterpret_cast<const uint4*>(&Kg[(int64_t)key * a.ldk + ld_col]);
                pk_v[i] = *reinterpret_cast<const uint4*>(&Vg[(int64_t)key * a.ldv + ld_col]);
            } else {
                pk_k[i] = make_uint4(0, 0, 0, 0);
                pk_v[i] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    fetch(0);

    // tr-read lane addressing: lane i of a 16-lane group points at row i/4, dims 4*(i%4) of a 4x16 block
    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 4 * (lane & 3) + 16 * ((lane >> 4) & 1);

    for (int kt = 0; kt < n_tiles; ++kt) {
        const int k0 = kt * kBN;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<uint4*>(&Ks[(ld_row + 16 * i) * kLdK + ld_col]) = pk_k[i];
            *reinterpret_cast<uint4*>(&Vs[(ld_row + 16 * i) * kLdV + ld_col]) = pk_v[i];
        }
        __syncthreads();
        if (kt + 1 < n_tiles) fetch(k0 + kBN);

        if (a.causal && k0 > qw0 + 31) continue;

        floatx16 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) st[kb][i] = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8 kf = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(&Ks[(32 * kb + ln) * kLdK + 16 * cc + 8 * hh]));
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[cc], st[kb], 0, 0, 0);
            }
        }

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
        const float alpha = exp2f((m_run - m_use) * c);
        float psum = 0.0f;
        // P in bf16: pb[kb][u] holds accumulator entries 8*u .. 8*u+7 of block kb
        bf16x8 pb[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][8 * u + 2 * e], c, -mc));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][8 * u + 2 * e + 1], c, -mc));
                    psum += p0 + p1;
                    w[e] = pack_bf16x2(p0, p1);
                }
                pb[kb][u] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
            }
        psum += xor32(psum);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;

        // O^T += V^T P^T. Chunk (kb, u): k index 8*hh + e <-> key 32*kb + 16*u + 8*(e/4) + 4*hh + (e%4).
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int kr = 32 * kb + 16 * u + 4 * hh + tr_row;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const uint16_t* base = &Vs[kr * kLdV + 32 * db + tr_col];
                    const shortx4 lo = lds_read_tr16(base);
                    const shortx4 hi = lds_read_tr16(base + 8 * kLdV);
                    const bf16x8 vf = __builtin_bit_cast(
                        bf16x8, (short __attribute__((ext_vector_type(8)))){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[kb][u], o[db], 0, 0, 0);
                }
            }
    }

    if (qrow < T) {
        const bool valid = qrow < L && l_run > 0.0f;
        const float inv = valid ? 1.0f / l_run : 0.0f;
        uint16_t* op = Og + (int64_t)qrow * a.ldo;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int I = 0; I < 4; ++I) {
                uint2 w;
                w.x = pack_bf16x2(o[db][4 * I + 0] * inv, o[db][4 * I + 1] * inv);
                w.y = pack_bf16x2(o[db][4 * I + 2] * inv, o[db][4 * I + 3] * inv);
                *reinterpret_cast<uint2*>(&op[32 * db + 8 * I + 4 * hh]) = w;
            }
        if (hh == 0) {
            if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? m_run * a.scale : kNegInf;
            if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l_run : 0.0f;
        }
    }
}

}  // namespace

int launch_flash_fwd_bf16(const FlashArgs& a, const SeqLens* lens, hipStream_t stream) {
    SeqLens sl;
    if (a.ragged) sl = *lens;
    else sl.len[0] = a.T;
    dim3 grid((a.T + kBM - 1) / kBM, a.H, a.B);
    hipLaunchKernelGGL(flash_fwd_bf16_kernel, grid, dim3(256), 0, stream, a, sl);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
